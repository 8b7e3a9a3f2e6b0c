"""Pins of the NumPy oracle (CPU).

The oracle is checked against (1) golden vectors written by the reference's
own PyTorch path (``tests/golden/make_golden.py``), (2) closed forms and
special cases the mathematics fixes, and (3) textbook routines
(``scipy.special.softmax``).  Each check is chosen so a plausible slip -- a
dropped beta, a transposed bank, a wrong mask side, a missing RMS factor --
fails at least one of them.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
from scipy.special import softmax as scipy_softmax

import oracle
from conftest import Golden, golden_names

RNG = np.random.default_rng(1234)


def _unit_columns(r: int, m: int, rng=RNG) -> np.ndarray:
    d = rng.standard_normal((r, m))
    return d / np.linalg.norm(d, axis=0, keepdims=True)


# ---------------------------------------------------------------- golden vectors


# The reference promotes the outer-attention scores to fp32 and runs that
# softmax in fp32 even for a float64 module (ops.py:86,91), so its float64
# outputs carry fp32 rounding (measured: <= 2.6e-7 of the output scale).  The
# oracle stays float64 throughout; outputs are compared at 1e-6 of their
# scale, which any formula slip (a lost beta, a wrong mask side, a missing
# RMS factor) exceeds by orders of magnitude.  The routed Q/K never pass
# through that fp32 step and are compared at 1e-10.
GOLDEN_SCALED_TOL = 1e-6


def assert_scaled_close(actual: np.ndarray, expected: np.ndarray, tol: float) -> None:
    err = np.abs(actual - expected).max() / np.abs(expected).max()
    assert err <= tol, f"max error {err:.3e} of the output scale exceeds {tol:.1e}"


@pytest.mark.parametrize("name", golden_names("attention"))
def test_oracle_matches_reference_attention_goldens(name: str) -> None:
    g = Golden(name)
    params = {k: v.astype(np.float64) for k, v in g.params.items()}
    out, rq, rk = oracle.shared_dictionary_attention(params, g.config, g["x"], return_routed=True)
    assert out.shape == g["out"].shape
    assert_scaled_close(out, g["out"], GOLDEN_SCALED_TOL)
    np.testing.assert_allclose(rq, g["routing_query"], rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(rk, g["routing_key"], rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("name", golden_names("lm"))
def test_oracle_matches_reference_lm_goldens(name: str) -> None:
    g = Golden(name)
    params = {k: v.astype(np.float64) for k, v in g.params.items()}
    logits = oracle.double_attention_lm(params, g.config, g["ids"], int(g["layers"]), int(g["group"]))
    assert logits.shape == g["logits"].shape
    assert_scaled_close(logits, g["logits"], GOLDEN_SCALED_TOL)


def test_golden_check_detects_planted_mistakes() -> None:
    # A slip planted in the oracle's inputs must break the golden comparison.
    g = Golden("qk2_s2_small")
    params = {k: v.astype(np.float64) for k, v in g.params.items()}
    wrong_beta = dict(params, log_beta=params["log_beta"] + 0.1)
    out = oracle.shared_dictionary_attention(wrong_beta, g.config, g["x"])
    assert np.abs(out - g["out"]).max() / np.abs(g["out"]).max() > 100 * GOLDEN_SCALED_TOL
    wrong_mix = dict(params, map_mix_logits=params["map_mix_logits"] + np.array([0.0, 0.2]))
    out = oracle.shared_dictionary_attention(wrong_mix, g.config, g["x"])
    assert np.abs(out - g["out"]).max() / np.abs(g["out"]).max() > 100 * GOLDEN_SCALED_TOL
    noncausal = dict(g.config, causal=False)
    out = oracle.shared_dictionary_attention(params, noncausal, g["x"])
    assert np.abs(out - g["out"]).max() / np.abs(g["out"]).max() > 100 * GOLDEN_SCALED_TOL
    # A dropped term (the value bias), a sign (of the value bias) and a
    # transposed operand (query and key projections swapped, which transposes
    # every score matrix before the causal mask).
    dropped = dict(params, **{"value.bias": np.zeros_like(params["value.bias"])})
    flipped = dict(params, **{"value.bias": -params["value.bias"]})
    swapped = dict(params, **{"query.weight": params["key.weight"], "key.weight": params["query.weight"]})
    for wrong in (dropped, flipped, swapped):
        out = oracle.shared_dictionary_attention(wrong, g.config, g["x"])
        assert np.abs(out - g["out"]).max() / np.abs(g["out"]).max() > 100 * GOLDEN_SCALED_TOL


# ---------------------------------------------------------------- normalization


def test_l2_normalize_eps_semantics() -> None:
    x = np.array([[3.0, 4.0], [0.0, 0.0], [3e-8, 4e-8]])
    y = oracle.l2_normalize(x, -1, 1e-6)
    np.testing.assert_allclose(y[0], [0.6, 0.8])
    np.testing.assert_array_equal(y[1], [0.0, 0.0])          # 0 / eps
    np.testing.assert_allclose(y[2], [3e-8 / 1e-6, 4e-8 / 1e-6])  # below eps: divided by eps, not unit


def test_bank_normalized_columns_are_unit_and_tied_is_shared() -> None:
    raw = RNG.standard_normal((8, 16)) * 3.0
    key, value = oracle.bank_normalized(raw, None)
    assert key is value
    np.testing.assert_allclose(np.linalg.norm(key, axis=0), 1.0, rtol=1e-12)
    # Direction is preserved column by column.
    np.testing.assert_allclose(key * np.linalg.norm(raw, axis=0), raw, rtol=1e-12)


# ---------------------------------------------------------------- dictionary route


def test_route_zero_input_gives_normalized_mean_atom() -> None:
    dk, dv = _unit_columns(8, 12), _unit_columns(8, 12)
    z = oracle.dictionary_route(np.zeros((3, 8)), dk, dv, 4.0)
    mean_atom = dv.mean(axis=1)
    np.testing.assert_allclose(z, np.broadcast_to(mean_atom / np.linalg.norm(mean_atom), z.shape), rtol=1e-12)


def test_route_large_beta_selects_argmax_atom() -> None:
    dk, dv = _unit_columns(16, 24), _unit_columns(16, 24)
    x = RNG.standard_normal((5, 16))
    z = oracle.dictionary_route(x, dk, dv, 1e5)
    best = np.argmax((x / np.linalg.norm(x, axis=1, keepdims=True)) @ dk, axis=1)
    np.testing.assert_allclose(z, dv[:, best].T, atol=1e-9)


def test_route_single_atom_bank() -> None:
    dk = RNG.standard_normal((8, 1))
    dv = RNG.standard_normal((8, 1))
    z = oracle.dictionary_route(RNG.standard_normal((4, 8)), dk, dv, 4.0)
    np.testing.assert_allclose(z, np.broadcast_to((dv[:, 0] / np.linalg.norm(dv[:, 0])), z.shape), rtol=1e-12)


def test_route_input_scale_and_atom_permutation_invariance() -> None:
    dk, dv = _unit_columns(8, 20), _unit_columns(8, 20)
    x = RNG.standard_normal((6, 8))
    z = oracle.dictionary_route(x, dk, dv, 4.0)
    np.testing.assert_allclose(oracle.dictionary_route(7.5 * x, dk, dv, 4.0), z, rtol=1e-12)
    perm = RNG.permutation(20)
    np.testing.assert_allclose(oracle.dictionary_route(x, dk[:, perm], dv[:, perm], 4.0), z, rtol=1e-12)


def test_route_identity_bank_reduces_to_textbook_softmax() -> None:
    # With Dk = Dv = I (R = M) and no output norm the route is softmax(beta * u).
    x = RNG.standard_normal((5, 9))
    eye = np.eye(9)
    z = oracle.dictionary_route(x, eye, eye, 3.0, normalize_output=False)
    u = x / np.linalg.norm(x, axis=1, keepdims=True)
    np.testing.assert_allclose(z, scipy_softmax(3.0 * u, axis=1), rtol=1e-12)


def test_route_distinguishes_key_and_value_banks() -> None:
    # Swapping the roles of the two banks must change the result.
    dk, dv = _unit_columns(8, 10), _unit_columns(8, 10)
    x = RNG.standard_normal((3, 8))
    assert not np.allclose(oracle.dictionary_route(x, dk, dv, 4.0), oracle.dictionary_route(x, dv, dk, 4.0))


def test_route_brute_force_loop() -> None:
    r, m = 5, 7
    dk, dv = _unit_columns(r, m), _unit_columns(r, m)
    x = RNG.standard_normal((3, r))
    beta = 2.5
    z = oracle.dictionary_route(x, dk, dv, beta)
    for i in range(3):
        norm = math.sqrt(sum(v * v for v in x[i]))
        logits = [sum(x[i, a] / norm * dk[a, j] for a in range(r)) for j in range(m)]
        top = max(logits)
        e = [math.exp(beta * (l - top)) for l in logits]
        w = [v / sum(e) for v in e]
        rec = [sum(w[j] * dv[a, j] for j in range(m)) for a in range(r)]
        n = math.sqrt(sum(v * v for v in rec))
        np.testing.assert_allclose(z[i], [v / n for v in rec], rtol=1e-12)


@pytest.mark.parametrize("tied", [False, True])
def test_bank_normalized_backward_matches_finite_differences(tied: bool) -> None:
    # Gradients at the raw bank through the column normalization, against
    # central differences of bank_normalized in fp64; one column is scaled
    # below eps (the h / eps branch) and one is large.
    rng = np.random.default_rng(21)
    r, m, eps = 5, 6, 1e-3
    raw_key = rng.standard_normal((r, m))
    raw_key[:, 2] *= 1e-5
    raw_key[:, 4] *= 30.0
    raw_value = None if tied else rng.standard_normal((r, m))
    wk, wv = rng.standard_normal((r, m)), rng.standard_normal((r, m))
    d_key, d_value = oracle.bank_normalized_backward(raw_key, raw_value, wk, wv, eps)
    assert (d_value is None) == tied

    def loss(k_, v_):
        key, value = oracle.bank_normalized(k_, v_, eps)
        return float((key * wk).sum() + (value * wv).sum())

    h = 1e-7
    for which, arr, grad in ((0, raw_key, d_key), (1, raw_value, d_value)):
        if arr is None:
            continue
        numeric = np.zeros_like(arr)
        for pos in np.ndindex(arr.shape):
            plus, minus = arr.copy(), arr.copy()
            plus[pos] += h
            minus[pos] -= h
            args_p, args_m = [raw_key, raw_value], [raw_key, raw_value]
            args_p[which], args_m[which] = plus, minus
            numeric[pos] = (loss(*args_p) - loss(*args_m)) / (2 * h)
        np.testing.assert_allclose(grad, numeric, rtol=1e-5, atol=1e-6)
    # The small column is in the h / eps branch: its gradient is the plain
    # scaled one, no projection.
    total = wk + wv if tied else wk
    np.testing.assert_allclose(d_key[:, 2], total[:, 2] / eps, rtol=1e-12)


@pytest.mark.parametrize(("normalize_input", "normalize_output"), [(True, True), (False, True), (True, False)])
def test_route_backward_matches_finite_differences(normalize_input: bool, normalize_output: bool) -> None:
    rng = np.random.default_rng(11)
    r, m = 4, 6
    x = rng.standard_normal((2, 3, r))
    dk, dv = _unit_columns(r, m, rng), _unit_columns(r, m, rng)
    beta = 2.3
    w = rng.standard_normal((2, 3, r))
    dx, ddk, ddv, dbeta = oracle.dictionary_route_backward(x, dk, dv, beta, w, 1e-6, normalize_input, normalize_output)

    def loss(x_, dk_, dv_, b_):
        out = oracle.dictionary_route(x_, dk_, dv_, b_, 1e-6, normalize_input=normalize_input,
                                      normalize_output=normalize_output)
        return float((out * w).sum())

    h = 1e-6
    for idx, arr, grad in ((0, x, dx), (1, dk, ddk), (2, dv, ddv)):
        numeric = np.zeros_like(arr)
        for pos in np.ndindex(arr.shape):
            plus, minus = arr.copy(), arr.copy()
            plus[pos] += h
            minus[pos] -= h
            args_p, args_m = [x, dk, dv, beta], [x, dk, dv, beta]
            args_p[idx], args_m[idx] = plus, minus
            numeric[pos] = (loss(*args_p) - loss(*args_m)) / (2 * h)
        np.testing.assert_allclose(grad, numeric, rtol=1e-6, atol=1e-8)
    numeric_beta = (loss(x, dk, dv, beta + h) - loss(x, dk, dv, beta - h)) / (2 * h)
    np.testing.assert_allclose(dbeta, numeric_beta, rtol=1e-6, atol=1e-8)


ROUTE_VARIANTS = [
    dict(activation="silu"),
    dict(standardize_logits=True),
    dict(standardize_logits=True, standardized_logit_scale=1.7),
    dict(assignment="silu", silu_gain=1.0),
    dict(assignment="silu", silu_gain=3.0),
    dict(activation="silu", standardize_logits=True),
    dict(activation="silu", standardize_logits=True, assignment="silu", silu_gain=2.0),
]


@pytest.mark.parametrize("variant", ROUTE_VARIANTS, ids=lambda v: "-".join(f"{k}={v[k]}" for k in v))
@pytest.mark.parametrize(("normalize_input", "normalize_output"), [(True, True), (False, False)])
def test_route_variant_backward_matches_finite_differences(variant, normalize_input, normalize_output) -> None:
    # The SiLU activation, standardized logits and the SiLU assignment
    # (ops.py:41-59): every gradient of the oracle's chain rule against
    # central differences of the oracle forward, in fp64.
    rng = np.random.default_rng(12)
    r, m = 4, 7
    x = rng.standard_normal((2, 3, r))
    dk, dv = _unit_columns(r, m, rng), _unit_columns(r, m, rng)
    beta = 1.9
    w = rng.standard_normal((2, 3, r))
    dx, ddk, ddv, dbeta = oracle.dictionary_route_backward(
        x, dk, dv, beta, w, 1e-6, normalize_input, normalize_output, **variant
    )

    def loss(x_, dk_, dv_, b_):
        out = oracle.dictionary_route(x_, dk_, dv_, b_, 1e-6, normalize_input=normalize_input,
                                      normalize_output=normalize_output, **variant)
        return float((out * w).sum())

    h = 1e-6
    for idx, arr, grad in ((0, x, dx), (1, dk, ddk), (2, dv, ddv)):
        numeric = np.zeros_like(arr)
        for pos in np.ndindex(arr.shape):
            plus, minus = arr.copy(), arr.copy()
            plus[pos] += h
            minus[pos] -= h
            args_p, args_m = [x, dk, dv, beta], [x, dk, dv, beta]
            args_p[idx], args_m[idx] = plus, minus
            numeric[pos] = (loss(*args_p) - loss(*args_m)) / (2 * h)
        np.testing.assert_allclose(grad, numeric, rtol=1e-5, atol=1e-8)
    numeric_beta = (loss(x, dk, dv, beta + h) - loss(x, dk, dv, beta - h)) / (2 * h)
    np.testing.assert_allclose(dbeta, numeric_beta, rtol=1e-5, atol=1e-8)
    if variant.get("assignment") == "silu":
        assert dbeta == 0.0


# ---------------------------------------------------------------- outer attention


def _qkv(b=2, s=3, t=6, r=4, d=5, rng=RNG):
    q = rng.standard_normal((b, s, t, r))
    k = rng.standard_normal((b, s, t, r))
    v = rng.standard_normal((b, t, d))
    return q, k, v


def test_attention_first_causal_row_is_first_value() -> None:
    q, k, v = _qkv()
    out = oracle.routed_attention(q, k, v, np.array([3.0, 5.0, 7.0]), causal=True)
    for s in range(3):
        np.testing.assert_allclose(out[:, s, 0], v[:, 0], rtol=1e-12)


def test_attention_equal_keys_gives_causal_running_mean() -> None:
    q, _, v = _qkv()
    k = np.broadcast_to(RNG.standard_normal(4), (2, 3, 6, 4)).copy()
    out = oracle.routed_attention(q, k, v, np.array([1.0, 9.0, 30.0]), causal=True)
    running = np.cumsum(v, axis=1) / np.arange(1, 7)[None, :, None]
    for s in range(3):
        np.testing.assert_allclose(out[:, s], running, rtol=1e-12)
    full = oracle.routed_attention(q, k, v, np.array([1.0, 9.0, 30.0]), causal=False)
    np.testing.assert_allclose(full[:, 0], np.broadcast_to(v.mean(axis=1, keepdims=True), (2, 6, 5)), rtol=1e-12)


def test_attention_rows_are_probability_weighted() -> None:
    q, k, _ = _qkv()
    ones = np.ones((2, 6, 5))
    out = oracle.routed_attention(q, k, ones, np.array([2.0, 4.0, 8.0]), causal=True)
    np.testing.assert_allclose(out, 1.0, rtol=1e-12)


def test_attention_causal_prefix_invariance_and_mask_side() -> None:
    q, k, v = _qkv()
    scales = np.array([2.0, 4.0, 8.0])
    base = oracle.routed_attention(q, k, v, scales, causal=True)
    k2, v2 = k.copy(), v.copy()
    k2[:, :, 4:] = RNG.standard_normal(k2[:, :, 4:].shape) * 10
    v2[:, 4:] = RNG.standard_normal(v2[:, 4:].shape) * 10
    changed = oracle.routed_attention(q, k2, v2, scales, causal=True)
    np.testing.assert_allclose(changed[:, :, :4], base[:, :, :4], rtol=1e-12)
    assert not np.allclose(changed[:, :, 4:], base[:, :, 4:])


def test_attention_matches_textbook_softmax_per_row() -> None:
    q, k, v = _qkv(b=1, s=2, t=5, r=3, d=4)
    scales = np.array([1.5, 6.0])
    out = oracle.routed_attention(q, k, v, scales, causal=True)
    for s in range(2):
        for t in range(5):
            w = scipy_softmax(scales[s] * (k[0, s, : t + 1] @ q[0, s, t]))
            np.testing.assert_allclose(out[0, s, t], w @ v[0, : t + 1], rtol=1e-12)


@pytest.mark.parametrize("causal", [True, False])
def test_attention_backward_matches_finite_differences(causal: bool) -> None:
    # Loss = sum(W * out) for a fixed random W, so d loss / d out = W; central
    # differences in fp64 of every input element pin each gradient, including
    # the scale gradient and the map sum of dV.
    rng = np.random.default_rng(7)
    q, k, v = _qkv(b=2, s=2, t=5, r=3, d=4, rng=rng)
    scales = np.array([1.7, 0.6])
    w = rng.standard_normal((2, 2, 5, 4))
    dq, dk, dv, ds = oracle.routed_attention_backward(q, k, v, scales, w, causal)

    def loss(q_, k_, v_, s_):
        return float((oracle.routed_attention(q_, k_, v_, s_, causal) * w).sum())

    h = 1e-6
    for arr, grad, idx in ((q, dq, 0), (k, dk, 1), (v, dv, 2), (scales, ds, 3)):
        numeric = np.zeros_like(arr)
        for pos in np.ndindex(arr.shape):
            args = [q, k, v, scales]
            plus, minus = arr.copy(), arr.copy()
            plus[pos] += h
            minus[pos] -= h
            args[idx] = plus
            up = loss(*args)
            args[idx] = minus
            numeric[pos] = (up - loss(*args)) / (2 * h)
        np.testing.assert_allclose(grad, numeric, rtol=1e-6, atol=1e-8)


def test_attention_backward_zero_gradient_and_value_map_sum() -> None:
    q, k, v = _qkv(b=1, s=3, t=6, r=4, d=5)
    scales = np.array([1.0, 2.0, 3.0])
    zero = oracle.routed_attention_backward(q, k, v, scales, np.zeros((1, 3, 6, 5)), True)
    for g in zero:
        assert not np.any(g)
    w = RNG.standard_normal((1, 3, 6, 5))
    _, _, dv, _ = oracle.routed_attention_backward(q, k, v, scales, w, True)
    per_map = [oracle.routed_attention_backward(q[:, s:s + 1], k[:, s:s + 1], v, scales[s:s + 1], w[:, s:s + 1], True)[2]
               for s in range(3)]
    np.testing.assert_allclose(dv, sum(per_map), rtol=1e-12)


# ---------------------------------------------------------------- score maps


def test_assemble_rms_sum_identity() -> None:
    q = RNG.standard_normal((2, 4, 5, 3))
    k = RNG.standard_normal((2, 4, 5, 3))
    sq, sk = oracle.assemble_score_maps(q, k, 2)
    assert sq.shape == (2, 2, 5, 6)
    for s in range(2):
        expected = sum(q[:, 2 * s + g] @ np.swapaxes(k[:, 2 * s + g], -1, -2) for g in range(2)) / math.sqrt(2)
        np.testing.assert_allclose(sq[:, s] @ np.swapaxes(sk[:, s], -1, -2), expected, rtol=1e-12)


def test_assemble_repeat_layout() -> None:
    q = RNG.standard_normal((1, 2, 3, 4))
    sq, sk = oracle.assemble_score_maps(q, q + 1, 4)
    for s in range(4):
        np.testing.assert_array_equal(sq[:, s], q[:, s // 2])
        np.testing.assert_array_equal(sk[:, s], q[:, s // 2] + 1)


def _module_case(rng, branches=1, maps=1, tied=False, bias=True, output=True, combine="weighted_sum", **route):
    """A tiny module (model width 8, routing width 4, 6 atoms) as a state dict
    and its config, with every parameter drawn away from the clamps' edges."""

    d, r, m = 8, 4, 6
    cfg = dict(qk_branches=branches, routing_dim=r, outer_maps=maps, eps=1e-6, causal=route.pop("causal", True),
               dictionary_activation="identity", dictionary_assignment="softmax", dictionary_silu_gain=1.0,
               standardize_dictionary_logits=False, standardized_logit_scale=None, normalize_routing_input=True,
               normalize_routing_output=True, map_combine=combine)
    cfg.update(route)
    params = {
        "query.weight": rng.standard_normal((branches * r, d)) * 0.5,
        "key.weight": rng.standard_normal((branches * r, d)) * 0.5,
        "value.weight": rng.standard_normal((d, d)) * 0.5,
        "bank.raw_key": rng.standard_normal((r, m)),
        "log_score_scales": np.log(np.array([2.0, 3.5, 1.2, 2.7][:maps])),
        "log_beta": np.array(math.log(3.0)),
    }
    if bias:
        params["value.bias"] = rng.standard_normal(d) * 0.1
    if not tied:
        params["bank.raw_value"] = rng.standard_normal((r, m))
    if combine == "weighted_sum" and maps > 1:
        params["map_mix_logits"] = rng.standard_normal(maps) * 0.5
    if output:
        params["output.weight"] = rng.standard_normal((d, d * (maps if combine == "concat" else 1))) * 0.5
    return params, cfg


MODULE_BACKWARD_LAYOUTS = [
    dict(),
    dict(tied=True),
    dict(branches=2, maps=2),
    dict(branches=2, maps=1),
    dict(branches=1, maps=2),
    dict(branches=2, maps=2, combine="concat"),
    dict(bias=False, output=False),
    dict(causal=False),
    dict(dictionary_activation="silu", standardize_dictionary_logits=True, normalize_routing_input=False),
    dict(dictionary_assignment="silu", dictionary_silu_gain=2.0, standardized_logit_scale=0.7,
         standardize_dictionary_logits=True),
]


@pytest.mark.parametrize("layout", MODULE_BACKWARD_LAYOUTS, ids=lambda c: "-".join(f"{k}={v}" for k, v in c.items()) or "a1")
def test_module_backward_matches_finite_differences(layout) -> None:
    # Loss = sum(W * out); central differences in fp64 of every element of x
    # and of every parameter (log beta included) pin the composed module
    # backward: the map combine, the score-map layouts, the clamps, the route
    # variants, the bank normalization and the projections.
    rng = np.random.default_rng(11)
    params, cfg = _module_case(rng, **dict(layout))
    x = rng.standard_normal((2, 5, 8))
    w = rng.standard_normal((2, 5, 8))
    grads = oracle.shared_dictionary_attention_backward(params, cfg, x, w)

    def loss(ps, x_):
        return float((oracle.shared_dictionary_attention(ps, cfg, x_) * w).sum())

    h = 1e-6
    targets = [("x", x)] + [(name, v) for name, v in params.items()]
    for name, arr in targets:
        numeric = np.zeros(np.shape(arr))
        for pos in np.ndindex(numeric.shape):
            def shifted(delta):
                a = np.array(arr, dtype=np.float64, copy=True)
                a[pos] += delta
                if name == "x":
                    return loss(params, a)
                return loss({**params, name: a}, x)
            numeric[pos] = (shifted(h) - shifted(-h)) / (2 * h)
        scale = max(float(np.abs(numeric).max()), 1e-12)
        np.testing.assert_allclose(grads[name], numeric, rtol=1e-5, atol=1e-6 * scale, err_msg=name)


def test_temperature_clamps() -> None:
    np.testing.assert_allclose(oracle.score_scale_from_log(np.array([-10.0, math.log(16.0), 20.0])), [0.25, 16.0, 1024.0])
    np.testing.assert_allclose(oracle.beta_from_log(np.array([-10.0, math.log(4.0), 20.0])), [0.05, 4.0, 64.0])
