"""NumPy restatement of the reference forward math (test infrastructure only).

Every function cites the reference lines it restates (paths relative to the
reference repository).  Arithmetic runs in the dtype of the inputs: float64
for the tight CPU checks, float32 for the parity tests and the CPU baseline.
Parameters are passed as a ``{state_dict name: ndarray}`` mapping so the
oracle consumes exactly the tensors the module under test holds.
"""

from __future__ import annotations

import math
from collections.abc import Mapping
from typing import Any

import numpy as np
from scipy.special import erf

LOG_BETA_MIN, LOG_BETA_MAX = math.log(0.05), math.log(64.0)     # modules.py:130-132
LOG_SCALE_MIN, LOG_SCALE_MAX = math.log(0.25), math.log(1024.0)  # ops.py:160-161


def _cfg(cfg: Any, name: str) -> Any:
    return cfg[name] if isinstance(cfg, Mapping) else getattr(cfg, name)


def l2_normalize(x: np.ndarray, axis: int, eps: float) -> np.ndarray:
    """``x / max(||x||_2, eps)`` along ``axis`` -- the semantics of ``F.normalize``."""

    norm = np.sqrt(np.sum(x * x, axis=axis, keepdims=True))
    return x / np.maximum(norm, eps)


def _softmax(x: np.ndarray, axis: int) -> np.ndarray:
    shifted = x - np.max(x, axis=axis, keepdims=True)
    e = np.exp(shifted)
    return e / np.sum(e, axis=axis, keepdims=True)


def _silu(x: np.ndarray) -> np.ndarray:
    return x / (1.0 + np.exp(-x))


def beta_from_log(log_beta: np.ndarray | float) -> np.ndarray:
    """``exp(clamp(log_beta, ln 0.05, ln 64))`` (modules.py:130-132)."""

    return np.exp(np.clip(np.asarray(log_beta), LOG_BETA_MIN, LOG_BETA_MAX))


def score_scale_from_log(log_scale: np.ndarray) -> np.ndarray:
    """``exp(clamp(log_scale, ln 0.25, ln 1024))`` (ops.py:160-161)."""

    return np.exp(np.clip(np.asarray(log_scale), LOG_SCALE_MIN, LOG_SCALE_MAX))


def bank_normalized(raw_key: np.ndarray, raw_value: np.ndarray | None, eps: float = 1e-6):
    """Unit-norm atoms (columns) of a bank; tied banks reuse the key (modules.py:45-48)."""

    key = l2_normalize(raw_key, 0, eps)
    value = key if raw_value is None else l2_normalize(raw_value, 0, eps)
    return key, value


def bank_normalized_backward(raw_key: np.ndarray, raw_value: np.ndarray | None, grad_key: np.ndarray,
                             grad_value: np.ndarray, eps: float = 1e-6):
    """Gradients at the raw bank of ``bank_normalized`` (modules.py:45-48 under
    autograd): each column through ``v / max(|v|, eps)``; a tied bank's key
    atoms collect both gradients.  Returns ``(d_raw_key, d_raw_value or None)``."""

    if raw_value is None:
        return _normalize_backward(raw_key.T, (grad_key + grad_value).T, eps).T, None
    return _normalize_backward(raw_key.T, grad_key.T, eps).T, _normalize_backward(raw_value.T, grad_value.T, eps).T


def dictionary_route(
    x: np.ndarray,
    dictionary_key: np.ndarray,
    dictionary_value: np.ndarray,
    beta: float | np.ndarray,
    eps: float = 1e-6,
    activation: str = "identity",
    assignment: str = "softmax",
    silu_gain: float = 1.0,
    standardize_logits: bool = False,
    standardized_logit_scale: float | None = None,
    normalize_input: bool = True,
    normalize_output: bool = True,
) -> np.ndarray:
    """Dictionary feature map of ``x [..., R]`` (ops.py:16-62)."""

    dt = x.dtype
    u = l2_normalize(x, -1, eps) if normalize_input else x
    logits = u @ dictionary_key.astype(dt)
    if activation == "silu":
        logits = 2.0 * _silu(logits)
    elif activation != "identity":
        raise ValueError(activation)
    if standardize_logits:
        centered = logits - logits.mean(axis=-1, keepdims=True)
        inv_std = 1.0 / np.sqrt(np.mean(centered * centered, axis=-1, keepdims=True) + eps)
        scale = x.shape[-1] ** -0.5 if standardized_logit_scale is None else standardized_logit_scale
        logits = centered * inv_std * scale
    if assignment == "softmax":
        weights = _softmax(logits * np.asarray(beta, dtype=dt), -1)
    elif assignment == "silu":
        weights = (2.0 / silu_gain) * _silu(silu_gain * logits)
    else:
        raise ValueError(assignment)
    recon = weights @ dictionary_value.astype(dt).T
    return l2_normalize(recon, -1, eps) if normalize_output else recon


def _normalize_backward(v: np.ndarray, grad: np.ndarray, eps: float) -> np.ndarray:
    """Gradient through ``v / max(|v|, eps)`` along the last axis."""

    norm = np.sqrt(np.sum(v * v, axis=-1, keepdims=True))
    unit = v / np.maximum(norm, eps)
    projected = (grad - unit * np.sum(unit * grad, axis=-1, keepdims=True)) / np.maximum(norm, eps)
    return np.where(norm > eps, projected, grad / eps)


def dictionary_route_backward(
    x: np.ndarray,
    dictionary_key: np.ndarray,
    dictionary_value: np.ndarray,
    beta: float,
    grad_out: np.ndarray,
    eps: float = 1e-6,
    normalize_input: bool = True,
    normalize_output: bool = True,
    activation: str = "identity",
    assignment: str = "softmax",
    silu_gain: float = 1.0,
    standardize_logits: bool = False,
    standardized_logit_scale: float | None = None,
    return_dbeta_rows: bool = False,
):
    """Gradients of :func:`dictionary_route` (ops.py:16-62), every variant.

    ``z = N_out(w Dv^T)`` with ``w = softmax(beta a)`` or ``(2/g) SiLU(g a)``,
    ``a = Std(Act(u Dk))`` and ``u = N_in(x)``; returns ``(dx, dDk, dDv,
    dbeta)`` for ``d loss / dz = grad_out`` -- what the reference's autograd
    returns for ``dictionary_route_reference`` (dbeta is 0 for the SiLU
    assignment, which does not use beta); with ``return_dbeta_rows`` also each
    row's term of dbeta (the sum is often far smaller than its terms).  The chain rule, step by step:
    the softmax backward ``d(beta a) = w (dw - sum w dw)``; the SiLU
    assignment ``da = dw 2 SiLU'(g a)``; the standardization's backward
    ``da0 = isd (dc - mean dc - c mean(dc c))`` with ``c`` the standardized
    values and ``dc = s da``; the activation ``dl = da0 2 SiLU'(l)``, where
    ``SiLU'(t) = sig(t) (1 + t (1 - sig(t)))``.
    """

    dt = x.dtype
    u = l2_normalize(x, -1, eps) if normalize_input else x
    logits = u @ dictionary_key.astype(dt)
    if activation == "silu":
        sig_l = 1.0 / (1.0 + np.exp(-logits))
        act = 2.0 * logits * sig_l
    elif activation == "identity":
        act = logits
    else:
        raise ValueError(activation)
    if standardize_logits:
        centered = act - act.mean(axis=-1, keepdims=True)
        inv_std = 1.0 / np.sqrt(np.mean(centered * centered, axis=-1, keepdims=True) + eps)
        standardized = centered * inv_std
        scale = x.shape[-1] ** -0.5 if standardized_logit_scale is None else standardized_logit_scale
        assign = standardized * scale
    else:
        assign = act
    if assignment == "softmax":
        weights = _softmax(assign * beta, -1)
    elif assignment == "silu":
        sig_a = 1.0 / (1.0 + np.exp(-silu_gain * assign))
        weights = (2.0 / silu_gain) * (silu_gain * assign) * sig_a
    else:
        raise ValueError(assignment)
    recon = weights @ dictionary_value.astype(dt).T
    d_recon = _normalize_backward(recon, grad_out, eps) if normalize_output else grad_out
    d_weights = d_recon @ dictionary_value.astype(dt)
    if assignment == "softmax":
        d_scores = weights * (d_weights - np.sum(weights * d_weights, axis=-1, keepdims=True))
        d_assign = beta * d_scores
        d_beta_rows = np.sum(d_scores * assign, axis=-1)
    else:
        t = silu_gain * assign
        d_assign = d_weights * 2.0 * sig_a * (1.0 + t * (1.0 - sig_a))
        d_beta_rows = np.zeros(assign.shape[:-1], dtype=dt)
    d_beta = float(np.sum(d_beta_rows))
    if standardize_logits:
        d_std = d_assign * scale
        d_act = inv_std * (
            d_std
            - d_std.mean(axis=-1, keepdims=True)
            - standardized * np.mean(d_std * standardized, axis=-1, keepdims=True)
        )
    else:
        d_act = d_assign
    if activation == "silu":
        d_logits = d_act * 2.0 * sig_l * (1.0 + logits * (1.0 - sig_l))
    else:
        d_logits = d_act
    d_u = d_logits @ dictionary_key.astype(dt).T
    dx = _normalize_backward(x, d_u, eps) if normalize_input else d_u
    rows_u = u.reshape(-1, u.shape[-1])
    d_key = rows_u.T @ d_logits.reshape(-1, d_logits.shape[-1])
    d_value = d_recon.reshape(-1, d_recon.shape[-1]).T @ weights.reshape(-1, weights.shape[-1])
    if return_dbeta_rows:
        return dx, d_key, d_value, d_beta, d_beta_rows
    return dx, d_key, d_value, d_beta


def routed_attention(
    query: np.ndarray, key: np.ndarray, value: np.ndarray, scales: np.ndarray, causal: bool = True
) -> np.ndarray:
    """``softmax(scale_s q k^T, causal) V`` for every map (ops.py:65-93).

    ``query``/``key`` ``[B, S, T, R]``, ``value`` ``[B, T, D]`` shared by all
    maps; returns ``[B, S, T, D]``.  Future positions get ``-inf``.
    """

    dt = query.dtype
    scores = np.matmul(query, np.swapaxes(key, -1, -2)) * np.asarray(scales, dtype=dt)[None, :, None, None]
    if causal:
        length = query.shape[-2]
        future = np.triu(np.ones((length, length), dtype=bool), 1)
        scores = np.where(future, -np.inf, scores)
    probs = _softmax(scores, -1)
    return np.matmul(probs, value.astype(dt)[:, None])


def routed_attention_backward(
    query: np.ndarray,
    key: np.ndarray,
    value: np.ndarray,
    scales: np.ndarray,
    grad_out: np.ndarray,
    causal: bool = True,
):
    """Gradients of :func:`routed_attention` for an output gradient ``grad_out``.

    With ``P = softmax(scale_s q k^T)``: ``dV = sum_s P^T dO``,
    ``dP = dO V^T``, ``dS = P (dP - rowsum(dP P))``, ``dq = scale_s dS k``,
    ``dk = scale_s dS^T q``, ``dscale_s = sum dS (q k^T)`` -- the gradients the
    reference's autograd path returns for ops.py:65-93 (its Triton backward,
    triton_kernels.py:2093-2263, computes the same products).  Returns
    ``(dq, dk, dv, dscales)``.
    """

    dt = query.dtype
    raw = np.matmul(query, np.swapaxes(key, -1, -2))
    scores = raw * np.asarray(scales, dtype=dt)[None, :, None, None]
    if causal:
        length = query.shape[-2]
        future = np.triu(np.ones((length, length), dtype=bool), 1)
        scores = np.where(future, -np.inf, scores)
    probs = _softmax(scores, -1)
    dv = np.matmul(np.swapaxes(probs, -1, -2), grad_out).sum(axis=1)
    dp = np.matmul(grad_out, value.astype(dt)[:, None].swapaxes(-1, -2))
    ds = probs * (dp - (dp * probs).sum(-1, keepdims=True))
    sc = np.asarray(scales, dtype=dt)[None, :, None, None]
    dq = np.matmul(ds, key) * sc
    dk = np.matmul(np.swapaxes(ds, -1, -2), query) * sc
    dscales = (ds * np.where(np.isfinite(scores), raw, 0)).sum(axis=(0, 2, 3))
    return dq, dk, dv.astype(dt), dscales


def assemble_score_maps(query: np.ndarray, key: np.ndarray, outer_maps: int):
    """Branch-to-map assembly (ops.py:96-139): identity, RMS-sum groups or repeats."""

    branches = query.shape[1]
    if branches == outer_maps:
        return query, key
    if branches > outer_maps:
        group = branches // outer_maps
        factor = group ** -0.25

        def grouped(t: np.ndarray) -> np.ndarray:
            b, _, length, width = t.shape
            parts = t.reshape(b, outer_maps, group, length, width).transpose(0, 1, 3, 2, 4)
            return parts.reshape(b, outer_maps, length, group * width) * factor

        return grouped(query), grouped(key)
    repeats = outer_maps // branches
    return np.repeat(query, repeats, axis=1), np.repeat(key, repeats, axis=1)


def shared_dictionary_attention(
    params: Mapping[str, np.ndarray],
    cfg: Any,
    x: np.ndarray,
    normalized_dictionary: tuple[np.ndarray, np.ndarray] | None = None,
    prefix: str = "",
    return_routed: bool = False,
    routed: tuple[np.ndarray, np.ndarray] | None = None,
):
    """``SharedDictionaryAttention.forward`` (modules.py:190-291) on NumPy arrays.

    ``params`` holds the module's state-dict entries under ``prefix``; the
    bank comes from ``prefix + 'bank.'`` unless ``normalized_dictionary`` is
    given.  ``routed`` = (routed query, routed key), each ``[B, H, T, R]``,
    replaces the route's output (modules.py:239-241) so that the stages after
    it (score maps, outer attention, mix, output projection) can be checked
    on given routed rows.
    """

    dt = x.dtype

    def p(name: str) -> np.ndarray | None:
        v = params.get(prefix + name)
        return None if v is None else np.asarray(v, dtype=dt)

    batch, length, _ = x.shape
    branches = _cfg(cfg, "qk_branches")
    routing = _cfg(cfg, "routing_dim")
    maps = _cfg(cfg, "outer_maps")
    eps = _cfg(cfg, "eps")

    def project(weight: np.ndarray) -> np.ndarray:
        return (x @ weight.T).reshape(batch, length, branches, routing).transpose(0, 2, 1, 3)

    query = project(p("query.weight"))
    key = project(p("key.weight"))
    value = x @ p("value.weight").T
    if p("value.bias") is not None:
        value = value + p("value.bias")
    if normalized_dictionary is None:
        dk, dv = bank_normalized(p("bank.raw_key"), p("bank.raw_value"), eps)
    else:
        dk, dv = (np.asarray(t, dtype=dt) for t in normalized_dictionary)
    beta = beta_from_log(p("log_beta"))
    if routed is None:
        pair = dictionary_route(
            np.concatenate([query, key], axis=2), dk, dv, beta, eps,
            _cfg(cfg, "dictionary_activation"), _cfg(cfg, "dictionary_assignment"),
            _cfg(cfg, "dictionary_silu_gain"), _cfg(cfg, "standardize_dictionary_logits"),
            _cfg(cfg, "standardized_logit_scale"), _cfg(cfg, "normalize_routing_input"),
            _cfg(cfg, "normalize_routing_output"),
        )
        routed_query, routed_key = pair[:, :, :length], pair[:, :, length:]
    else:
        routed_query, routed_key = (np.asarray(t, dtype=dt) for t in routed)
    score_query, score_key = assemble_score_maps(routed_query, routed_key, maps)
    scales = score_scale_from_log(p("log_score_scales"))
    map_output = routed_attention(score_query, score_key, value, scales, _cfg(cfg, "causal"))
    if _cfg(cfg, "map_combine") == "weighted_sum":
        if maps == 1:
            combined = map_output[:, 0]
        else:
            alpha = _softmax(p("map_mix_logits"), 0)
            combined = np.einsum("s,bstd->btd", alpha, map_output)
    else:
        combined = map_output.transpose(0, 2, 1, 3).reshape(batch, length, -1)
    out = combined @ p("output.weight").T if p("output.weight") is not None else combined
    if return_routed:
        return out, routed_query, routed_key
    return out


def assemble_score_maps_backward(grad_query: np.ndarray, grad_key: np.ndarray, branches: int):
    """Gradients at the routed branches of :func:`assemble_score_maps` (its
    three layouts are linear: identity, scaled concatenation of a group, repeat)."""

    outer_maps = grad_query.shape[1]
    if branches == outer_maps:
        return grad_query, grad_key
    if branches > outer_maps:
        group = branches // outer_maps
        factor = group ** -0.25

        def ungrouped(g: np.ndarray) -> np.ndarray:
            b, _, length, gw = g.shape
            width = gw // group
            parts = g.reshape(b, outer_maps, length, group, width).transpose(0, 1, 3, 2, 4)
            return parts.reshape(b, branches, length, width) * factor

        return ungrouped(grad_query), ungrouped(grad_key)
    repeats = outer_maps // branches

    def summed(g: np.ndarray) -> np.ndarray:
        b, _, length, width = g.shape
        return g.reshape(b, branches, repeats, length, width).sum(axis=2)

    return summed(grad_query), summed(grad_key)


def shared_dictionary_attention_backward(
    params: Mapping[str, np.ndarray],
    cfg: Any,
    x: np.ndarray,
    grad_out: np.ndarray,
    prefix: str = "",
) -> dict[str, np.ndarray]:
    """Gradients of :func:`shared_dictionary_attention` (modules.py:190-291
    under autograd) for ``d loss / d out = grad_out``, the module's own bank.

    The chain of the forward's stages, each through a backward pinned on its
    own: the output projection, the map combine (the mix softmax's backward
    ``alpha (da - sum alpha da)``, or the concat split),
    :func:`routed_attention_backward` (with the score scale's clamp),
    :func:`assemble_score_maps_backward`, :func:`dictionary_route_backward`
    over the Q and K rows together (with beta's clamp),
    :func:`bank_normalized_backward`, then the Q, K and V projections.
    Returns ``{"x": dx, <state-dict name>: gradient}`` for every parameter
    (and for ``log_beta`` whether or not it is a parameter).
    """

    dt = x.dtype

    def p(name: str) -> np.ndarray | None:
        v = params.get(prefix + name)
        return None if v is None else np.asarray(v, dtype=dt)

    batch, length, model_dim = x.shape
    branches = _cfg(cfg, "qk_branches")
    routing = _cfg(cfg, "routing_dim")
    maps = _cfg(cfg, "outer_maps")
    eps = _cfg(cfg, "eps")
    causal = _cfg(cfg, "causal")
    grads: dict[str, np.ndarray] = {}

    # Forward again, keeping the intermediates.
    def project(weight: np.ndarray) -> np.ndarray:
        return (x @ weight.T).reshape(batch, length, branches, routing).transpose(0, 2, 1, 3)

    query, key = project(p("query.weight")), project(p("key.weight"))
    value = x @ p("value.weight").T
    if p("value.bias") is not None:
        value = value + p("value.bias")
    raw_key, raw_value = p("bank.raw_key"), p("bank.raw_value")
    dk, dv = bank_normalized(raw_key, raw_value, eps)
    log_beta = p("log_beta")
    beta = float(beta_from_log(log_beta))
    route_kw = dict(
        activation=_cfg(cfg, "dictionary_activation"), assignment=_cfg(cfg, "dictionary_assignment"),
        silu_gain=_cfg(cfg, "dictionary_silu_gain"), standardize_logits=_cfg(cfg, "standardize_dictionary_logits"),
        standardized_logit_scale=_cfg(cfg, "standardized_logit_scale"),
        normalize_input=_cfg(cfg, "normalize_routing_input"), normalize_output=_cfg(cfg, "normalize_routing_output"),
    )
    rows = np.concatenate([query, key], axis=2)
    pair = dictionary_route(
        rows, dk, dv, beta, eps, route_kw["activation"], route_kw["assignment"], route_kw["silu_gain"],
        route_kw["standardize_logits"], route_kw["standardized_logit_scale"], route_kw["normalize_input"],
        route_kw["normalize_output"],
    )
    score_query, score_key = assemble_score_maps(pair[:, :, :length], pair[:, :, length:], maps)
    log_scales = p("log_score_scales")
    scales = score_scale_from_log(log_scales)
    map_output = routed_attention(score_query, score_key, value, scales, causal)
    combine = _cfg(cfg, "map_combine")
    alpha = None
    if combine == "weighted_sum":
        combined = map_output[:, 0] if maps == 1 else np.einsum("s,bstd->btd", _softmax(p("map_mix_logits"), 0),
                                                               map_output)
        if maps > 1:
            alpha = _softmax(p("map_mix_logits"), 0)
    else:
        combined = map_output.transpose(0, 2, 1, 3).reshape(batch, length, -1)

    # Output projection.
    g = np.asarray(grad_out, dtype=dt)
    w_out = p("output.weight")
    if w_out is not None:
        grads["output.weight"] = g.reshape(-1, g.shape[-1]).T @ combined.reshape(-1, combined.shape[-1])
        d_combined = g @ w_out
    else:
        d_combined = g
    # Map combine.
    if combine == "weighted_sum":
        if maps == 1:
            d_maps = d_combined[:, None]
        else:
            d_maps = alpha[None, :, None, None] * d_combined[:, None]
            d_alpha = np.einsum("btd,bstd->s", d_combined, map_output)
            grads["map_mix_logits"] = alpha * (d_alpha - np.sum(alpha * d_alpha))
    else:
        d_maps = d_combined.reshape(batch, length, maps, model_dim).transpose(0, 2, 1, 3)
    # Outer attention and its score scales (clamp: the gradient passes inside).
    d_sq, d_sk, d_value, d_scales = routed_attention_backward(score_query, score_key, value, scales, d_maps, causal)
    inside = (log_scales >= LOG_SCALE_MIN) & (log_scales <= LOG_SCALE_MAX)
    grads["log_score_scales"] = d_scales * scales * inside
    # Score maps, then the route of the Q and K rows together.
    d_rq, d_rk = assemble_score_maps_backward(d_sq, d_sk, branches)
    d_rows, d_dk, d_dv, d_beta = dictionary_route_backward(
        rows, dk, dv, beta, np.concatenate([d_rq, d_rk], axis=2), eps, **route_kw
    )
    inside_beta = LOG_BETA_MIN <= float(log_beta) <= LOG_BETA_MAX
    grads["log_beta"] = np.asarray(d_beta * beta * inside_beta, dtype=dt)
    d_raw_key, d_raw_value = bank_normalized_backward(raw_key, raw_value, d_dk, d_dv, eps)
    grads["bank.raw_key"] = d_raw_key
    if d_raw_value is not None:
        grads["bank.raw_value"] = d_raw_value
    # Projections.
    x2 = x.reshape(-1, model_dim)

    def unproject(d: np.ndarray) -> np.ndarray:
        return d.transpose(0, 2, 1, 3).reshape(-1, branches * routing)

    d_q, d_k = unproject(d_rows[:, :, :length]), unproject(d_rows[:, :, length:])
    d_v = d_value.reshape(-1, model_dim)
    grads["query.weight"] = d_q.T @ x2
    grads["key.weight"] = d_k.T @ x2
    grads["value.weight"] = d_v.T @ x2
    if p("value.bias") is not None:
        grads["value.bias"] = d_v.sum(axis=0)
    dx = d_q @ p("query.weight") + d_k @ p("key.weight") + d_v @ p("value.weight")
    grads["x"] = dx.reshape(x.shape)
    return grads


def layer_norm(x: np.ndarray, weight: np.ndarray, bias: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """``nn.LayerNorm`` over the last axis (biased variance)."""

    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    return (x - mean) / np.sqrt(var + eps) * weight + bias


def gelu(x: np.ndarray) -> np.ndarray:
    """Exact (erf) GELU, ``nn.GELU()``'s default."""

    return 0.5 * x * (1.0 + erf(x / math.sqrt(2.0)))


def double_attention_lm(
    params: Mapping[str, np.ndarray],
    cfg: Any,
    token_ids: np.ndarray,
    num_layers: int,
    dictionary_group_size: int | None = None,
    dtype: np.dtype = np.float64,
) -> np.ndarray:
    """``DoubleAttentionLM.forward`` logits (modules.py:332-356, 398-412, 444-460)."""

    def p(name: str) -> np.ndarray:
        return np.asarray(params[name], dtype=dtype)

    length = token_ids.shape[1]
    hidden = p("token_embedding.weight")[token_ids] + p("position_embedding.weight")[:length][None]
    group = dictionary_group_size or num_layers
    bank_count = math.ceil(num_layers / group)
    eps = _cfg(cfg, "eps")
    banks = []
    for i in range(bank_count):
        raw_value = params.get(f"stack.banks.{i}.raw_value")
        banks.append(
            bank_normalized(p(f"stack.banks.{i}.raw_key"), None if raw_value is None else np.asarray(raw_value, dtype), eps)
        )
    qffn = _cfg(cfg, "q_dictionary_feedforward")
    for layer in range(num_layers):
        pre = f"stack.blocks.{layer}."
        dictionary = banks[min(layer // group, bank_count - 1)]
        normed = layer_norm(hidden, p(pre + "attention_norm.weight"), p(pre + "attention_norm.bias"))
        hidden = hidden + shared_dictionary_attention(
            params, cfg, normed, normalized_dictionary=dictionary, prefix=pre + "attention."
        )
        normed = layer_norm(hidden, p(pre + "feedforward_norm.weight"), p(pre + "feedforward_norm.bias"))
        if qffn:
            expanded = (normed @ p(pre + "attention.query.weight").T) @ dictionary[0]
        else:
            expanded = normed @ p(pre + "feedforward.0.weight").T + p(pre + "feedforward.0.bias")
        hidden = hidden + gelu(expanded) @ p(pre + "feedforward.2.weight").T + p(pre + "feedforward.2.bias")
    hidden = layer_norm(hidden, p("final_norm.weight"), p("final_norm.bias"))
    return hidden @ p("token_embedding.weight").T
