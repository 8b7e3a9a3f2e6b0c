"""CPU tests of the package's PyTorch path, API surface and backend dispatch.

Mirrors the reference's CPU test strategy (reference ``tests/test_modules.py``):
golden outputs written by the reference itself, the default-init RNG stream,
state-dict names, normalize-once behaviour, config validation and clean
errors for unavailable backends.
"""

from __future__ import annotations

import copy
import math

import numpy as np
import pytest
import torch

import double_attention as da
import double_attention._lib as lib
import double_attention.modules as modules
from conftest import Golden, golden_names


def _assert_scaled(actual: torch.Tensor, expected: np.ndarray, tol: float = 1e-6) -> None:
    err = np.abs(actual.detach().numpy() - expected).max() / np.abs(expected).max()
    assert err <= tol, err


def _config(g: Golden) -> da.DoubleAttentionConfig:
    return da.DoubleAttentionConfig(**g.config)


# ---------------------------------------------------------------- goldens


@pytest.mark.parametrize("name", golden_names("attention"))
def test_default_init_and_forward_match_reference(name: str) -> None:
    g = Golden(name)
    torch.manual_seed(int(g["seed"]))
    module = da.SharedDictionaryAttention(_config(g))
    state = module.state_dict()
    # Same names in the same order, and bit-identical seeded default init.
    assert list(state) == list(g.params)
    for key, value in g.params.items():
        np.testing.assert_array_equal(state[key].numpy(), value, err_msg=key)
    module64 = copy.deepcopy(module).double().eval()
    with torch.no_grad():
        out, aux = module64(torch.from_numpy(g["x"]), return_aux=True)
    _assert_scaled(out, g["out"])
    np.testing.assert_allclose(aux.routing_query.numpy(), g["routing_query"], rtol=1e-10, atol=1e-12)
    assert aux.backend == "torch"


@pytest.mark.parametrize("name", golden_names("lm"))
def test_lm_default_init_and_logits_match_reference(name: str) -> None:
    g = Golden(name)
    torch.manual_seed(int(g["seed"]))
    model = da.DoubleAttentionLM(
        vocab_size=int(g["vocab"]),
        max_sequence_length=int(g["max_len"]),
        config=_config(g),
        num_layers=int(g["layers"]),
        dictionary_group_size=int(g["group"]),
        feedforward_dim=int(g["ffn"]),
    )
    state = model.state_dict()
    assert list(state) == list(g.params)
    for key, value in g.params.items():
        np.testing.assert_array_equal(state[key].numpy(), value, err_msg=key)
    with torch.no_grad():
        logits, loss = copy.deepcopy(model).double()(torch.from_numpy(g["ids"]))
    assert loss is None
    _assert_scaled(logits, g["logits"])


def test_lm_position_rows_match_an_embedding_lookup() -> None:
    """The LM reads positions 0..T-1 as the first T rows of its position
    table; the reference gathers them with an arange (modules.py:452-453).
    Logits, loss and every gradient agree bit for bit."""

    torch.manual_seed(3)
    model = da.DoubleAttentionLM(
        vocab_size=64, max_sequence_length=24,
        config=da.experiment_config("a1", model_dim=64, routing_dim=32, dictionary_size=48, backend="torch"),
        num_layers=1, feedforward_dim=96,
    )
    ids = torch.randint(0, 64, (2, 17))
    targets = torch.randint(0, 64, (2, 17))
    twin = copy.deepcopy(model)
    logits, loss = model(ids, targets)
    loss.backward()

    def lookup_forward(self, token_ids, targets=None):
        positions = torch.arange(token_ids.shape[1])
        hidden = self.token_embedding(token_ids) + self.position_embedding(positions)[None]
        out = self.lm_head(self._final_norm(self.stack(hidden)))
        return out, torch.nn.functional.cross_entropy(out.flatten(0, 1), targets.flatten())

    ref_logits, ref_loss = lookup_forward(twin, ids, targets)
    ref_loss.backward()
    assert torch.equal(logits, ref_logits) and torch.equal(loss, ref_loss)
    for (name, p), (_, q) in zip(model.named_parameters(), twin.named_parameters()):
        assert torch.equal(p.grad, q.grad), name
    assert model.position_embedding.weight.grad[17:].abs().max() == 0


# Parameter counts recorded in the reference's run reports for the 6-layer,
# d=512, vocab 2048, sequence 64 models (runs/tied/RESULTS.md:11,
# runs/screen/RESULTS.md:13, runs/a1_multicorpus_8k/python_docs/
# a1-r512-d1536_tied_s0_steps8000_sched12000.json).
@pytest.mark.parametrize(
    ("preset", "untied", "count"),
    [("qk2-s2", False, 16_969_752), ("a1", True, 15_527_942), ("a1-r512-d1536", False, 17_625_094)],
)
def test_parameter_counts_match_reference_runs(preset: str, untied: bool, count: int) -> None:
    config = da.experiment_config(preset, model_dim=512, untied_dictionary=untied, backend="torch")
    with torch.device("meta"):
        model = da.DoubleAttentionLM(2048, 64, config, 6, dictionary_group_size=6, feedforward_dim=1536)
    assert sum(p.numel() for p in model.parameters()) == count


# ---------------------------------------------------------------- module behaviour


def small_config(name: str, **overrides: object) -> da.DoubleAttentionConfig:
    values: dict[str, object] = {"model_dim": 32, "routing_dim": 8, "dictionary_size": 16, "backend": "torch"}
    values.update(overrides)
    return da.experiment_config(name, **values)


@pytest.mark.parametrize("name", da.experiment_names())
def test_all_presets_forward_and_backward(name: str) -> None:
    torch.manual_seed(7)
    module = da.SharedDictionaryAttention(small_config(name))
    x = torch.randn(2, 7, 32, requires_grad=True)
    out, aux = module(x, return_aux=True)
    assert out.shape == x.shape
    assert aux.routing_query.shape[:3] == (2, module.config.qk_branches, 7)
    assert aux.score_query.shape[:3] == (2, module.config.outer_maps, 7)
    assert aux.map_weights.shape == (module.config.outer_maps,)
    out.square().mean().backward()
    assert x.grad is not None and torch.isfinite(x.grad).all()
    assert module.bank.raw_key.grad is not None


def test_fused_and_separate_projection_agree(monkeypatch: pytest.MonkeyPatch) -> None:
    torch.manual_seed(8)
    module = da.SharedDictionaryAttention(small_config("qk2-s2"))
    assert not any("fused" in k for k in module.state_dict())
    x = torch.randn(2, 7, 32)
    monkeypatch.setattr(modules, "FUSED_QUERY_KEY_PROJECTION", False)
    separate = module(x)
    monkeypatch.setattr(modules, "FUSED_QUERY_KEY_PROJECTION", True)
    torch.testing.assert_close(module(x), separate, atol=1e-6, rtol=1e-5)


def test_stack_normalizes_each_bank_once(monkeypatch: pytest.MonkeyPatch) -> None:
    stack = da.DoubleAttentionStack(small_config("a1"), num_layers=6, dictionary_group_size=3, feedforward_dim=48)
    calls = 0
    original = modules.SharedDictionaryBank.normalized

    def counted(bank, eps=1e-6):
        nonlocal calls
        calls += 1
        return original(bank, eps)

    monkeypatch.setattr(modules.SharedDictionaryBank, "normalized", counted)
    stack(torch.randn(2, 6, 32)).square().mean().backward()
    assert calls == len(stack.banks) == 2


def test_tied_bank_shares_storage() -> None:
    module = da.SharedDictionaryAttention(small_config("a1", untied_dictionary=False))
    assert module.bank.raw_value is None
    key, value = module.bank.normalized()
    assert key.data_ptr() == value.data_ptr()


def test_causal_prefix_independent_of_future() -> None:
    torch.manual_seed(11)
    module = da.SharedDictionaryAttention(
        da.DoubleAttentionConfig(model_dim=16, routing_dim=8, dictionary_size=16, output_projection=False, backend="torch")
    ).eval()
    a = torch.randn(1, 8, 16)
    b = a.clone()
    b[:, 4:] = torch.randn_like(b[:, 4:]) * 10
    with torch.no_grad():
        torch.testing.assert_close(module(a)[:, :4], module(b)[:, :4], atol=1e-6, rtol=1e-5)


def test_config_validation_and_presets() -> None:
    with pytest.raises(ValueError, match="divide one another"):
        da.DoubleAttentionConfig(qk_branches=3, outer_maps=2)
    with pytest.raises(ValueError, match="unsupported backend"):
        da.DoubleAttentionConfig(backend="cuda")  # type: ignore[arg-type]
    assert da.DoubleAttentionConfig(backend="hip").backend == "hip"
    c = da.experiment_config("a1-r512-d1536")
    assert (c.routing_dim, c.dictionary_size) == (512, 1536)
    assert c.beta == pytest.approx(4 * math.sqrt(2)) and c.initial_score_scale == pytest.approx(math.sqrt(512))
    assert da.experiment_config("QK4_S4").qk_branches == 4
    with pytest.raises(ValueError, match="unknown experiment"):
        da.experiment_config("nope")
    assert len(da.experiment_names()) == 21


# ---------------------------------------------------------------- backend dispatch


def test_auto_backend_uses_torch_on_cpu() -> None:
    module = da.SharedDictionaryAttention(small_config("a1", backend="auto"))
    _, aux = module(torch.randn(1, 4, 32), return_aux=True)
    assert aux.backend == "torch"


def test_explicit_hip_backend_fails_cleanly_on_cpu() -> None:
    module = da.SharedDictionaryAttention(
        da.DoubleAttentionConfig(model_dim=64, routing_dim=64, dictionary_size=64, backend="hip")
    )
    with pytest.raises(RuntimeError, match="HIP backend requested"):
        module(torch.randn(1, 4, 64))


def test_triton_backend_fails_cleanly() -> None:
    module = da.SharedDictionaryAttention(small_config("a1", backend="triton"))
    with pytest.raises(RuntimeError, match="Triton backend requested"):
        module(torch.randn(1, 4, 32))
    assert da.TRITON_AVAILABLE is False


def test_missing_library_is_reported(monkeypatch: pytest.MonkeyPatch, tmp_path) -> None:
    monkeypatch.setenv("DOUBLE_ATTENTION_HIP_LIBRARY", str(tmp_path / "missing.so"))
    lib.reset()
    try:
        assert not lib.available()
        with pytest.raises(RuntimeError, match="HIP backend requested but unavailable.*missing.so"):
            da.ops.resolve_backend("hip", [torch.empty(1)])
        # auto on CPU tensors never needs the library
        assert da.ops.resolve_backend("auto", [torch.empty(1)]) == "torch"
    finally:
        monkeypatch.delenv("DOUBLE_ATTENTION_HIP_LIBRARY")
        lib.reset()


def test_hip_supports_every_preset_and_rejects_other_widths() -> None:
    from double_attention.hip_ops import check_module_supported

    for name in da.config._PRESETS:
        check_module_supported(da.experiment_config(name))
    with pytest.raises(NotImplementedError):
        check_module_supported(da.experiment_config("a1", routing_dim=96))
    # model_dim: any multiple of 64 up to 4096 (the attention's value slices
    # are 64, 128 or 256 features wide).
    for model_dim in (64, 192, 384, 768, 1024, 4096):
        check_module_supported(da.experiment_config("a1", model_dim=model_dim))
    for model_dim in (100, 32, 4160):
        with pytest.raises(NotImplementedError):
            check_module_supported(da.experiment_config("a1", model_dim=model_dim))


def test_route_variant_flags_follow_the_config() -> None:
    from double_attention import _lib
    from double_attention.hip_ops import RouteVariant

    assert RouteVariant.of_config(da.experiment_config("a1")).flags() == 0
    v = RouteVariant.of_config(da.experiment_config("a1-silu-logitnorm-t1"))
    assert v.flags() == _lib.DA_ROUTE_SILU_LOGITS | _lib.DA_ROUTE_STANDARDIZE
    assert v.logit_scale(256) == 0.25
    v = RouteVariant.of_config(da.experiment_config("a1-silu-logitnorm"))
    assert v.logit_scale(256) == 256 ** -0.5   # ops.py:50-54 default
    v = RouteVariant.of_config(da.experiment_config("a1-no-softmax-g4"))
    assert v.flags() == _lib.DA_ROUTE_DIRECT_SILU and v.silu_gain == 4.0


def test_backward_dispatch_rules() -> None:
    # Which shapes take the native backward kernels (host logic only).
    from double_attention import hip_ops

    q = torch.empty(2, 3, 10, 512)
    assert hip_ops._native_backward_supported(q, torch.empty(2, 10, 512))
    assert not hip_ops._native_backward_supported(torch.empty(1, 2, 10, 600), torch.empty(1, 10, 64))
    assert not hip_ops._native_backward_supported(torch.empty(40000, 2, 4, 64), torch.empty(40000, 4, 64))
    standard, silu = hip_ops.RouteVariant(), hip_ops.RouteVariant(silu_logits=True)
    key = torch.empty(256, 100)
    # CPU tensors never take the GPU path; on the GPU the width and variant decide.
    assert not hip_ops._route_backward_supported(torch.empty(5, 256, dtype=torch.bfloat16), key, standard)
    meta = torch.empty(5, 256, dtype=torch.bfloat16, device="meta")
    assert not hip_ops._route_backward_supported(meta, key, standard)   # not a CUDA tensor
    assert hip_ops.ROUTE_BACKWARD_WIDTHS == (64, 128, 256)
    assert 512 in hip_ops.BACKWARD_SCORE_WIDTHS
    assert silu.flags() != 0 and standard.flags() == 0
    # The row-kernel path takes every width, variant and bank size, on the GPU only.
    assert not hip_ops._route_backward_rows_supported(meta, key)
    assert hip_ops.ROUTE_BACKWARD_ROWS_MAX_ATOMS == 1 << 24
    # The dense attention backward: long sequences, 512-wide scores, wide values.
    assert hip_ops.DENSE_BACKWARD_MIN_LENGTH == 2048
    assert hip_ops._dense_backward_fits(torch.empty(1, 1, 8192, 256, device="meta"), torch.empty(1, 8192, 512, device="meta"))
    assert not hip_ops._dense_backward_fits(torch.empty(8, 1, 512, 256, device="meta"), torch.empty(8, 512, 512, device="meta"))
    assert hip_ops._dense_backward_fits(torch.empty(2, 1, 40, 256, device="meta"), torch.empty(2, 40, 768, device="meta"))
    assert not hip_ops._dense_backward_fits(torch.empty(1, 1, 20000, 256, device="meta"), torch.empty(1, 20000, 512, device="meta"))
    # route_backward_is_native: the module's choice of the raw-bank path.
    assert hip_ops.route_backward_is_native(256, 512, torch.bfloat16, standard)
    assert hip_ops.route_backward_is_native(512, 1536, torch.float16, silu)
    assert hip_ops.route_backward_is_native(128, 4096, torch.bfloat16, silu)
    assert hip_ops.route_backward_is_native(512, 4097, torch.bfloat16, standard)
    assert hip_ops.route_backward_is_native(256, 20000, torch.float16, silu)
    assert not hip_ops.route_backward_is_native(256, 512, torch.float32, standard)
    assert not hip_ops.route_backward_is_native(96, 512, torch.bfloat16, silu)


def test_auto_backend_picks_torch_for_uncovered_configs() -> None:
    # backend="auto" keeps a configuration the kernels do not cover on torch;
    # "hip" raises for it instead (host logic: no GPU needed).
    assert modules._hip_covers(da.experiment_config("a1"))
    assert not modules._hip_covers(da.experiment_config("a1", routing_dim=96))
    assert not modules._hip_covers(da.experiment_config("a1", model_dim=100))
    assert modules._hip_covers(da.experiment_config("a1", model_dim=384))


def test_module_operands_follow_parameter_updates() -> None:
    # The cast operands of the fused forward are reused while the parameters
    # are unchanged and rebuilt after an in-place update (version counter) or
    # a new tensor (data pointer).
    from double_attention import hip_ops

    module = da.SharedDictionaryAttention(da.experiment_config("a1"))
    first = hip_ops._module_operands(module, torch.bfloat16)
    assert hip_ops._module_operands(module, torch.bfloat16) is first
    with torch.no_grad():
        module.query.weight.mul_(2.0)
    second = hip_ops._module_operands(module, torch.bfloat16)
    assert second is not first
    torch.testing.assert_close(second[0], module.query.weight.detach().to(torch.bfloat16))
    module.key.weight = torch.nn.Parameter(torch.zeros_like(module.key.weight))
    third = hip_ops._module_operands(module, torch.bfloat16)
    assert third is not second and torch.count_nonzero(third[1]) == 0
    assert hip_ops._module_operands(module, torch.float16)[0].dtype == torch.float16


def test_route_layout_is_reused_while_the_bank_is_unchanged() -> None:
    # The blocks of a stack share one normalized bank: the first lays it out,
    # the others reuse that layout; an in-place change (version bump) makes it
    # stale, and parameters are never tagged (writes through .data bypass the
    # version counter).  The layout itself holds the atom-major keys and the
    # 32-atom value tiles of the same numbers.
    from double_attention import hip_ops

    g = torch.Generator().manual_seed(0)
    key = torch.randn(64, 40, generator=g)
    value = torch.randn(64, 40, generator=g)
    first = hip_ops.route_layout(key, value, torch.float16)
    assert hip_ops.route_layout(key, value, torch.float16) is first
    assert torch.equal(first.key_t[:40].float(), key.t().half().float())
    assert torch.count_nonzero(first.key_t[40:]) == 0 and first.key_t.shape == (64, 64)
    assert torch.equal(hip_ops._untile_value(first.value)[:, :40].float(), value.half().float())
    # Another key dtype lays it out again.
    assert hip_ops.route_layout(key, value, torch.bfloat16) is not first
    again = hip_ops.route_layout(key, value, torch.float16)
    value.mul_(2.0)
    fresh = hip_ops.route_layout(key, value, torch.float16)
    assert fresh is not again
    assert torch.equal(hip_ops._untile_value(fresh.value)[:, :40].float(), value.half().float())
    param = torch.nn.Parameter(torch.randn(64, 40, generator=g))
    a = hip_ops.route_layout(param, param, torch.float16)
    assert hip_ops.route_layout(param, param, torch.float16) is not a
