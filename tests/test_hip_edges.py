"""GPU parity at the edges of the module's numerics.

* The C4 LM (qk2-s2, tied bank, 6 layers, tokens [64, 64]) layer by layer:
  every layer's HIP attention gets the same LayerNorm output as the fp32
  oracle, and its attention output is held to the absolute bar (relative L2
  <= 5e-3, max-abs <= 2e-2) in bf16 and fp16.
* A caller-supplied ``normalized_dictionary`` whose atoms are not unit
  vectors (norm 2): the route must not assume unit keys (its bounded,
  fixed-reference softmax would overflow fp16 there).  Reference: a
  non-normalized dictionary is accepted by ``modules.py:190-231``.
* The beta and gamma clamps (reference ``modules.py:130-132``,
  ``ops.py:160-161``): ``log_beta`` and ``log_score_scales`` below and above
  their clamp ranges.  At gamma = 1024 a 1e-3 difference in a routed row moves
  a score by about 1, so no 16-bit path can match the fp32 oracle end to end;
  there the oracle takes the kernel's own fp16 routed rows and checks every
  stage after the route (score maps, attention with the clamped scale, mix,
  output projection), while the routed rows themselves are checked against
  the oracle's route with the clamped beta.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import double_attention as da
import oracle
from test_hip_parity import DTYPES, REL_L2, _device, assert_parity, np32, oracle_params

pytestmark = pytest.mark.gpu


def _hip_routed(module, x, dtype, normalized_dictionary=None):
    """The fused forward's output and its fp16 routed rows as [B, H, T, R] (query, key)."""

    with torch.inference_mode():
        result = module._hip_call(x, module.bank, normalized_dictionary, dtype)
    torch.cuda.synchronize()
    routed = result.routed  # [B, T, 2, H, R] fp16
    rq = routed[:, :, 0].permute(0, 2, 1, 3)
    rk = routed[:, :, 1].permute(0, 2, 1, 3)
    return result.output, rq, rk


@pytest.mark.parametrize("dtype", DTYPES)
def test_lm_c4_attention_output_per_layer(dtype) -> None:
    device = _device()
    config = da.experiment_config("qk2-s2", untied_dictionary=False, backend="hip")
    torch.manual_seed(0)
    model = da.DoubleAttentionLM(2048, 64, config, 6, dictionary_group_size=6, feedforward_dim=1536)
    model = model.to(device=device, dtype=dtype).eval()
    ids = torch.randint(0, 2048, (64, 64), generator=torch.Generator().manual_seed(1)).to(device)
    params = oracle_params(model)
    bank = model.stack.banks[0]
    # The oracle's bank: the tied raw atoms (in the model dtype) normalized in fp32.
    dk, dv = oracle.bank_normalized(params["stack.banks.0.raw_key"], None, config.eps)
    with torch.inference_mode():
        dictionary = bank.normalized_hip(config.eps, da.hip_ops.route_key_dtype(True, dtype))
        positions = torch.arange(64, device=device)
        hidden = model.token_embedding(ids) + model.position_embedding(positions)[None]
        for layer, block in enumerate(model.stack.blocks):
            normed = block.attention_norm(hidden)
            out = block.attention(normed, bank=bank, normalized_dictionary=dictionary)
            torch.cuda.synchronize()
            expected = oracle.shared_dictionary_attention(
                params, config, np32(normed), normalized_dictionary=(dk, dv), prefix=f"stack.blocks.{layer}.attention."
            )
            assert_parity(out, expected, label=f"c4 layer {layer} attention output {dtype}")
            hidden = block(hidden, bank, normalized_dictionary=dictionary)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("log_beta", [math.log(4.0), math.log(9.0)])
def test_module_non_unit_normalized_dictionary(dtype, log_beta) -> None:
    # Atoms of norm 2: logits reach 2 beta, past the fixed-reference range the
    # kernel may use only for unit atoms.
    device = _device()
    config = da.experiment_config("a1", backend="hip")
    torch.manual_seed(2)
    module = da.SharedDictionaryAttention(config).to(device=device, dtype=dtype).eval()
    with torch.no_grad():
        module.log_beta.fill_(log_beta)
    g = torch.Generator().manual_seed(3)
    dk = 2.0 * torch.nn.functional.normalize(torch.randn(256, 512, generator=g), dim=0)
    dv = 2.0 * torch.nn.functional.normalize(torch.randn(256, 512, generator=g), dim=0)
    # Align some atoms with typical rows so the largest logits approach 2 beta.
    x = torch.randn(2, 96, 512, generator=g)
    dictionary = (dk.to(device, dtype), dv.to(device, dtype))
    x = x.to(device, dtype)
    out, rq, rk = _hip_routed(module, x, dtype, dictionary)
    params = oracle_params(module)
    expected, eq, ek = oracle.shared_dictionary_attention(
        params, config, np32(x), normalized_dictionary=tuple(np32(t) for t in dictionary), return_routed=True
    )
    assert torch.isfinite(out).all()
    assert_parity(rq, eq, label=f"norm-2 atoms routed q {dtype} beta {math.exp(log_beta):.1f}")
    assert_parity(rk, ek, label=f"norm-2 atoms routed k {dtype} beta {math.exp(log_beta):.1f}")
    assert_parity(out, expected, label=f"norm-2 atoms output {dtype} beta {math.exp(log_beta):.1f}")


def test_route_op_non_unit_atoms_large_logits() -> None:
    # The operator-level route with atoms of norm 3 and beta 8: logits up to 24.
    device = _device()
    g = torch.Generator().manual_seed(9)
    x = torch.randn(300, 128, generator=g).to(device, torch.bfloat16)
    dk = (3.0 * torch.nn.functional.normalize(torch.randn(128, 200, generator=g), dim=0)).to(device, torch.bfloat16)
    dv = torch.nn.functional.normalize(torch.randn(128, 200, generator=g), dim=0).to(device, torch.bfloat16)
    out = da.dictionary_route_hip(x, dk, dv, torch.tensor(8.0, device=device))
    expected = oracle.dictionary_route(np32(x), np32(dk), np32(dv), 8.0)
    assert_parity(out, expected, label="route norm-3 atoms beta 8")


# (preset, log_beta, log_score_scales): each value below or above its clamp
# range [ln .05, ln 64] / [ln .25, ln 1024].
CLAMP_CASES = [
    ("a1", math.log(0.01), (math.log(0.05),)),
    ("a1", math.log(500.0), (math.log(5000.0),)),
    ("a1", -20.0, (20.0,)),
    ("qk2-s2", math.log(200.0), (math.log(0.01), math.log(3000.0))),
    ("qk4-s4", math.log(0.001), (-9.0, math.log(2.0), math.log(1e5), math.log(16.0))),
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("preset", "log_beta", "log_scales"), CLAMP_CASES)
def test_module_beta_gamma_clamps(dtype, preset, log_beta, log_scales) -> None:
    device = _device()
    config = da.experiment_config(preset, backend="hip")
    torch.manual_seed(4)
    module = da.SharedDictionaryAttention(config).to(device=device, dtype=dtype).eval()
    with torch.no_grad():
        module.log_beta.fill_(log_beta)
        module.log_score_scales.copy_(torch.tensor(log_scales))
    x = torch.randn(2, 160, 512, generator=torch.Generator().manual_seed(5)).to(device, dtype)
    out, rq, rk = _hip_routed(module, x, dtype)
    params = oracle_params(module)
    _, eq, ek = oracle.shared_dictionary_attention(params, config, np32(x), return_routed=True)
    label = f"{preset} log_beta={log_beta:.2f} log_scales={tuple(round(v, 2) for v in log_scales)} {dtype}"
    # The route with the clamped beta.
    assert_parity(rq, eq, label=label + " routed q")
    assert_parity(rk, ek, label=label + " routed k")
    # Every later stage on the kernel's own fp16 routed rows, with the clamped gammas.
    expected = oracle.shared_dictionary_attention(params, config, np32(x), routed=(np32(rq), np32(rk)))
    assert_parity(out, expected, label=label + " output on the kernel's routed rows")
    # The check can see a skipped upper clamp: the unclamped beta and (one
    # map) the unclamped gamma give results well outside the bar.
    if log_beta > math.log(64.0):
        rows = (np32(x) @ params["query.weight"].T).reshape(-1, config.routing_dim)
        bank = oracle.bank_normalized(params["bank.raw_key"], params.get("bank.raw_value"), config.eps)
        unclamped_rows = oracle.dictionary_route(rows, *bank, float(np.exp(log_beta)), config.eps)
        clamped_rows = oracle.dictionary_route(rows, *bank, float(oracle.beta_from_log(log_beta)), config.eps)
        diff = np.linalg.norm(unclamped_rows - clamped_rows) / np.linalg.norm(clamped_rows)
        assert diff > 4 * REL_L2, f"an unclamped beta would not be detected: {diff:.2e}"
    if preset == "a1" and log_scales[0] > math.log(1024.0):
        value = np32(x) @ params["value.weight"].T + params["value.bias"]
        sq, sk = oracle.assemble_score_maps(np32(rq), np32(rk), 1)
        unclamped = oracle.routed_attention(sq, sk, value, np.exp(np.asarray(log_scales, np.float32)), True)
        unclamped = unclamped[:, 0] @ params["output.weight"].T
        diff = np.linalg.norm(unclamped - expected) / np.linalg.norm(expected)
        assert diff > 4 * REL_L2, f"an unclamped gamma would not be detected: {diff:.2e}"
