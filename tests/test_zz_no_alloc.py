"""The allocation-free forward entry point against the workspace one.

``da_shared_dictionary_attention_forward_noalloc`` runs the same kernels as
``da_shared_dictionary_attention_forward`` with the workspace taken from the
library's per-GPU scratch array.  The kernels are deterministic (no atomics
in the forward), so its output must equal the workspace entry point's bit
for bit.  Each case makes two calls in a row through the C ABI, the second on
a smaller input, so stale scratch contents from the first call cannot leak
into the second.
"""

from __future__ import annotations

import pytest
import torch

import double_attention as da
from double_attention import _lib, hip_ops

pytestmark = pytest.mark.gpu


def _device() -> torch.device:
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    if not da.HIP_AVAILABLE:
        raise RuntimeError("HIP library not built; run python double-attention_amd/build.py")
    return torch.device("cuda")


def _both(module, x, dtype):
    key_dtype = hip_ops.route_key_dtype(module.config.normalize_routing_input, dtype)
    bank = (module.bank.raw_key, module.bank.raw_value)
    with torch.inference_mode():
        expected = hip_ops.shared_dictionary_attention_hip(
            module, x, hip_ops.own_bank_layout(module.bank, key_dtype), dtype, raw_bank=bank
        ).output
        got = hip_ops.shared_dictionary_attention_hip(
            module, x, hip_ops.own_bank_layout(module.bank, key_dtype), dtype, raw_bank=bank, no_alloc=True
        )
    torch.cuda.synchronize()
    assert got.routed is None
    return got.output, expected


@pytest.mark.parametrize(("preset", "first", "second"), [
    ("a1", (8, 512), (2, 77)),            # C1, then a ragged smaller batch
    ("qk4-s4", (8, 1024), (1, 300)),      # C2 (map mix), then smaller
    ("a1", (1, 8192), (1, 2000)),         # C5 (split key ranges: partials in the scratch), then smaller
    ("qk2-s2", (2, 600), (1, 65)),        # concat-free two-map mix
])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_noalloc_forward_matches_workspace_forward(preset, first, second, dtype) -> None:
    device = _device()
    config = da.experiment_config(preset, backend="hip")
    torch.manual_seed(0)
    module = da.SharedDictionaryAttention(config).to(device=device, dtype=dtype).eval()
    g = torch.Generator().manual_seed(1)
    for batch, length in (first, second):
        print(f"[noalloc] {preset} [{batch},{length},512] {dtype}", flush=True)
        x = torch.randn(batch, length, 512, generator=g).to(device, dtype)
        got, expected = _both(module, x, dtype)
        assert torch.isfinite(got).all()
        assert torch.equal(got, expected), f"{preset} {batch}x{length}: max diff {(got.float() - expected.float()).abs().max()}"


def test_noalloc_forward_rejects_oversized_problems() -> None:
    device = _device()
    config = da.experiment_config("a1", backend="hip")
    module = da.SharedDictionaryAttention(config).to(device=device, dtype=torch.bfloat16).eval()
    # [8, 8192] needs 8x the C5 workspace: beyond the scratch array.
    x = torch.zeros(8, 8192, 512, device=device, dtype=torch.bfloat16)
    need = _lib.get().da_sda_workspace_bytes(8, 8192, 512, 256, 1, 0, 1)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    with pytest.raises(ValueError, match="scratch"):
        hip_ops.shared_dictionary_attention_hip(
            module, x, hip_ops.own_bank_layout(module.bank, torch.float16), torch.bfloat16,
            raw_bank=(module.bank.raw_key, module.bank.raw_value), no_alloc=True,
        )
