"""CPU checks of the C-ABI library: it loads, exports every declared symbol,
and rejects bad arguments on the host before anything is launched."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

import double_attention._lib as lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "double_attention_hip.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(da_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol() -> None:
    handle = lib.get()
    names = declared_functions()
    assert len(names) == 28
    for name in names:
        assert hasattr(handle, name), name
        assert name in lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(lib.SIGNATURES) == set(names)


def test_abi_version_and_helpers() -> None:
    h = lib.get()
    assert h.da_abi_version() == lib.ABI_VERSION
    assert h.da_padded_atoms(512) == 512 and h.da_padded_atoms(513) == 576 and h.da_padded_atoms(2855) == 2880
    assert h.da_padded_length(65) == 128 and h.da_padded_length(8192) == 8192
    # C1 workspace: routed [4096, 512] + V^T [8, 512, 512] + mixed [4096, 512], bf16.
    assert h.da_sda_workspace_bytes(8, 512, 512, 256, 1, 0, 1) == 3 * 4096 * 512 * 2
    assert h.da_sda_workspace_bytes(8, 512, 512, 256, 1, 0, 0) == 2 * 4096 * 512 * 2
    # C5 (one long sequence) adds the fp32 partials of split causal key ranges.
    base_c5 = 8192 * 512 * 2 * 3
    partials = h.da_sda_workspace_bytes(1, 8192, 512, 256, 1, 0, 1) - base_c5
    assert partials > 0 and partials % 256 == 0
    assert h.da_sda_workspace_bytes(1, 8192, 512, 256, 4, 0, 1) == base_c5
    assert h.da_sda_workspace_offset(8, 512, 512, 256, 1) == 4096 * 512 * 2


def _fake(addr: int = 1 << 20) -> int:
    # A 256-aligned non-null address: only reaches host-side validation.
    return addr


@pytest.mark.parametrize(
    ("kwargs", "code", "pattern"),
    [
        ({"routing_dim": 96}, -2, "routing_dim 96"),
        ({"x_dtype": lib.DA_F32}, -1, "element types"),
        ({"flags": 2, "key_dtype": lib.DA_F16}, -2, "without input normalization"),
        ({"x_dtype": lib.DA_F16, "out_dtype": lib.DA_BF16}, -2, "out_dtype"),
        ({"x": 0, "rows": 0}, 0, "^$"),
        ({"x_row_stride": 100}, -3, "row strides"),
        ({"x": 0}, -1, "null pointer"),
        ({"x": (1 << 20) + 2}, -3, "16-byte aligned"),
        ({"atoms": 0}, -1, "rows/atoms"),
        ({"flags": 3 | lib.DA_ROUTE_BETA_IS_LOG_SCALE}, -1, "unknown flag bits"),   # row backward only
        ({"flags": 3 | lib.DA_ROUTE_DIRECT_SILU, "silu_gain": 0.0}, -1, "silu_gain"),
        ({"flags": 3 | lib.DA_ROUTE_STANDARDIZE, "logit_scale": float("inf")}, -1, "logit_scale"),
    ],
)
def test_route_rejects_bad_arguments_before_launch(kwargs, code, pattern) -> None:
    h = lib.get()
    args = dict(
        x=_fake(), rows=16, routing_dim=128, x_row_stride=128, x_dtype=lib.DA_BF16,
        key_t=_fake(), key_dtype=lib.DA_F16, value=_fake(), atoms=512,
        beta=None, beta_dtype=lib.DA_F32, beta_value=4.0, eps=1e-6, flags=3,
        silu_gain=1.0, logit_scale=0.0625,
        out=_fake(), out_row_stride=128, out_dtype=lib.DA_F16, stream=None,
    )
    args.update(kwargs)
    rc = h.da_dictionary_route(*args.values())
    assert rc == code
    assert re.search(pattern, h.da_last_error().decode())


def test_attention_rejects_bad_arguments_before_launch() -> None:
    h = lib.get()
    base = [
        _fake(), _fake(), 512 * 256, 256, 512 * 256, 1, 256,  # q, k, strides, map stride/repeat, score dim
        _fake(), 512 * 512,  # value_t, per-sequence pitch
        2, 1, 512, 512,  # batch, maps, length, value dim
        _fake(), lib.DA_F32, 1.0, None, lib.DA_F32,
        lib.DA_ATTN_CAUSAL, 1.0, lib.DA_F16, lib.DA_BF16, _fake(), 512 * 512, 512, 0, None, 0, None,
    ]
    bad_types = list(base)
    bad_types[20], bad_types[21] = lib.DA_BF16, lib.DA_F16
    assert h.da_routed_attention(*bad_types) == -2
    bad_dim = list(base)
    bad_dim[6] = 384
    assert h.da_routed_attention(*bad_dim) == -2
    short_pitch = list(base)
    short_pitch[8] = 512 * 448   # per-sequence pitch below value_dim * padded length
    assert h.da_routed_attention(*short_pitch) == -3
    assert "padded length" in h.da_last_error().decode()
    no_scales = list(base)
    no_scales[13] = None
    assert h.da_routed_attention(*no_scales) == -1
    bad_bound = list(base)
    bad_bound[19] = -1.0
    assert h.da_routed_attention(*bad_bound) == -1
    assert "score_bound" in h.da_last_error().decode()
    # Split-key scratch: a C5-sized causal problem wants some, a short one none;
    # a workspace that is given must be large enough.
    need = h.da_attention_workspace_bytes(1, 1, 8192, 256, 512, lib.DA_ATTN_CAUSAL)
    assert need > 0 and need % 256 == 0
    assert h.da_attention_workspace_bytes(2, 1, 512, 256, 512, lib.DA_ATTN_CAUSAL) == 0
    long_ctx = list(base)
    long_ctx[9], long_ctx[11], long_ctx[26], long_ctx[27] = 1, 8192, _fake(), need - 256
    long_ctx[8] = 8192 * 512
    assert h.da_routed_attention(*long_ctx) == -5


def test_forward_rejects_small_workspace() -> None:
    h = lib.get()
    f = _fake()
    args = lib.SdaForwardArgs(
        f, 8, 512, 512, 1, 1, 256, 512, f, f, f, f, f, f, f, f, f, None,
        lib.DA_F32, lib.DA_BF16, 1e-6, 7, f, 1024, f,
    )
    assert h.da_shared_dictionary_attention_forward(ctypes.byref(args), None) == -5
    assert "workspace" in h.da_last_error().decode()
    with pytest.raises(ValueError, match="workspace too small"):
        lib.check(-5, "forward")


def test_linear_ex_and_layer_norm_reject_bad_arguments() -> None:
    h = lib.get()
    good = [_fake(), 64, 512, _fake(), 512, None, lib.DA_F32, lib.DA_BF16, lib.DA_ACT_GELU, None, _fake(), None]
    bad_act = list(good)
    bad_act[8] = 7
    assert h.da_linear_ex(*bad_act) == -1
    assert "activation" in h.da_last_error().decode()
    bad_res = list(good)
    bad_res[9] = (1 << 20) + 2
    assert h.da_linear_ex(*bad_res) == -3
    ln = [_fake(), 64, 512, None, None, lib.DA_F32, 1e-5, lib.DA_BF16, _fake(), None]
    bad_dim = list(ln)
    bad_dim[2] = 100
    assert h.da_layer_norm(*bad_dim) == -2
    assert "multiple of 8" in h.da_last_error().decode()
    empty = list(ln)
    empty[1] = 0
    assert h.da_layer_norm(*empty) == 0


def test_attention_backward_rejects_bad_arguments() -> None:
    h = lib.get()
    f = _fake()
    need = h.da_attention_backward_workspace_bytes(2, 3, 100, 100, 128, 256)
    # Q^T, K^T and dO^T tiles over 128 padded tokens, two fp32 rows (6 * 100 * 4
    # = 2400 bytes, rounded up to 2560), value rows [2, 128, 256] for V^T
    # tiles (da_routed_attention_backward_ex), then eight fp32 copies of the
    # value bias's gradient [8, 256].
    assert need == 2 * (6 * 128 * 128 * 2) + 6 * 128 * 256 * 2 + 2 * 2560 + 2 * 128 * 256 * 2 + 8 * 256 * 4
    # Cross attention: K^T tiles follow the key count (300 -> 320 padded).
    cross = h.da_attention_backward_workspace_bytes(2, 3, 100, 300, 128, 256)
    assert cross == (6 * 128 * 128 * 2 + 6 * 320 * 128 * 2 + 6 * 128 * 256 * 2 + 2 * 2560 + 2 * 320 * 256 * 2
                     + 8 * 256 * 4)
    good = [f, f, f, f, f, f, 2, 3, 100, 100, 128, 256, lib.DA_ATTN_CAUSAL, lib.DA_BF16, lib.DA_BF16,
            f, need, f, f, f, f, None]
    cases = [
        (10, 96, -2, "score_dim 96"),
        (11, 96, -2, "value_dim 96"),
        (12, 4, -1, "flag bits"),
        (13, lib.DA_F32, -2, "qk_dtype"),
        (7, 65, -1, "maps"),
        (9, 300, -1, "key_length == length"),
        (0, 0, -1, "null pointer"),
        (3, (1 << 20) + 4, -3, "16-byte"),
        (19, (1 << 20) + 4, -3, "gradients"),
        (15, (1 << 20) + 16, -3, "workspace must be 256-byte"),
        (16, need - 1, -5, "workspace of"),
    ]
    for index, value, code, pattern in cases:
        args = list(good)
        args[index] = value
        assert h.da_routed_attention_backward(*args) == code, pattern
        assert pattern in h.da_last_error().decode(), h.da_last_error()
    empty = list(good)
    empty[8] = empty[9] = 0
    assert h.da_routed_attention_backward(*empty) == 0
    no_keys = list(good)
    no_keys[9] = 0
    no_keys[12] = 0
    assert h.da_routed_attention_backward(*no_keys) == -1
    # Log scales only through da_routed_attention_backward_ex.
    logs = list(good)
    logs[12] = lib.DA_ATTN_SCALES_ARE_LOG
    assert h.da_routed_attention_backward(*logs) == -1
    assert "flag bits" in h.da_last_error().decode()


def test_strided_attention_backward_rejects_bad_arguments() -> None:
    # da_routed_attention_backward_ex: the module layout [B, T, 2, H, R] of
    # C1's shape, then one bad field at a time.
    h = lib.get()
    f = _fake()
    need = h.da_attention_backward_workspace_bytes(8, 1, 512, 512, 256, 512)
    assert h.da_routed_attention_backward_ex(None, None) == -1
    assert "null args" in h.da_last_error().decode()

    def args(**changes):
        a = lib.AttentionBackwardArgs()
        a.query, a.query_stride_b, a.query_stride_t, a.query_map_stride = f, 512 * 512, 512, 256
        a.key, a.key_stride_b, a.key_stride_t, a.key_map_stride = f + 512, 512 * 512, 512, 256
        a.map_repeat = 1
        a.value = a.out = a.grad_out = a.scales = f
        a.out_dtype = lib.DA_F32
        a.scales_dtype, a.scale_mult = lib.DA_BF16, 1.0
        a.log_min, a.log_max = -1.3862944, 6.9314718
        a.batch, a.maps, a.length, a.key_length, a.score_dim, a.value_dim = 8, 1, 512, 512, 256, 512
        a.flags = lib.DA_ATTN_CAUSAL | lib.DA_ATTN_SCALES_ARE_LOG
        a.qk_dtype, a.v_dtype = lib.DA_F16, lib.DA_BF16
        a.workspace, a.workspace_bytes = f, need
        a.grad_query, a.grad_key, a.grad_value, a.grad_scales = f, f + 1024, f, f
        for name, value in changes.items():
            setattr(a, name, value)
        return a

    cases = [
        (dict(map_repeat=0), -1, "map_repeat"),
        (dict(maps=3, map_repeat=2), -1, "map_repeat"),
        (dict(query_stride_t=260), -3, "multiples of 8"),
        (dict(key_map_stride=-8), -3, "multiples of 8"),
        (dict(query_stride_t=128), -1, "stride_t must be >= score_dim"),
        (dict(scales_dtype=7), -1, "scales dtype"),
        (dict(scale_mult=0.0), -1, "scale_mult"),
        (dict(log_min=2.0, log_max=1.0), -1, "log_min <= log_max"),
        (dict(flags=lib.DA_ATTN_MIX), -1, "flag bits"),
        (dict(flags=lib.DA_ATTN_OUT_F32), -1, "flag bits"),   # out_dtype says it
        (dict(out_dtype=5), -1, "bad out dtype"),
        (dict(value=None, value_t=f, value_t_dtype=lib.DA_F32), -1, "V^T tiles"),
        (dict(value=None, value_t=f, value_t_dtype=lib.DA_F16, value_t_stride_b=12), -1, "V^T tiles"),
        (dict(value=None, value_t=None, value_t_dtype=lib.DA_F16), -1, "null pointer"),
        # Rows of scale * dS instead of the query gradient: padded key count, 16 bytes.
        (dict(grad_scores=f, grad_scores_ld=504), -3, "grad_scores"),
        (dict(grad_scores=f, grad_scores_ld=516), -3, "grad_scores"),
        (dict(grad_scores=f + 8, grad_scores_ld=512), -3, "grad_scores"),
        (dict(grad_scores=f, grad_scores_ld=512, grad_key=f + 1028), -3, "gradients"),
        (dict(grad_key=f + 1028), -3, "gradients"),
        (dict(scales=f + 1, scales_dtype=lib.DA_BF16), -3, "element size"),
        (dict(workspace_bytes=need - 1), -5, "workspace of"),
    ]
    for changes, code, pattern in cases:
        a = args(**changes)
        assert h.da_routed_attention_backward_ex(ctypes.byref(a), None) == code, (changes, h.da_last_error())
        assert pattern in h.da_last_error().decode(), h.da_last_error()
    empty = args(batch=0)
    assert h.da_routed_attention_backward_ex(ctypes.byref(empty), None) == 0


def test_noalloc_forward_rejects_oversized_problems_on_the_host() -> None:
    # The size check runs before anything touches a device: [8, 8192] tokens
    # need more workspace than the library's per-GPU scratch array.
    h = lib.get()
    args = lib.SdaForwardArgs()
    args.batch, args.length, args.model_dim = 8, 8192, 512
    args.qk_branches, args.outer_maps, args.routing_dim, args.atoms = 1, 1, 256, 512
    args.wo = _fake()
    assert h.da_sda_workspace_bytes(8, 8192, 512, 256, 1, 0, 1) > lib.NOALLOC_SCRATCH_BYTES
    rc = h.da_shared_dictionary_attention_forward_noalloc(ctypes.byref(args), None)
    assert rc == -5
    assert "scratch" in h.da_last_error().decode()
    args.batch = 0
    assert h.da_shared_dictionary_attention_forward_noalloc(ctypes.byref(args), None) == -1


def test_route_backward_rows_rejects_bad_arguments() -> None:
    # Host-side checks only: every call below fails before anything is launched.
    h = lib.get()
    buf = ctypes.c_void_p(16)   # never dereferenced

    def call(**kw):
        args = dict(logits=buf, grad_weights=buf, rows=10, atoms=100, causal_period=0, ld_in=100, beta=None,
                    beta_dtype=lib.DA_F32,
                    beta_value=1.0, beta_count=1, beta_period=1, flags=0, silu_gain=1.0, logit_scale=1.0, eps=1e-6, grad_logits=buf, weights=buf,
                    ld_out=100, out_dtype=lib.DA_BF16, dbeta_rows=None, stream=None)
        args.update(kw)
        return h.da_dictionary_route_backward_rows(*args.values())

    big = (1 << 24) + 1
    assert call(atoms=big, ld_in=big, ld_out=big) == -2    # more atoms than the row kernels take
    assert call(flags=lib.DA_ROUTE_NORMALIZE_INPUT) == -1   # not a flag of this entry point
    assert call(out_dtype=lib.DA_F32) == -1
    assert call(ld_in=50) == -1
    assert call(flags=lib.DA_ROUTE_DIRECT_SILU, silu_gain=0.0) == -1
    assert call(flags=lib.DA_ROUTE_STANDARDIZE, logit_scale=-1.0) == -1
    assert call(logits=None) == -1
    assert b"null" in h.da_last_error()
    assert call(causal_period=-1) == -1
    assert call(beta_count=3, beta_period=0) == -1
    assert b"beta_count" in h.da_last_error()
    assert call(rows=0, logits=None) == 0               # nothing to do
    both = lib.DA_ROUTE_BETA_IS_LOG | lib.DA_ROUTE_BETA_IS_LOG_SCALE
    assert call(flags=both) == -1 and b"exclude each other" in h.da_last_error()
    assert call(rows=0, flags=lib.DA_ROUTE_BETA_IS_LOG_SCALE) == 0



def test_normalize_backward_rejects_bad_arguments() -> None:
    h = lib.get()
    buf = ctypes.c_void_p(16)   # never dereferenced

    def call(**kw):
        args = dict(raw_key=buf, raw_value=buf, raw_dtype=lib.DA_F32, routing_dim=64, atoms=100, eps=1e-6,
                    grad_key=buf, grad_value=buf, grad_ld_r=100, grad_ld_j=1, d_raw_key=buf, d_raw_value=buf,
                    stream=None)
        args.update(kw)
        return h.da_dictionary_normalize_backward(*args.values())

    assert call(raw_dtype=7) == -1
    assert call(routing_dim=0) == -1
    assert call(atoms=0) == -1
    assert call(eps=-1.0) == -1
    assert call(grad_key=None) == -1
    assert b"null" in h.da_last_error()
    assert call(raw_value=None) == -1                   # d_raw_value for a tied bank
    assert b"tied" in h.da_last_error()
    # Gradient strides: coordinate-major (>= atoms, 1) or atom-major (1, >= routing_dim).
    assert call(grad_ld_r=99) == -1
    assert b"gradient strides" in h.da_last_error()
    assert call(grad_ld_r=1, grad_ld_j=63) == -1
    assert call(grad_ld_r=2, grad_ld_j=64) == -1


def test_row_normalize_rejects_bad_arguments() -> None:
    h = lib.get()
    buf = ctypes.c_void_p(1 << 20)   # never dereferenced

    def fwd(**kw):
        args = dict(x=buf, x_dtype=lib.DA_BF16, rows=10, width=256, ld_x=256, eps=1e-6, out=buf,
                    out_dtype=lib.DA_F16, ld_out=256, stream=None)
        args.update(kw)
        return h.da_row_normalize(*args.values())

    def bwd(**kw):
        args = dict(x=buf, x_dtype=lib.DA_F16, rows=10, width=256, ld_x=256, eps=1e-6, grad=buf,
                    grad_dtype=lib.DA_F32, ld_grad=256, grad_x=buf, out_dtype=lib.DA_BF16, ld_out=256, stream=None)
        args.update(kw)
        return h.da_row_normalize_backward(*args.values())

    assert fwd(x_dtype=7) == -1 and bwd(grad_dtype=7) == -1
    assert fwd(width=6) == -2 and b"multiple of 4" in h.da_last_error()
    assert fwd(eps=-1.0) == -1
    assert fwd(x=None) == -1 and bwd(grad=None) == -1
    assert b"null" in h.da_last_error()
    assert fwd(ld_x=128) == -3 and bwd(ld_grad=258) == -3
    assert fwd(x=ctypes.c_void_p((1 << 20) + 2)) == -3                     # 4 bf16 elements are 8 bytes
    assert bwd(grad=ctypes.c_void_p((1 << 20) + 8)) == -3 and b"aligned" in h.da_last_error()
    assert fwd(rows=0, x=None) == -1                                      # null checked before the empty case
    assert fwd(rows=0) == 0 and bwd(rows=0) == 0                          # nothing to do
    # DA_OUT_SPLIT: backward only, 16-bit outputs, two widths per output row.
    split = lib.DA_BF16 | lib.DA_OUT_SPLIT
    assert bwd(out_dtype=lib.DA_F32 | lib.DA_OUT_SPLIT) == -1 and b"16-bit" in h.da_last_error()
    assert bwd(out_dtype=split) == -3 and b"2 width" in h.da_last_error()
    assert bwd(out_dtype=split, ld_out=512, rows=0) == 0
    assert fwd(out_dtype=split) == -1                                     # not a forward dtype


def test_map_combine_rejects_bad_arguments() -> None:
    h = lib.get()
    buf = ctypes.c_void_p(1 << 20)   # never dereferenced

    def fwd(**kw):
        args = dict(maps=buf, batch=2, n_maps=4, length=10, width=64, weights=buf, out=buf, out_dtype=lib.DA_BF16,
                    stream=None)
        args.update(kw)
        return h.da_map_combine(*args.values())

    def bwd(**kw):
        args = dict(maps=buf, batch=2, n_maps=4, length=10, width=64, weights=buf, grad=buf, grad_dtype=lib.DA_BF16,
                    grad_maps=buf, weight_sums=buf, stream=None)
        args.update(kw)
        return h.da_map_combine_backward(*args.values())

    assert fwd(out_dtype=lib.DA_F32) == -1 and bwd(grad_dtype=7) == -1
    assert fwd(n_maps=0) == -2 and fwd(n_maps=9) == -2 and b"maps must be in [1, 8]" in h.da_last_error()
    assert bwd(width=12) == -2 and b"multiple of 8" in h.da_last_error()
    assert fwd(maps=None) == -1 and bwd(weights=None) == -1 and b"null" in h.da_last_error()
    assert fwd(out=None) == -1 and bwd(weight_sums=None) == -1
    assert fwd(maps=ctypes.c_void_p((1 << 20) + 8)) == -3
    assert bwd(grad_maps=ctypes.c_void_p((1 << 20) + 4)) == -3 and b"aligned" in h.da_last_error()
    assert fwd(batch=0, out=None) == 0 and bwd(length=0, grad=None) == 0   # nothing to do


def test_sum_partials_rejects_bad_arguments() -> None:
    h = lib.get()
    buf = ctypes.c_void_p(1 << 20)   # never dereferenced

    def call(**kw):
        args = dict(partials=buf, count=4, n=1024, out=buf, out_dtype=lib.DA_BF16, stream=None)
        args.update(kw)
        return h.da_sum_partials(*args.values())

    assert call(out_dtype=lib.DA_F32) == -1
    assert call(count=0) == -2 and call(count=1025) == -2 and call(n=12) == -2
    assert b"multiple of 8" in h.da_last_error()
    assert call(out=None) == -1 and b"null" in h.da_last_error()
    assert call(partials=ctypes.c_void_p((1 << 20) + 4)) == -3
    assert call(n=0, out=None) == 0


def test_layer_norm_backward_rejects_bad_arguments() -> None:
    h = lib.get()
    buf = ctypes.c_void_p(1 << 20)   # never dereferenced

    def call(**kw):
        args = dict(x=buf, grad=buf, rows=10, dim=512, weight=buf, param_dtype=lib.DA_BF16, eps=1e-5,
                    dtype=lib.DA_BF16, grad_x=buf, grad_params=buf, stream=None)
        args.update(kw)
        return h.da_layer_norm_backward(*args.values())

    assert call(dtype=lib.DA_F32) == -1 and call(param_dtype=9) == -1
    assert call(dim=12) == -2 and call(dim=8192) == -2 and b"multiple of 8" in h.da_last_error()
    assert call(grad_params=None) == -1 and b"null" in h.da_last_error()
    assert call(grad=ctypes.c_void_p((1 << 20) + 8)) == -3
    assert call(eps=-1.0) == -1
    assert call(rows=0, x=None) == 0


def test_dense_attention_operands_rejects_bad_arguments() -> None:
    h = lib.get()
    buf = ctypes.c_void_p(1 << 20)   # never dereferenced

    def call(**kw):
        args = dict(query=buf, key=buf, stride_b=100 * 1024, stride_t=1024, map_stride=256, map_repeat=1,
                    qk_dtype=lib.DA_F16, batch=2, maps=2, length=100, score_dim=256, key_t=buf, query_out=buf,
                    key_out=buf, out_dtype=lib.DA_BF16, stream=None)
        args.update(kw)
        return h.da_dense_attention_operands(*args.values())

    assert call(qk_dtype=lib.DA_F32) == -1 and call(out_dtype=9) == -1
    assert call(score_dim=96) == -2 and b"multiple of 64" in h.da_last_error()
    assert call(map_repeat=0) == -1 and call(batch=300, maps=300) == -1
    assert call(key_t=None) == -1 and b"null" in h.da_last_error()
    assert call(stride_t=128) == -3 and call(map_stride=4) == -3
    assert call(key=ctypes.c_void_p((1 << 20) + 8)) == -3
    assert call(length=0, query=None) == 0
