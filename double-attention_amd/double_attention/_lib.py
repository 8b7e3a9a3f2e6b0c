"""ctypes binding of the gfx950 C ABI (``include/double_attention_hip.h``).

The library is built in-tree by ``double-attention_amd/build.py`` into
``double_attention/lib/libdouble_attention_hip.so``.  Loading needs no GPU
(the HIP runtime initializes lazily), so CPU-only machines can still check
that every declared symbol is exported.  ``DOUBLE_ATTENTION_HIP_LIBRARY``
overrides the path, which tests use to simulate a missing library.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libdouble_attention_hip.so"

DA_F32, DA_F16, DA_BF16 = 0, 1, 2
DA_OUT_SPLIT = 0x100

DA_ROUTE_NORMALIZE_INPUT = 1
DA_ROUTE_NORMALIZE_OUTPUT = 2
DA_ROUTE_BETA_IS_LOG = 4
DA_ROUTE_UNIT_KEYS = 8
DA_ROUTE_SILU_LOGITS = 16
DA_ROUTE_STANDARDIZE = 32
DA_ROUTE_DIRECT_SILU = 64
DA_ROUTE_BETA_IS_LOG_SCALE = 128

DA_ATTN_CAUSAL = 1
DA_ATTN_SCALES_ARE_LOG = 2
DA_ATTN_MIX = 4
DA_ATTN_OUT_F32 = 8

DA_SDA_NORMALIZE_INPUT = 1
DA_SDA_NORMALIZE_OUTPUT = 2
DA_SDA_CAUSAL = 4
DA_SDA_CONCAT = 8
DA_SDA_UNIT_KEYS = 16

DA_ACT_NONE = 0
DA_ACT_GELU = 1

ERROR_NAMES = {
    -1: "invalid argument",
    -2: "unsupported",
    -3: "alignment",
    -4: "launch failure",
    -5: "workspace too small",
}

ABI_VERSION = 19
NOALLOC_SCRATCH_BYTES = 128 << 20

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float


class SdaForwardArgs(ctypes.Structure):
    """Mirror of ``da_sda_forward_args``."""

    _fields_ = [
        ("x", _vp),
        ("batch", _i64),
        ("length", _i64),
        ("model_dim", _i64),
        ("qk_branches", _i64),
        ("outer_maps", _i64),
        ("routing_dim", _i64),
        ("atoms", _i64),
        ("wq", _vp),
        ("wk", _vp),
        ("wv", _vp),
        ("bv", _vp),
        ("wo", _vp),
        ("key_t", _vp),
        ("value", _vp),
        ("log_beta", _vp),
        ("log_score_scales", _vp),
        ("map_mix_logits", _vp),
        ("param_dtype", _i32),
        ("dtype", _i32),
        ("eps", _f32),
        ("flags", _i32),
        ("workspace", _vp),
        ("workspace_bytes", _i64),
        ("out", _vp),
        ("raw_key", _vp),
        ("raw_value", _vp),
        ("raw_dtype", _i32),
        ("route_variant", _i32),
        ("silu_gain", _f32),
        ("logit_scale", _f32),
        ("residual", _vp),
    ]


class AttentionBackwardArgs(ctypes.Structure):
    """Mirror of ``da_attention_backward_args``."""

    _fields_ = [
        ("query", _vp),
        ("query_stride_b", _i64),
        ("query_stride_t", _i64),
        ("query_map_stride", _i64),
        ("key", _vp),
        ("key_stride_b", _i64),
        ("key_stride_t", _i64),
        ("key_map_stride", _i64),
        ("map_repeat", _i64),
        ("value", _vp),
        ("value_t", _vp),
        ("value_t_stride_b", _i64),
        ("value_t_dtype", _i32),
        ("out", _vp),
        ("out_dtype", _i32),
        ("grad_out", _vp),
        ("scales", _vp),
        ("scales_dtype", _i32),
        ("scale_mult", _f32),
        ("log_min", _f32),
        ("log_max", _f32),
        ("batch", _i64),
        ("maps", _i64),
        ("length", _i64),
        ("key_length", _i64),
        ("score_dim", _i64),
        ("value_dim", _i64),
        ("flags", _i32),
        ("qk_dtype", _i32),
        ("v_dtype", _i32),
        ("workspace", _vp),
        ("workspace_bytes", _i64),
        ("grad_query", _vp),
        ("grad_key", _vp),
        ("grad_value", _vp),
        ("grad_scales", _vp),
        ("grad_value_sum", _vp),
        ("grad_scores", _vp),
        ("grad_scores_ld", _i64),
    ]


# name -> (restype, argtypes); every function declared in the public header.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "da_abi_version": (_i32, []),
    "da_last_error": (ctypes.c_char_p, []),
    "da_padded_atoms": (_i64, [_i64]),
    "da_padded_length": (_i64, [_i64]),
    "da_dictionary_normalize": (_i32, [_vp, _vp, _i32, _i64, _i64, _f32, _vp, _i32, _vp, _vp, _vp]),
    "da_dictionary_normalize_backward": (
        _i32, [_vp, _vp, _i32, _i64, _i64, _f32, _vp, _vp, _i64, _i64, _vp, _vp, _vp]
    ),
    "da_row_normalize": (_i32, [_vp, _i32, _i64, _i64, _i64, _f32, _vp, _i32, _i64, _vp]),
    "da_row_normalize_backward": (_i32, [_vp, _i32, _i64, _i64, _i64, _f32, _vp, _i32, _i64, _vp, _i32, _i64, _vp]),
    "da_dictionary_route": (
        _i32,
        [
            _vp, _i64, _i64, _i64, _i32,  # x, rows, routing_dim, row pitch, x dtype
            _vp, _i32, _vp, _i64,  # key_t, key dtype, value, atoms
            _vp, _i32, _f32, _f32, _i32,  # beta, beta dtype, beta value, eps, flags
            _f32, _f32,  # silu gain, logit scale
            _vp, _i64, _i32, _vp,  # out, out pitch, out dtype, stream
        ],
    ),
    "da_dictionary_route_backward_rows": (
        _i32,
        [
            _vp, _vp, _i64, _i64, _i64, _i64,  # logits, grad_weights, rows, atoms, causal period, input pitch
            _vp, _i32, _f32, _i64, _i64, _i32,  # beta, beta dtype, beta value, beta count, beta period, flags
            _f32, _f32, _f32,  # silu gain, logit scale, eps
            _vp, _vp, _i64, _i32, _vp, _vp,  # grad_logits, weights, output pitch, out dtype, dbeta rows, stream
        ],
    ),
    "da_attention_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64, _i32]),
    "da_routed_attention": (
        _i32,
        [
            _vp, _vp, _i64, _i64, _i64, _i64, _i64,  # q, k, strides, map stride/repeat, score dim
            _vp, _i64,  # value_t, per-sequence pitch
            _i64, _i64, _i64, _i64,  # batch, maps, length, value_dim
            _vp, _i32, _f32, _vp, _i32,  # scales, mix logits
            _i32, _f32,  # flags, score bound
            _i32, _i32, _vp, _i64, _i64, _i64,  # qk/v dtypes, out + strides
            _vp, _i64, _vp,  # workspace, its bytes, stream
        ],
    ),
    "da_qkv_projection": (
        _i32,
        [_vp, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _i64, _i32, _i32, _vp, _vp, _i64, _i64, _vp],
    ),
    "da_linear": (_i32, [_vp, _i64, _i64, _vp, _i64, _vp, _i32, _i32, _vp, _vp]),
    "da_linear_ex": (_i32, [_vp, _i64, _i64, _vp, _i64, _vp, _i32, _i32, _i32, _vp, _vp, _vp]),
    "da_layer_norm": (_i32, [_vp, _i64, _i64, _vp, _vp, _i32, _f32, _i32, _vp, _vp]),
    "da_layer_norm_backward": (_i32, [_vp, _vp, _i64, _i64, _vp, _i32, _f32, _i32, _vp, _vp, _vp]),
    "da_map_combine": (_i32, [_vp, _i64, _i64, _i64, _i64, _vp, _vp, _i32, _vp]),
    "da_sum_partials": (_i32, [_vp, _i64, _i64, _vp, _i32, _vp]),
    "da_dense_attention_operands": (
        _i32, [_vp, _vp, _i64, _i64, _i64, _i64, _i32, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i32, _vp]),
    "da_map_combine_backward": (_i32, [_vp, _i64, _i64, _i64, _i64, _vp, _vp, _i32, _vp, _vp, _vp]),
    "da_attention_backward_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "da_routed_attention_backward": (
        _i32,
        [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _vp, _i64,
         _vp, _vp, _vp, _vp, _vp],
    ),
    "da_routed_attention_backward_ex": (_i32, [ctypes.POINTER(AttentionBackwardArgs), _vp]),
    "da_sda_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64, _i32, _i32]),
    "da_sda_workspace_offset": (_i64, [_i64, _i64, _i64, _i64, _i32]),
    "da_shared_dictionary_attention_forward": (_i32, [ctypes.POINTER(SdaForwardArgs), _vp]),
    "da_shared_dictionary_attention_forward_noalloc": (_i32, [ctypes.POINTER(SdaForwardArgs), _vp]),
}

_lib: ctypes.CDLL | None = None
_load_error: str | None = None


def library_path() -> Path:
    override = os.environ.get("DOUBLE_ATTENTION_HIP_LIBRARY")
    return Path(override) if override else LIB_PATH


def _load() -> ctypes.CDLL:
    path = library_path()
    if not path.exists():
        raise OSError(
            f"{path} does not exist; build it with `python double-attention_amd/build.py`"
        )
    lib = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError if the symbol is missing
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.da_abi_version()
    if version != ABI_VERSION:
        raise OSError(f"{path} has ABI version {version}, expected {ABI_VERSION}")
    return lib


def get() -> ctypes.CDLL:
    """Return the loaded library or raise ``RuntimeError`` naming the reason."""

    global _lib, _load_error
    if _lib is None and _load_error is None:
        try:
            _lib = _load()
        except (OSError, AttributeError) as exc:
            _load_error = str(exc)
    if _lib is None:
        raise RuntimeError(f"HIP library unavailable: {_load_error}")
    return _lib


def available() -> bool:
    try:
        get()
    except RuntimeError:
        return False
    return True


def unavailable_reason() -> str | None:
    return None if available() else _load_error


def reset() -> None:
    """Forget a cached load result (tests switch the library path)."""

    global _lib, _load_error
    _lib = None
    _load_error = None


def check(rc: int, what: str) -> None:
    if rc == 0:
        return
    message = get().da_last_error().decode(errors="replace")
    kind = ERROR_NAMES.get(rc, f"error {rc}")
    if rc in (-1, -3, -5):
        raise ValueError(f"{what}: {kind}: {message}")
    if rc == -2:
        raise NotImplementedError(f"{what}: {kind}: {message}")
    raise RuntimeError(f"{what}: {kind}: {message}")
