"""PyTorch-facing wrappers of the gfx950 kernels.

Operator-level entry points mirror the reference's Triton functions so that
code and tests written against those read the same:

* ``dictionary_route_hip``   <- ``dictionary_route_triton`` (reference
  ``src/double_attention/triton_kernels.py:1984-2019``)
* ``routed_attention_hip``   <- ``routed_attention_triton`` (``triton_kernels.py:2290-2305``)
* ``dictionary_normalize_hip`` <- ``SharedDictionaryBank.normalized`` (``modules.py:45-48``)

``shared_dictionary_attention_hip`` runs a whole ``SharedDictionaryAttention``
forward (``modules.py:190-291``) in one C call: projection GEMM, route, flash
attention with the fused map mix, output GEMM.

PyTorch only supplies device memory and the current stream.  Every buffer,
including the workspace, is allocated here with the caching allocator and
handed to the library as a raw pointer; kernels run on
``torch.cuda.current_stream()``.  Nothing here falls back to another
implementation: an unsupported shape or variant raises.

Autograd: the route and the outer attention have native backwards
(``route_gradients``, ``attention_gradients``): the attention backward
kernels, or library GEMMs around the row kernel of the assignment's
backward.  Shapes neither covers (more than 4096 atoms, a row kernel width
it lacks) recompute the PyTorch reference composition (``ops.py``) on the
same device under autograd.
"""

from __future__ import annotations

import ctypes
import math

from typing import NamedTuple

import torch
from torch import Tensor

from . import _lib
from .ops import dictionary_route_reference, routed_attention_reference

_DTYPE_CODES = {torch.float32: _lib.DA_F32, torch.float16: _lib.DA_F16, torch.bfloat16: _lib.DA_BF16}
SUPPORTED_WIDTHS = (64, 128, 256, 512)
# The attention forward's value (model) widths: multiples of 64 up to 4096
# (its value slices are 64, 128 or 256 features wide).
VALUE_WIDTH_STEP = 64
MAX_VALUE_WIDTH = 4096
ATOM_PAD = 64
TOKEN_PAD = 64
# Clamp windows of the learned logs: beta = exp(clamp(log_beta, ln 0.05,
# ln 64)) (reference modules.py:130-132) and the outer-map temperatures
# exp(clamp(log_scale, ln 1/4, ln 1024)) (ops.py:160-161).
LOG_BETA_RANGE = (math.log(0.05), math.log(64.0))
LOG_SCALE_RANGE = (math.log(0.25), math.log(1024.0))


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError as exc:
        raise ValueError(f"unsupported dtype {dtype}") from exc


def _half_code(dtype: torch.dtype) -> int:
    if dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"HIP kernels require fp16 or bf16 tensors, got {dtype}")
    return _DTYPE_CODES[dtype]


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device) -> int:
    """The device's current stream as a raw ``hipStream_t`` (the one
    ``torch.cuda.current_stream(device)`` wraps, without building the wrapper
    object: this runs once per kernel call)."""

    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def _require_cuda(*tensors: Tensor) -> None:
    for t in tensors:
        if not t.is_cuda:
            raise ValueError("HIP kernels require tensors on a ROCm device")


def _aligned(t: Tensor) -> Tensor:
    """``t`` contiguous at a 16-byte aligned address (views at odd offsets
    are copied): the kernels load and store 16-byte chunks."""

    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _round_up(v: int, m: int) -> int:
    return (v + m - 1) // m * m


def _ptr(t: Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# --------------------------------------------------------------------------
# Dictionary normalization and route layouts
# --------------------------------------------------------------------------


class RouteDictionary(NamedTuple):
    """A normalized bank in the layouts the route kernel reads.

    ``key_t`` is ``[Mp, R]`` (atom-major) in the key dtype; ``value`` is
    ``[Mp / 32, R, 32]`` in fp16, i.e. 32-atom tiles with coordinate ``r`` of
    atom ``j`` at ``value[j // 32, r, j % 32]``.  Atoms past ``atoms`` are zero
    and ``Mp`` is ``atoms`` rounded up to a multiple of 64.  Normalized atoms
    are bounded by one, so fp16 holds them with eight times finer rounding than
    bf16.
    """

    key_t: Tensor
    value: Tensor
    atoms: int
    unit: bool = False   # key atoms have L2 norm <= 1 (a normalized bank)


def _version_of(t: Tensor) -> int | None:
    # Inference tensors keep no version counter.
    return None if t.is_inference() else t._version


def _tag(key: Tensor, value: Tensor, layout: RouteDictionary) -> tuple[Tensor, Tensor]:
    """Attach ``layout`` to the ``[R, M]`` pair it was built from, with the
    pair's version counters: an in-place change of either (an optimizer
    step) makes the layout stale, and ``_tagged_layout`` then ignores it."""

    versions = (_version_of(key), _version_of(value))
    for t in (key, value):
        t._da_route_layout = layout  # type: ignore[attr-defined]
        t._da_route_versions = versions  # type: ignore[attr-defined]
    return key, value


def _tagged_layout(key: Tensor, value: Tensor) -> RouteDictionary | None:
    """The route layout attached to this key/value pair, if still current."""

    layout = getattr(key, "_da_route_layout", None)
    if layout is None or getattr(value, "_da_route_layout", None) is not layout:
        return None
    if getattr(key, "_da_route_versions", None) != (_version_of(key), _version_of(value)):
        return None
    return layout


def route_key_dtype(normalize_input: bool, dtype: torch.dtype) -> torch.dtype:
    """Key-atom dtype the route uses: fp16 for unit (normalized) inputs, else the input dtype."""

    return torch.float16 if normalize_input else dtype


def dictionary_normalize_hip(
    raw_key: Tensor,
    raw_value: Tensor | None,
    eps: float = 1e-6,
    key_dtype: torch.dtype = torch.float16,
) -> tuple[Tensor, Tensor]:
    """Column-normalize a bank in one launch; returns ``(key, value)`` as ``[R, M]``.

    Matches ``F.normalize(raw, dim=0, eps=eps)``.  ``key`` (in ``key_dtype``)
    is a view of the route's atom-major key layout and ``value`` (fp16) a view
    of a coordinate-major copy the same kernel writes beside the route's tiled
    value layout; both carry the layouts, so handing them back to the route
    re-lays nothing out.  For a tied bank both hold the same normalized atoms.
    """

    if raw_key.ndim != 2:
        raise ValueError("raw_key must be [routing_dim, atoms]")
    if raw_value is not None and raw_value.shape != raw_key.shape:
        raise ValueError("raw_value must match raw_key")
    _require_cuda(raw_key, *(() if raw_value is None else (raw_value,)))
    routing_dim, atoms = raw_key.shape
    if routing_dim not in SUPPORTED_WIDTHS:
        raise NotImplementedError(f"HIP route supports routing_dim in {SUPPORTED_WIDTHS}, got {routing_dim}")
    padded = _round_up(atoms, ATOM_PAD)
    key_t = torch.empty(padded, routing_dim, dtype=key_dtype, device=raw_key.device)
    value = torch.empty(padded // 32, routing_dim, 32, dtype=torch.float16, device=raw_key.device)
    value_rows = torch.empty(routing_dim, padded, dtype=torch.float16, device=raw_key.device)
    raw_key_c = raw_key.detach().contiguous()
    raw_value_c = None if raw_value is None else raw_value.detach().to(raw_key.dtype).contiguous()
    lib = _lib.get()
    _lib.check(
        lib.da_dictionary_normalize(
            raw_key_c.data_ptr(),
            _ptr(raw_value_c),
            dtype_code(raw_key_c.dtype),
            routing_dim,
            atoms,
            float(eps),
            key_t.data_ptr(),
            _half_code(key_dtype),
            value.data_ptr(),
            value_rows.data_ptr(),
            _stream(raw_key.device),
        ),
        "dictionary_normalize_hip",
    )
    layout = RouteDictionary(key_t, value, atoms, True)
    return _tag(key_t[:atoms].t(), value_rows[:, :atoms], layout)


def dictionary_normalize_backward_hip(
    raw_key: Tensor,
    raw_value: Tensor | None,
    grad_key: Tensor | None,
    grad_value: Tensor | None,
    eps: float = 1e-6,
) -> tuple[Tensor, Tensor | None]:
    """Gradients at the raw bank of ``SharedDictionaryBank.normalized``
    (``modules.py:45-48`` under autograd) in one launch.

    ``grad_key`` / ``grad_value`` are the gradients at the normalized key and
    value atoms (``[R, M]``; None = zero); a tied bank (``raw_value`` None)
    takes both into its key atoms.  Returns ``(d_raw_key, d_raw_value)`` in
    the raw dtype (``d_raw_value`` None for a tied bank).
    """

    if raw_key.ndim != 2:
        raise ValueError("raw_key must be [routing_dim, atoms]")
    if raw_value is not None and raw_value.shape != raw_key.shape:
        raise ValueError("raw_value must match raw_key")
    _require_cuda(raw_key)
    routing_dim, atoms = raw_key.shape
    device = raw_key.device
    if grad_key is None:
        grad_key = torch.zeros(routing_dim, atoms, dtype=torch.float32, device=device)

    def as_grad(g: Tensor | None) -> Tensor | None:
        if g is None:
            return None
        if g.shape != raw_key.shape:
            raise ValueError("bank gradients must be [routing_dim, atoms]")
        g = g.detach().to(torch.float32)
        # [R, M] rows, or the transposed view of atom-major [M, R] rows (the
        # route backward's), are read in place.
        if g.stride() not in ((atoms, 1), (1, routing_dim)) or g.data_ptr() % 4:
            g = g.contiguous()
        return g

    key_c = raw_key.detach().contiguous()
    value_c = None if raw_value is None else raw_value.detach().to(key_c.dtype).contiguous()
    gk, gv = as_grad(grad_key), as_grad(grad_value)
    if gv is not None and gv.stride() != gk.stride():
        gk, gv = gk.contiguous(), gv.contiguous()
    d_key = torch.empty_like(key_c)
    d_value = None if value_c is None else torch.empty_like(value_c)
    lib = _lib.get()
    _lib.check(
        lib.da_dictionary_normalize_backward(
            key_c.data_ptr(), _ptr(value_c), dtype_code(key_c.dtype), routing_dim, atoms, float(eps),
            gk.data_ptr(), _ptr(gv), gk.stride(0), gk.stride(1), d_key.data_ptr(), _ptr(d_value), _stream(device),
        ),
        "dictionary_normalize_hip backward",
    )
    return d_key, d_value


def _untile_value(value: Tensor) -> Tensor:
    """``[Mp / 32, R, 32]`` value tiles -> ``[R, Mp]``."""

    return value.permute(1, 0, 2).reshape(value.shape[1], -1)


def route_layout(dictionary_key: Tensor, dictionary_value: Tensor, key_dtype: torch.dtype) -> RouteDictionary:
    """Route layouts for a normalized ``[R, M]`` key/value pair.

    Copy-free when the pair carries current layouts (a bank normalized into
    them, or a pair laid out before and unchanged since): the blocks of a
    stack that share one normalized bank lay it out once per forward.
    """

    layout = _tagged_layout(dictionary_key, dictionary_value)
    if layout is not None and layout.key_t.dtype == key_dtype:
        return layout
    if dictionary_key.ndim != 2 or dictionary_value.shape != dictionary_key.shape:
        raise ValueError("dictionary key and value must both be [routing_dim, atoms]")
    routing_dim, atoms = dictionary_key.shape
    padded = _round_up(atoms, ATOM_PAD)
    key_t = torch.zeros(padded, routing_dim, dtype=key_dtype, device=dictionary_key.device)
    value = torch.zeros(routing_dim, padded, dtype=torch.float16, device=dictionary_key.device)
    key_t[:atoms].copy_(dictionary_key.detach().t())
    value[:, :atoms].copy_(dictionary_value.detach())
    tiles = value.view(routing_dim, padded // 32, 32).permute(1, 0, 2).contiguous()
    layout = RouteDictionary(key_t, tiles, atoms)
    # Parameters are left untagged (writes through .data, which the version
    # counter does not see, would leave their layout stale), and so are
    # inference tensors, which keep no version counter.
    if not any((t.is_leaf and t.requires_grad) or t.is_inference() for t in (dictionary_key, dictionary_value)):
        _tag(dictionary_key, dictionary_value, layout)
    return layout


# --------------------------------------------------------------------------
# Route
# --------------------------------------------------------------------------


class RouteVariant(NamedTuple):
    """Activation, standardization and assignment of ``ops.py:41-59``."""

    silu_logits: bool = False
    direct_silu: bool = False
    silu_gain: float = 1.0
    standardize_logits: bool = False
    standardized_logit_scale: float | None = None

    def flags(self) -> int:
        return (
            (_lib.DA_ROUTE_SILU_LOGITS if self.silu_logits else 0)
            | (_lib.DA_ROUTE_STANDARDIZE if self.standardize_logits else 0)
            | (_lib.DA_ROUTE_DIRECT_SILU if self.direct_silu else 0)
        )

    def logit_scale(self, routing_dim: int) -> float:
        """``standardized_logit_scale``, or ``routing_dim ** -0.5`` (ops.py:50-54)."""

        if self.standardized_logit_scale is None:
            return routing_dim ** -0.5
        return float(self.standardized_logit_scale)

    @classmethod
    def of_config(cls, config) -> "RouteVariant":
        return cls(
            silu_logits=config.dictionary_activation == "silu",
            direct_silu=config.dictionary_assignment == "silu",
            silu_gain=float(config.dictionary_silu_gain),
            standardize_logits=bool(config.standardize_dictionary_logits),
            standardized_logit_scale=config.standardized_logit_scale,
        )


def _route_forward(
    x: Tensor,
    layout: RouteDictionary,
    beta: Tensor | float,
    eps: float,
    normalize_input: bool,
    normalize_output: bool,
    variant: RouteVariant = RouteVariant(),
    out_dtype: torch.dtype | None = None,
    beta_is_log: bool = False,
) -> Tensor:
    """Route launch; ``beta_is_log``: ``beta`` is a log-beta tensor and the
    kernel applies exp(clamp(., ln 0.05, ln 64))."""

    routing_dim = x.shape[-1]
    out_dtype = x.dtype if out_dtype is None else out_dtype
    if routing_dim != layout.key_t.shape[1]:
        raise ValueError("input width does not match the dictionary routing_dim")
    if routing_dim not in SUPPORTED_WIDTHS:
        raise NotImplementedError(f"HIP route supports routing_dim in {SUPPORTED_WIDTHS}, got {routing_dim}")
    rows_view = x.reshape(-1, routing_dim)
    if rows_view.shape[0] == 0:
        return torch.empty(x.shape, dtype=out_dtype, device=x.device)
    if rows_view.stride(-1) != 1 or rows_view.stride(0) % 8 or rows_view.data_ptr() % 16:
        rows_view = _aligned(rows_view)
    out = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    flags = (
        (_lib.DA_ROUTE_NORMALIZE_INPUT if normalize_input else 0)
        | (_lib.DA_ROUTE_NORMALIZE_OUTPUT if normalize_output else 0)
        | (_lib.DA_ROUTE_UNIT_KEYS if layout.unit else 0)
        | variant.flags()
    )
    if beta_is_log:
        if not isinstance(beta, Tensor):
            raise ValueError("a log beta must be a tensor")
        flags |= _lib.DA_ROUTE_BETA_IS_LOG
    if isinstance(beta, Tensor):
        if beta.numel() != 1:
            raise ValueError("beta must be a scalar")
        _require_cuda(beta)
        beta_c = beta.detach().contiguous()
        beta_ptr, beta_code, beta_value = beta_c.data_ptr(), dtype_code(beta_c.dtype), 0.0
    else:
        beta_c = None
        beta_ptr, beta_code, beta_value = None, _lib.DA_F32, float(beta)
    lib = _lib.get()
    _lib.check(
        lib.da_dictionary_route(
            rows_view.data_ptr(),
            rows_view.shape[0],
            routing_dim,
            rows_view.stride(0),
            _half_code(x.dtype),
            layout.key_t.data_ptr(),
            _half_code(layout.key_t.dtype),
            layout.value.data_ptr(),
            layout.atoms,
            beta_ptr,
            beta_code,
            beta_value,
            float(eps),
            flags,
            float(variant.silu_gain),
            float(variant.logit_scale(routing_dim)),
            out.data_ptr(),
            routing_dim,
            _half_code(out_dtype),
            _stream(x.device),
        ),
        "dictionary_route_hip",
    )
    del beta_c
    return out


# Routing widths whose route backward runs on the attention backward kernels.
# Up to 256 they take about the time of the GEMM path and keep fp32
# accumulation throughout; at 512-wide rows the two-workgroup split recomputes
# S and dP per half, and the GEMM path around the row kernel is faster.  So
# is it for banks above 1024 atoms (ms, plain softmax, both norms, against the
# attention kernels: 16384 rows R 256 M 1536: 0.447 / 0.595; at M 512 the
# attention kernels take 0.19-0.28 against 0.28-0.29 for 8192-32768 rows).
ROUTE_BACKWARD_WIDTHS = (64, 128, 256)
ROUTE_BACKWARD_MAX_ATOMS = 1024


def _route_backward_supported(x: Tensor, dictionary_key: Tensor, variant: RouteVariant) -> bool:
    return (
        variant.flags() == 0
        and x.is_cuda
        and x.dtype in (torch.float16, torch.bfloat16)
        and x.shape[-1] in ROUTE_BACKWARD_WIDTHS
        and 1 <= dictionary_key.shape[1] <= ROUTE_BACKWARD_MAX_ATOMS
    )


def _row_normalize(rows: Tensor, eps: float, dtype: torch.dtype) -> Tensor:
    """``F.normalize(rows, dim=-1, eps)`` of ``[n, R]`` rows (``ops.py:39, 62``):
    fp32 arithmetic, one rounding to ``dtype`` (``da_row_normalize``)."""

    rows = _aligned(rows)
    n, width = rows.shape
    out = torch.empty(n, width, dtype=dtype, device=rows.device)
    lib = _lib.get()
    _lib.check(
        lib.da_row_normalize(
            rows.data_ptr(), dtype_code(rows.dtype), n, width, width, float(eps), out.data_ptr(), dtype_code(dtype),
            width, _stream(rows.device),
        ),
        "row normalize",
    )
    return out


def _normalize_backward(v: Tensor, h: Tensor, eps: float, dtype: torch.dtype, split: bool = False) -> Tensor:
    """The backward of N(v) = v / max(|v|, eps) (``F.normalize``) at gradient h.

    (h - n <n, h>) / |v| with n = v / |v| where |v| > eps, h / eps elsewhere,
    for ``[n, R]`` rows v and h: one pass of ``da_row_normalize_backward``,
    fp32 arithmetic, one rounding to ``dtype``.  With ``split`` (16-bit
    ``dtype``) the result is ``[n, 2R]``: the rounded gradient, then its
    rounding residual (rounded), side by side.
    """

    v = _aligned(v)
    h = _aligned(h)
    n, width = v.shape
    cols = 2 * width if split else width
    out = torch.empty(n, cols, dtype=dtype, device=v.device)
    lib = _lib.get()
    _lib.check(
        lib.da_row_normalize_backward(
            v.data_ptr(), dtype_code(v.dtype), n, width, width, float(eps), h.data_ptr(), dtype_code(h.dtype), width,
            out.data_ptr(), dtype_code(dtype) | (_lib.DA_OUT_SPLIT if split else 0), cols, _stream(v.device),
        ),
        "row normalize backward",
    )
    return out


def _attention_backward_ex(
    query: tuple[int, int, int, int],
    key: tuple[int, int, int, int],
    map_repeat: int,
    value: Tensor | tuple[Tensor, int, torch.dtype],
    out: Tensor,
    grad_out: Tensor,
    scales: Tensor,
    scale_mult: float,
    log_range: tuple[float, float] | None,
    shape: tuple[int, int, int, int, int, int],
    causal: bool,
    qk_dtype: torch.dtype,
    grad_query: int,
    grad_key: int,
    grad_value: Tensor,
    grad_scales: Tensor,
    what: str,
    grad_value_sum: Tensor | None = None,
    grad_scores: Tensor | None = None,
) -> None:
    """One ``da_routed_attention_backward_ex`` call.

    ``query`` / ``key`` are (data pointer, stride_b, stride_t, map_stride) in
    elements; ``grad_query`` / ``grad_key`` point at fp32 buffers with the
    same strides.  ``value`` is the value rows, or (V^T tiles, their
    per-sequence stride, the dtype the kernels take them in).  ``shape`` is
    (batch, maps, length, key_length, score_dim, value_dim).  ``log_range``
    set: ``scales`` holds logs clamped to it, and ``grad_scales`` receives the
    gradient at the logs.  ``grad_scores`` (a 2-D view of rows, score dtype):
    the kernels write scale * dS there instead of the query gradient.
    """

    batch, maps, length, key_length, score_dim, value_dim = shape
    lib = _lib.get()
    ws_bytes = lib.da_attention_backward_workspace_bytes(batch, maps, length, key_length, score_dim, value_dim)
    device = out.device
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    args = _lib.AttentionBackwardArgs()
    args.query, args.query_stride_b, args.query_stride_t, args.query_map_stride = query
    args.key, args.key_stride_b, args.key_stride_t, args.key_map_stride = key
    args.map_repeat = map_repeat
    if isinstance(value, Tensor):
        args.value = value.data_ptr()
        v_dtype = value.dtype
    else:
        tiles, args.value_t_stride_b, v_dtype = value
        args.value_t = tiles.data_ptr()
        args.value_t_dtype = _half_code(tiles.dtype)
    args.out = out.data_ptr()
    args.out_dtype = dtype_code(out.dtype)
    args.grad_out = grad_out.data_ptr()
    args.scales = scales.data_ptr()
    args.scales_dtype = dtype_code(scales.dtype)
    args.scale_mult = scale_mult
    args.log_min, args.log_max = log_range if log_range is not None else (0.0, 0.0)
    args.batch, args.maps, args.length, args.key_length = batch, maps, length, key_length
    args.score_dim, args.value_dim = score_dim, value_dim
    args.flags = (_lib.DA_ATTN_CAUSAL if causal else 0) | (_lib.DA_ATTN_SCALES_ARE_LOG if log_range is not None else 0)
    args.qk_dtype = _half_code(qk_dtype)
    args.v_dtype = _half_code(v_dtype)
    args.workspace = workspace.data_ptr()
    args.workspace_bytes = ws_bytes
    args.grad_query = grad_query
    args.grad_key = grad_key
    args.grad_value = grad_value.data_ptr()
    args.grad_scales = grad_scales.data_ptr()
    args.grad_value_sum = _ptr(grad_value_sum)
    if grad_scores is not None:
        args.grad_scores = grad_scores.data_ptr()
        args.grad_scores_ld = grad_scores.stride(0)
    _lib.check(lib.da_routed_attention_backward_ex(ctypes.byref(args), _stream(device)), what)


def _route_backward(
    x: Tensor,
    dictionary_key: Tensor,
    dictionary_value: Tensor,
    beta: Tensor | float,
    eps: float,
    normalize_input: bool,
    normalize_output: bool,
    grad: Tensor,
    r: Tensor | None = None,
    bank_grad_dtype: torch.dtype | None = None,
    beta_is_log: bool = False,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Gradients of the softmax route (``ops.py:16-62``) on the attention backward kernels.

    The route is one attention per row: the (normalized) row u is the query,
    the key atoms the keys, the value atoms the values, beta the score scale
    and r = softmax(beta u Dk) Dv^T the output, then z = r / max(|r|, eps).
    The host forms u, r (the forward's, or one route launch without the
    output norm) and the output-norm backward dr; ``da_routed_attention_backward_ex``
    with the atoms as a key sequence of their own returns du, dDk, dDv and
    dbeta; the input-norm backward gives dx.  Returns fp32-accumulated
    gradients in the dtypes of ``x`` and the dictionary tensors (or
    ``bank_grad_dtype`` for the two bank gradients).  ``beta_is_log``: ``beta``
    is log-beta, clamped in the kernels, and the last gradient is at the log.
    """

    routing_dim = x.shape[-1]
    atoms = dictionary_key.shape[1]
    device = x.device
    rows = _aligned(x.detach().reshape(-1, routing_dim))
    n = rows.shape[0]
    # The forward kernel's operands: unit rows rounded once to fp16 with fp16
    # keys; raw 16-bit rows in their own dtype with keys in that dtype (the
    # backward kernels recompute P from the same values the forward used).
    if normalize_input:
        qk_type = torch.float16
        u16 = _row_normalize(rows, eps, qk_type)
    else:
        qk_type = x.dtype if x.dtype in (torch.float16, torch.bfloat16) else torch.float16
        u16 = _aligned(rows.to(qk_type))
    beta_t = beta.detach().reshape(1) if isinstance(beta, Tensor) else torch.full((1,), float(beta), device=device)
    if r is None:
        layout16 = route_layout(dictionary_key.detach(), dictionary_value.detach(), qk_type)
        r = _route_forward(u16, layout16, beta_t, eps, False, False, RouteVariant(), beta_is_log=beta_is_log)
    r = r.reshape(-1, routing_dim)
    g = grad.detach().reshape(-1, routing_dim)
    # Values, r and dr in fp16 for fp16 inputs (8x finer than bf16: with the
    # output norm, rowsum(dr . r) is analytically zero and its rounding noise
    # reaches every atom's gradient), bf16 for bf16 inputs.
    v_type = torch.float16 if x.dtype == torch.float16 else torch.bfloat16
    if normalize_output:
        go = _normalize_backward(r, g, eps, v_type)
    else:
        go = _aligned(g.to(v_type))
    # The keys as the route layout's atom-major rows and the values as its
    # 32-atom tiles when the bank carries them (the prep kernel turns the
    # tiles into v_type rows), else laid out here; r in its own dtype (it only
    # enters rowsum(dr . r)).
    layout = _tagged_layout(dictionary_key, dictionary_value)
    if layout is not None and layout.atoms == atoms and layout.key_t.dtype == qk_type:
        keys = layout.key_t[:atoms]
    else:
        keys = _aligned(dictionary_key.detach().t().to(qk_type))
    if layout is not None and layout.atoms == atoms:
        values: Tensor | tuple[Tensor, int, torch.dtype] = (layout.value, 0, v_type)
    else:
        values = _aligned(dictionary_value.detach().t().to(v_type))
    out = _aligned(r)
    dkt = torch.empty(atoms, routing_dim, dtype=torch.float32, device=device)
    dvt = torch.empty(atoms, routing_dim, dtype=torch.float32, device=device)
    dbeta = torch.empty(1, dtype=torch.float32, device=device)
    # Every row meets every atom: the kernels write beta dS (the gradient at
    # the logits, rounded once) and one GEMM forms du = beta dS Dk, instead
    # of one fp32 atomic add per row element and 64-atom tile -- while the
    # [rows, atoms] score gradients stay within ROUTE_SCORES_MAX_BYTES.
    padded = _round_up(atoms, ATOM_PAD)
    use_scores = n * padded * 2 <= ROUTE_SCORES_MAX_BYTES
    scores = torch.empty(n, padded, dtype=qk_type, device=device) if use_scores else None
    du = None if use_scores else torch.empty(n, routing_dim, dtype=torch.float32, device=device)
    _attention_backward_ex(
        (u16.data_ptr(), n * routing_dim, routing_dim, 0), (keys.data_ptr(), atoms * routing_dim, routing_dim, 0), 1,
        values, out, go, beta_t, 1.0, LOG_BETA_RANGE if beta_is_log else None,
        (1, 1, n, atoms, routing_dim, routing_dim), False, qk_type,
        0 if use_scores else du.data_ptr(), dkt.data_ptr(), dvt, dbeta, "dictionary_route_hip backward",
        grad_scores=scores,
    )
    if use_scores:
        du = _mm_f32(scores[:, :atoms], keys)
    dx = _normalize_backward(rows, du, eps, x.dtype) if normalize_input else du.to(x.dtype)
    return (
        dx.reshape(x.shape),
        dkt.t().to(bank_grad_dtype or dictionary_key.dtype),
        dvt.t().to(bank_grad_dtype or dictionary_value.dtype),
        dbeta,
    )


# Largest [rows, atoms] buffer of score gradients the route backward uses in
# place of the query-gradient atomics (beyond it, the atomics).
ROUTE_SCORES_MAX_BYTES = 512 << 20


# The row kernel holds rows of up to 4096 atoms in VGPRs and takes longer
# rows in passes over the row; the bound is the C ABI's.
ROUTE_BACKWARD_ROWS_MAX_ATOMS = 1 << 24


def route_backward_is_native(routing_dim: int, atoms: int, dtype: torch.dtype, variant: RouteVariant) -> bool:
    """Whether ``route_gradients`` takes rows of this width and dtype (on a
    ROCm device) and a bank of this size on a native path."""

    if dtype not in (torch.float16, torch.bfloat16) or atoms < 1:
        return False
    if variant.flags() == 0 and routing_dim in ROUTE_BACKWARD_WIDTHS:
        return True
    return routing_dim in SUPPORTED_WIDTHS and atoms <= ROUTE_BACKWARD_ROWS_MAX_ATOMS


def _route_backward_rows_supported(x: Tensor, dictionary_key: Tensor) -> bool:
    return (
        x.is_cuda
        and x.dtype in (torch.float16, torch.bfloat16)
        and x.shape[-1] in SUPPORTED_WIDTHS
        and 1 <= dictionary_key.shape[1] <= ROUTE_BACKWARD_ROWS_MAX_ATOMS
    )


def _mm_f32(a: Tensor, b: Tensor) -> Tensor:
    """``a @ b`` of 16-bit operands with fp32 accumulation and an fp32 result
    (a library GEMM; no 16-bit rounding of the product)."""

    return torch.mm(a, b, out_dtype=torch.float32)


# Split-K for the weight-gradient products: chunks of at least this many
# rows of K, at most this many chunks.
SPLIT_K_MIN_CHUNK = 1024
SPLIT_K_MAX = 8


def _mm_tn_f32(a: Tensor, b: Tensor, out_dtype: torch.dtype = torch.float32) -> Tensor:
    """``a^T b`` for row-major ``a [K, M]`` and ``b [K, N]`` (16-bit, unit
    column stride), accumulated in fp32 and rounded once to ``out_dtype``.

    The weight gradients have a long K (tokens or rows) over a small output:
    one library GEMM runs a few dozen output tiles on 256 CUs.  K is cut into
    s chunks whose partial products run as one batched GEMM (fp32 partials,
    summed in fp32, then rounded; a reduction into a 16-bit output would
    round the partials first): up to 2.3x faster at [16384 x 512]^T
    [16384 x 1536].
    """

    k, m = a.shape
    n = b.shape[1]
    if a.stride(1) != 1:
        a = a.contiguous()
    if b.stride(1) != 1:
        b = b.contiguous()
    tiles = -(-m // 128) * -(-n // 128)
    s = 1
    while s < SPLIT_K_MAX and k % (2 * s) == 0 and k // (2 * s) >= SPLIT_K_MIN_CHUNK and tiles * s < 512:
        s *= 2
    if s == 1:
        # The library accumulates in fp32 and rounds once to its output dtype
        # (the operands' dtype; another 16-bit dtype is rounded from fp32).
        return torch.mm(a.t(), b) if out_dtype == a.dtype else _mm_f32(a.t(), b).to(out_dtype)
    chunk = k // s
    # Left operand: the transposed chunks of a (column-major views); right
    # operand: row-major chunks of b.
    a3 = a.as_strided((s, m, chunk), (chunk * a.stride(0), 1, a.stride(0)))
    b3 = b.as_strided((s, chunk, n), (chunk * b.stride(0), b.stride(0), 1))
    partials = torch.bmm(a3, b3, out_dtype=torch.float32)
    if out_dtype in (torch.float16, torch.bfloat16) and (m * n) % 8 == 0 and partials.is_cuda:
        # The fp32 sum and the one rounding in one launch.
        out = torch.empty(m, n, dtype=out_dtype, device=partials.device)
        _lib.check(
            _lib.get().da_sum_partials(partials.data_ptr(), s, m * n, out.data_ptr(), _half_code(out_dtype),
                                       _stream(partials.device)),
            "sum partials",
        )
        return out
    return partials.sum(0).to(out_dtype)


_ONES: dict[tuple[torch.device, int, torch.dtype], Tensor] = {}


def column_sums(x: Tensor, out_dtype: torch.dtype) -> Tensor:
    """Column sums of a 16-bit ``[K, N]`` matrix (a bias gradient): one
    library product with a ones row, fp32 accumulation, one rounding to
    ``out_dtype``."""

    key = (x.device, x.shape[0], x.dtype)
    ones = _ONES.get(key)
    if ones is None:
        ones = _ONES[key] = torch.ones(1, x.shape[0], dtype=x.dtype, device=x.device)
    if out_dtype == x.dtype:
        return torch.mm(ones, x).view(-1)
    return _mm_f32(ones, x).view(-1).to(out_dtype)


def _route_backward_rows(
    x: Tensor,
    dictionary_key: Tensor,
    dictionary_value: Tensor,
    beta: Tensor | float,
    eps: float,
    normalize_input: bool,
    normalize_output: bool,
    grad: Tensor,
    variant: RouteVariant,
    r: Tensor | None = None,
    bank_grad_dtype: torch.dtype | None = None,
    beta_is_log: bool = False,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Gradients of the route (``ops.py:16-62``) for every variant and width.

    The structure of the reference's large-shape backward
    (``triton_kernels.py:1929-1973``): two GEMMs give each row's raw logits
    l = N_in(x) Dk and dW = dr Dv (fp32 results), ``da_dictionary_route_backward_rows``
    turns them into the gradient at the logits and the assignment weights,
    and three GEMMs give dN_in(x), dDk and dDv.  The logits use the forward
    kernel's operands (unit rows rounded once to fp16 with fp16 keys; raw rows
    in their own dtype); r, the reconstruction before the output norm, is the
    forward's (``r``) or comes from one route launch.  Returns gradients in
    the dtypes of ``x`` and the dictionary tensors (or ``bank_grad_dtype`` for
    the two bank gradients), and d beta as a 1-element fp32 tensor (at the
    log with ``beta_is_log``: ``beta`` is then log-beta, clamped in the kernels).
    """

    routing_dim = x.shape[-1]
    atoms = dictionary_key.shape[1]
    device = x.device
    rows = _aligned(x.detach().reshape(-1, routing_dim))
    n = rows.shape[0]
    # 16-bit operands of the GEMMs: fp16 for fp16 inputs, bf16 for bf16 ones.
    v_type = torch.float16 if x.dtype == torch.float16 else torch.bfloat16
    if normalize_input:
        key_type = torch.float16
        u_h = _row_normalize(rows, eps, key_type)
        u_v = u_h if v_type == key_type else _row_normalize(rows, eps, v_type)
    else:
        key_type = x.dtype
        u_h = u_v = rows
    beta_t = beta.detach().reshape(1) if isinstance(beta, Tensor) else torch.full((1,), float(beta), device=device)
    if r is None:
        layout = route_layout(dictionary_key.detach(), dictionary_value.detach(), key_type)
        r = _route_forward(u_h, layout, beta_t, eps, False, False, variant, beta_is_log=beta_is_log)
    r = r.reshape(-1, routing_dim)
    g = grad.detach().reshape(-1, routing_dim)
    # dW = dr Dv takes dr as a 16-bit head and its rounding residual ([n, 2R]
    # against [Dv; Dv]): the softmax backward differences dW_j - sum_k w_k dW_k,
    # so one 16-bit rounding of dr would reach every atom's gradient.
    # The row-norm backward writes the pair in one pass; a 16-bit gradient of
    # the value dtype is its own head (no residual).
    keys_h = dictionary_key.detach().to(key_type)
    logits = _mm_f32(u_h, keys_h)
    values_v = dictionary_value.detach().to(v_type)
    if normalize_output:
        dr2 = _normalize_backward(r, g, eps, v_type, split=True)
        dr_v = dr2[:, :routing_dim]
        grad_weights = _mm_f32(dr2, torch.cat((values_v, values_v)))
    elif g.dtype == v_type:
        dr_v = _aligned(g)
        grad_weights = _mm_f32(dr_v, values_v)
    else:
        dr = g.float()
        dr2 = torch.empty(n, 2 * routing_dim, dtype=v_type, device=device)
        dr_v = dr2[:, :routing_dim]
        dr_v.copy_(dr)
        torch.sub(dr, dr_v, out=dr2[:, routing_dim:])
        del dr
        grad_weights = _mm_f32(dr2, torch.cat((values_v, values_v)))
    grad_logits = torch.empty(n, atoms, dtype=v_type, device=device)
    weights = torch.empty(n, atoms, dtype=v_type, device=device)
    dbeta_rows = torch.empty(n, dtype=torch.float32, device=device)
    lib = _lib.get()
    _lib.check(
        lib.da_dictionary_route_backward_rows(
            logits.data_ptr(), grad_weights.data_ptr(), n, atoms, 0, atoms,
            beta_t.data_ptr(), dtype_code(beta_t.dtype), 0.0, 1, 1,
            variant.flags() | (_lib.DA_ROUTE_BETA_IS_LOG if beta_is_log else 0),
            float(variant.silu_gain), float(variant.logit_scale(routing_dim)), float(eps),
            grad_logits.data_ptr(), weights.data_ptr(), atoms, _half_code(v_type), dbeta_rows.data_ptr(),
            _stream(device),
        ),
        "dictionary_route_hip backward rows",
    )
    del logits, grad_weights
    keys_vt = dictionary_key.detach().to(v_type).t().contiguous()
    du = _mm_f32(grad_logits, keys_vt)
    d_key = _mm_tn_f32(u_v, grad_logits)
    d_value = _mm_tn_f32(dr_v, weights)
    # With beta_is_log the row kernel writes the terms at log beta (times
    # beta inside the clamp's window, zero outside).
    dbeta = dbeta_rows.sum().reshape(1)
    dx = _normalize_backward(rows, du, eps, x.dtype) if normalize_input else du.to(x.dtype)
    return (
        dx.reshape(x.shape),
        d_key.to(bank_grad_dtype or dictionary_key.dtype),
        d_value.to(bank_grad_dtype or dictionary_value.dtype),
        dbeta,
    )


def route_gradients(
    x: Tensor,
    dictionary_key: Tensor,
    dictionary_value: Tensor,
    beta: Tensor | float,
    eps: float,
    normalize_input: bool,
    normalize_output: bool,
    variant: RouteVariant,
    grad: Tensor,
    needs: tuple[bool, bool, bool, bool] = (True, True, True, True),
    r: Tensor | None = None,
    bank_grad_dtype: torch.dtype | None = None,
    beta_is_log: bool = False,
) -> tuple[Tensor | None, Tensor | None, Tensor | None, Tensor | None]:
    """(dx, dDk, dDv, dbeta) of the route for ``d loss / d out = grad``.

    The attention backward kernels take the plain softmax route up to
    256-wide rows and 1024 atoms; the row kernel with library GEMMs takes
    every other width, variant and bank size.
    ``needs`` marks the wanted gradients (dbeta only for a tensor beta); ``r``
    is the forward's reconstruction before the output norm, when the caller
    kept it (else one route launch forms it again); ``bank_grad_dtype``
    overrides the dtype of the two bank gradients (the native paths only).
    ``beta_is_log``: ``beta`` is the log-beta tensor (the route uses
    exp(clamp(., ln 0.05, ln 64))) and the last gradient is at the log.
    """

    native = None
    if _route_backward_supported(x, dictionary_key, variant):
        native = _route_backward(
            x, dictionary_key, dictionary_value, beta, eps, normalize_input, normalize_output, grad, r,
            bank_grad_dtype, beta_is_log,
        )
    elif _route_backward_rows_supported(x, dictionary_key):
        native = _route_backward_rows(
            x, dictionary_key, dictionary_value, beta, eps, normalize_input, normalize_output, grad, variant, r,
            bank_grad_dtype, beta_is_log,
        )
    if native is not None:
        dx, ddk, ddv, dbeta = native
        beta_grad = dbeta.reshape(beta.shape).to(beta.dtype) if isinstance(beta, Tensor) and needs[3] else None
        return (dx if needs[0] else None, ddk if needs[1] else None, ddv if needs[2] else None, beta_grad)
    with torch.enable_grad():
        inputs = [t.detach().requires_grad_(need) for t, need in zip((x, dictionary_key, dictionary_value), needs)]
        beta_in = beta.detach().requires_grad_(needs[3]) if isinstance(beta, Tensor) else beta
        beta_used = beta_in.clamp(*LOG_BETA_RANGE).exp() if beta_is_log else beta_in
        out = dictionary_route_reference(
            inputs[0], inputs[1], inputs[2], beta_used, eps,
            activation="silu" if variant.silu_logits else "identity",
            assignment="silu" if variant.direct_silu else "softmax",
            silu_gain=variant.silu_gain,
            standardize_logits=variant.standardize_logits,
            standardized_logit_scale=variant.standardized_logit_scale,
            normalize_input=normalize_input, normalize_output=normalize_output,
        )
        wrt = [t for t in inputs if t.requires_grad]
        if isinstance(beta_in, Tensor) and beta_in.requires_grad:
            wrt.append(beta_in)
        grads = torch.autograd.grad(out, wrt, grad.to(out.dtype), allow_unused=True) if wrt else ()
    it = iter(grads)
    result = [next(it) if t.requires_grad else None for t in inputs]
    beta_grad = next(it) if isinstance(beta_in, Tensor) and beta_in.requires_grad else None
    return (*result, beta_grad)


class _RouteFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, dictionary_key, dictionary_value, beta, eps, normalize_input, normalize_output, variant):  # type: ignore[override]
        layout = route_layout(dictionary_key, dictionary_value, route_key_dtype(normalize_input, x.dtype))
        ctx.save_for_backward(x, dictionary_key, dictionary_value, *(beta,) if isinstance(beta, Tensor) else ())
        ctx.beta_is_tensor = isinstance(beta, Tensor)
        ctx.beta = None if ctx.beta_is_tensor else beta
        ctx.eps = eps
        ctx.flags = (normalize_input, normalize_output)
        ctx.variant = variant
        return _route_forward(x, layout, beta, eps, normalize_input, normalize_output, variant)

    @staticmethod
    def backward(ctx, grad):  # type: ignore[override]
        saved = ctx.saved_tensors
        x, dk, dv = saved[:3]
        beta = saved[3] if ctx.beta_is_tensor else ctx.beta
        grads = route_gradients(x, dk, dv, beta, ctx.eps, *ctx.flags, ctx.variant, grad, tuple(ctx.needs_input_grad[:4]))
        return (*grads, None, None, None, None)


def dictionary_route_hip(
    input: Tensor,
    dictionary_key: Tensor,
    dictionary_value: Tensor,
    beta: Tensor | float,
    eps: float = 1e-6,
    silu_logits: bool = False,
    direct_silu: bool = False,
    silu_gain: float = 1.0,
    standardize_logits: bool = False,
    standardized_logit_scale: float | None = None,
    normalize_input: bool = True,
    normalize_output: bool = True,
) -> Tensor:
    """Fused dictionary route on gfx950; same arguments as ``dictionary_route_triton``.

    ``input`` is ``[..., R]`` (any number of rows), ``dictionary_key`` and
    ``dictionary_value`` are normalized ``[R, M]`` banks in the input dtype.
    """

    variant = RouteVariant(silu_logits, direct_silu, float(silu_gain), standardize_logits, standardized_logit_scale)
    if direct_silu and not silu_gain > 0:
        raise ValueError("silu_gain must be positive")
    if standardize_logits and standardized_logit_scale is not None and not standardized_logit_scale > 0:
        raise ValueError("standardized_logit_scale must be positive when provided")
    _require_cuda(input, dictionary_key, dictionary_value)
    _half_code(input.dtype)
    tagged = _tagged_layout(dictionary_key, dictionary_value) is not None
    if not tagged and (dictionary_key.dtype != input.dtype or dictionary_value.dtype != input.dtype):
        raise ValueError("input and dictionaries must have one matching dtype")
    needs_grad = torch.is_grad_enabled() and any(
        t.requires_grad for t in (input, dictionary_key, dictionary_value, *((beta,) if isinstance(beta, Tensor) else ()))
    )
    if needs_grad:
        return _RouteFunction.apply(
            input, dictionary_key, dictionary_value, beta, eps, normalize_input, normalize_output, variant
        )
    layout = route_layout(dictionary_key, dictionary_value, route_key_dtype(normalize_input, input.dtype))
    return _route_forward(input, layout, beta, eps, normalize_input, normalize_output, variant)


# --------------------------------------------------------------------------
# Outer attention
# --------------------------------------------------------------------------


def _next_width(width: int) -> int:
    for w in SUPPORTED_WIDTHS:
        if width <= w:
            return w
    raise NotImplementedError(f"HIP attention supports widths up to {SUPPORTED_WIDTHS[-1]}, got {width}")


def _value_width(width: int) -> int:
    """The attention forward's value width for ``width`` features: the next
    multiple of 64 (the tail is zero-padded), at most 4096."""

    padded = _round_up(max(width, 1), VALUE_WIDTH_STEP)
    if padded > MAX_VALUE_WIDTH:
        raise NotImplementedError(f"HIP attention supports value widths up to {MAX_VALUE_WIDTH}, got {width}")
    return padded


def value_transposed(value: Tensor, width: int | None = None) -> Tensor:
    """``[B, T, D]`` -> zero-padded V^T in 32-token tiles ``[B, Tp/32, width, 32]``."""

    batch, length, model_dim = value.shape
    width = width or model_dim
    padded = _round_up(max(length, 1), TOKEN_PAD)
    vt = torch.zeros(batch, padded // 32, width, 32, dtype=value.dtype, device=value.device)
    src = torch.zeros(batch, padded, width, dtype=value.dtype, device=value.device)
    src[:, :length, :model_dim].copy_(value.detach())
    vt.copy_(src.view(batch, padded // 32, 32, width).transpose(2, 3))
    return vt


def _attention_forward(
    query: Tensor, key: Tensor, value: Tensor | None, scales: Tensor, causal: bool, score_bound: float = 0.0,
    vt: Tensor | None = None, out_dtype: torch.dtype | None = None,
) -> Tensor:
    """Per-map outputs ``[B, S, T, D]``; the values come as rows ``value``
    ``[B, T, D]`` (zero-padded to a multiple of 64 features) or already as the
    projection's V^T tiles ``vt`` (D a multiple of 64).  ``out_dtype``
    torch.float32 keeps the outputs in fp32 (else the value dtype)."""

    batch, maps, length, score_dim = query.shape
    model_dim = value.shape[-1] if vt is None else vt.shape[2]
    value_dtype = value.dtype if vt is None else vt.dtype
    device = query.device
    score_width = _next_width(score_dim)
    value_width = _value_width(model_dim)
    q = query.detach()
    k = key.detach()
    if score_width != score_dim:
        pad = (0, score_width - score_dim)
        q = torch.nn.functional.pad(q, pad)
        k = torch.nn.functional.pad(k, pad)
    q = _aligned(q)
    k = _aligned(k)
    if vt is None:
        vt = value_transposed(value, value_width)
    elif value_width != model_dim:
        raise ValueError(f"V^T tiles need a value width that is a multiple of {VALUE_WIDTH_STEP}")
    out_f32 = out_dtype == torch.float32
    out = torch.empty(batch, maps, length, value_width, dtype=torch.float32 if out_f32 else value_dtype, device=device)
    scales_c = scales.detach().contiguous()
    lib = _lib.get()
    flags = (_lib.DA_ATTN_CAUSAL if causal else 0) | (_lib.DA_ATTN_OUT_F32 if out_f32 else 0)
    ws_bytes = lib.da_attention_workspace_bytes(batch, maps, length, score_width, value_width, flags)
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device) if ws_bytes > 0 else None
    _lib.check(
        lib.da_routed_attention(
            q.data_ptr(), k.data_ptr(),
            maps * length * score_width, score_width, length * score_width, 1, score_width,
            vt.data_ptr(), vt.stride(0),
            batch, maps, length, value_width,
            scales_c.data_ptr(), dtype_code(scales_c.dtype), 1.0, None, _lib.DA_F32,
            flags, float(score_bound),
            _half_code(q.dtype), _half_code(value_dtype),
            out.data_ptr(), out.stride(0), out.stride(2), out.stride(1),
            _ptr(workspace), ws_bytes,
            _stream(device),
        ),
        "routed_attention_hip",
    )
    return out if value_width == model_dim else out[..., :model_dim]


def routed_score_layout(branches: int, maps: int, routing_dim: int) -> tuple[int, int, int, float]:
    """(score width, map stride, map repeat, scale multiplier) of the score maps
    read as views of routed ``[B, T, 2, branches, routing_dim]`` rows: the
    assembly of ``assemble_score_maps`` (``ops.py:96-139``) without copies.
    Grouped branches (``branches > maps``) form one map of ``group`` adjacent
    branches with the scores multiplied by ``group^-1/2`` (the ``group^-1/4``
    factor on both operands); repeated branches (``maps > branches``) serve
    ``maps / branches`` maps each."""

    if branches > maps:
        group = branches // maps
        return group * routing_dim, group * routing_dim, 1, group ** -0.5
    return routing_dim, routing_dim, maps // branches, 1.0


def _attention_forward_rows(
    routed: Tensor, branches: int, maps: int, vt: Tensor, log_scales: Tensor, causal: bool, score_bound: float,
) -> Tensor:
    """Per-map fp32 outputs ``[B, S, T, D]`` of the outer attention
    (``modules.py:242-263`` without the combine), reading the score maps as
    views of the routed ``[B, T, 2, H, R]`` rows (``routed_score_layout``)
    and the temperatures as the kernel's exp(clamp(log_scales, ln 1/4,
    ln 1024)); values come as the projection's V^T tiles ``vt``."""

    batch, length, _, _, routing_dim = routed.shape
    if routed.stride(-1) != 1 or not routed.is_contiguous() or routed.data_ptr() % 16:
        raise ValueError("routed rows must be contiguous and 16-byte aligned")
    width = branches * routing_dim
    score_dim, map_stride, repeat, mult = routed_score_layout(branches, maps, routing_dim)
    model_dim = vt.shape[2]
    device = routed.device
    out = torch.empty(batch, maps, length, model_dim, dtype=torch.float32, device=device)
    scales = log_scales.detach().contiguous()
    flags = (_lib.DA_ATTN_CAUSAL if causal else 0) | _lib.DA_ATTN_OUT_F32 | _lib.DA_ATTN_SCALES_ARE_LOG
    lib = _lib.get()
    ws_bytes = lib.da_attention_workspace_bytes(batch, maps, length, score_dim, model_dim, flags)
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device) if ws_bytes > 0 else None
    _lib.check(
        lib.da_routed_attention(
            routed.data_ptr(), routed.data_ptr() + width * routed.element_size(),
            length * 2 * width, 2 * width, map_stride, repeat, score_dim,
            vt.data_ptr(), vt.stride(0),
            batch, maps, length, model_dim,
            scales.data_ptr(), dtype_code(scales.dtype), float(mult), None, _lib.DA_F32,
            flags, float(score_bound),
            _half_code(routed.dtype), _half_code(vt.dtype),
            out.data_ptr(), out.stride(0), out.stride(2), out.stride(1),
            _ptr(workspace), ws_bytes,
            _stream(device),
        ),
        "routed_attention_hip",
    )
    return out


BACKWARD_SCORE_WIDTHS = (64, 128, 256, 512)


def _padded_rows(t: Tensor, width: int) -> Tensor:
    """Contiguous, 16-byte-aligned copy of ``t`` zero-padded on its last dim to ``width``."""

    if t.shape[-1] != width:
        t = torch.nn.functional.pad(t, (0, width - t.shape[-1]))
    return _aligned(t)


def _attention_backward(
    query: Tensor, key: Tensor, value: Tensor, scales: Tensor, out: Tensor, grad: Tensor, causal: bool,
    qk_grad_dtype: torch.dtype | None = None,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Gradients of ``routed_attention_reference`` on the library's backward kernels.

    The flash-attention backward of ``triton_kernels.py:2093-2263``: a prep
    pass (transposed tiles, rowsum(dO . O), zeroed gradients), a pass for each
    query row's log-sum-exp, then one workgroup per (sequence, map, 64-key
    tile, run of query tiles) forming dV, dK, dQ and d(scale).
    """

    batch, maps, length, score_dim = query.shape
    model_dim = value.shape[-1]
    score_width = _next_width(score_dim)
    value_width = _next_width(model_dim)   # the backward kernels take 64 .. 512
    rows = batch * maps
    device = value.device
    q = _padded_rows(query.detach(), score_width)
    k = _padded_rows(key.detach(), score_width)
    v = _padded_rows(value.detach(), value_width)
    # fp32 forward outputs stay fp32 (the kernel's rowsum(dO . O) reads them so).
    out_f32 = out.dtype == torch.float32
    o = _padded_rows(out.detach() if out_f32 else out.detach().to(value.dtype), value_width)
    go = _padded_rows(grad.detach().to(value.dtype), value_width)
    gamma = scales.detach().float().contiguous()
    lib = _lib.get()
    ws_bytes = lib.da_attention_backward_workspace_bytes(batch, maps, length, length, score_width, value_width)
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    dq = torch.empty(rows, length, score_width, dtype=torch.float32, device=device)
    dk = torch.empty_like(dq)
    dv = torch.empty(batch, length, value_width, dtype=torch.float32, device=device)
    dg = torch.empty(maps, dtype=torch.float32, device=device)
    _lib.check(
        lib.da_routed_attention_backward(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), go.data_ptr(), gamma.data_ptr(),
            batch, maps, length, length, score_width, value_width,
            (_lib.DA_ATTN_CAUSAL if causal else 0) | (_lib.DA_ATTN_OUT_F32 if out_f32 else 0),
            _half_code(q.dtype), _half_code(value.dtype),
            workspace.data_ptr(), ws_bytes, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dg.data_ptr(),
            _stream(device),
        ),
        "routed_attention_hip backward",
    )
    shape = (batch, maps, length, score_width)
    return (
        dq.view(shape)[..., :score_dim].to(qk_grad_dtype or query.dtype),
        dk.view(shape)[..., :score_dim].to(qk_grad_dtype or key.dtype),
        dv[..., :model_dim].to(value.dtype),
        dg.to(scales.dtype),
    )


def rows_backward_supported(
    batch: int, length: int, branches: int, maps: int, routing_dim: int, model_dim: int
) -> bool:
    """Whether ``attention_gradients_rows`` takes this module shape: the
    key-tile kernels' score and value widths, and not the dense path."""

    score_dim = routed_score_layout(branches, maps, routing_dim)[0]
    if score_dim not in BACKWARD_SCORE_WIDTHS or model_dim not in SUPPORTED_WIDTHS:
        return False
    if batch * maps > 65535 or length < 1:
        return False
    return not _dense_fits(batch, maps, length, score_dim, model_dim)


def attention_gradients_rows(
    routed: Tensor, branches: int, maps: int, vt: Tensor, log_scales: Tensor, out: Tensor, grad: Tensor,
    causal: bool,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Outer-attention gradients at the routed rows (the backward of
    ``_attention_forward_rows``) on the key-tile kernels, for shapes
    ``rows_backward_supported`` accepts.

    ``routed`` ``[B, T, 2, H, R]`` (16-bit), ``vt`` the forward's V^T tiles
    ``[B, Tp/32, D, 32]`` (read as they are: the prep kernel turns them into
    value rows), ``out`` the fp32 per-map outputs ``[B, S, T, D]`` and
    ``grad`` their gradient.  Returns ``(d_routed, d_value, d_log_scales,
    d_value_sums)``, all fp32 (the last the column sums of ``d_value``, the
    gradient of the value projection's bias):
    ``d_routed`` has the routed rows' shape (the score-map assembly's
    backward, maps sharing rows summed), ``d_log_scales`` the gradient at
    ``log_scales`` through the kernels' clamp.
    """

    batch, length, _, _, routing_dim = routed.shape
    model_dim = vt.shape[2]
    if vt.shape[0] != batch or vt.shape[1] * 32 < length or vt.shape[3] != 32 or not vt.is_contiguous():
        raise ValueError("vt must be contiguous [B, Tp/32, D, 32] V^T tiles covering the sequence")
    if vt.shape[1] * 32 != _round_up(length, TOKEN_PAD):
        raise ValueError(f"vt must hold the sequence padded to a multiple of {TOKEN_PAD} tokens")
    width = branches * routing_dim
    score_dim, map_stride, repeat, mult = routed_score_layout(branches, maps, routing_dim)
    device = routed.device
    v_type = vt.dtype
    v = (vt, vt.stride(0), v_type)
    o = _aligned(out.detach())
    go = _aligned(grad.detach().to(v_type))
    scales = log_scales.detach().contiguous()
    d_routed = torch.empty(batch, length, 2, branches, routing_dim, dtype=torch.float32, device=device)
    d_value = torch.empty(batch, length, model_dim, dtype=torch.float32, device=device)
    d_scales = torch.empty(maps, dtype=torch.float32, device=device)
    d_sums = torch.empty(model_dim, dtype=torch.float32, device=device)
    row = (length * 2 * width, 2 * width, map_stride)
    q_ptr, k_off = routed.data_ptr(), width * routed.element_size()
    dq_ptr, dk_off = d_routed.data_ptr(), width * 4
    _attention_backward_ex(
        (q_ptr, *row), (q_ptr + k_off, *row), repeat, v, o, go, scales, float(mult), LOG_SCALE_RANGE,
        (batch, maps, length, length, score_dim, model_dim), causal, routed.dtype,
        dq_ptr, dq_ptr + dk_off, d_value, d_scales, "routed_attention_hip backward", d_sums,
    )
    return d_routed, d_value, d_scales, d_sums


def _native_backward_supported(query: Tensor, value: Tensor) -> bool:
    batch, maps, _, score_dim = query.shape
    return score_dim <= BACKWARD_SCORE_WIDTHS[-1] and batch * maps <= 65535 and value.shape[-1] <= SUPPORTED_WIDTHS[-1]


# The dense backward (library GEMMs around the row kernel, the score matrices
# materialized: 12 bytes per score) against the key-tile kernels, measured at
# outer-attention shapes (ms, causal, fp16 q/k, bf16 v): T 8192 R 256: 1.177
# flash / 0.884 dense; T 4096: 0.376 / 0.265; 4 x 2048: 0.333 / 0.274; 4 x 2048
# at 512-wide scores: 0.523 / 0.305 (there the flash backward splits each key
# tile over two workgroups and forms S and dP twice); 8 x 512: 0.126 / 0.243;
# 8 sequences x 4 maps x 1024 at R 128: 0.397 / 0.399.  So the dense path takes
# sequences of at least 2048 tokens, 512-wide scores, and value widths past the
# key-tile kernels' 512, whenever B*S*T*T <= 2^27.
DENSE_BACKWARD_MIN_SCORE_DIM = 512
DENSE_BACKWARD_MIN_LENGTH = 2048
DENSE_BACKWARD_MAX_SCORES = 1 << 27


def _dense_fits(batch: int, maps: int, length: int, score_dim: int, model_dim: int) -> bool:
    if not (score_dim <= BACKWARD_SCORE_WIDTHS[-1] and length >= 1 and maps <= 64
            and batch * maps * length * length <= DENSE_BACKWARD_MAX_SCORES):
        return False
    return (score_dim >= DENSE_BACKWARD_MIN_SCORE_DIM or length >= DENSE_BACKWARD_MIN_LENGTH
            or model_dim > SUPPORTED_WIDTHS[-1])


def _dense_backward_fits(query: Tensor, value: Tensor) -> bool:
    batch, maps, length, score_dim = query.shape
    return _dense_fits(batch, maps, length, score_dim, value.shape[-1])


def _dense_operands(query: Tensor, key: Tensor, v_type: torch.dtype) -> tuple[Tensor, Tensor, Tensor] | None:
    """``(K^T, q, k)`` of the dense backward from the score maps ``query`` and
    ``key`` ``[B, S, T, R]`` (16-bit, rows of unit stride, the same layout):
    ``da_dense_attention_operands``, or None where the kernel does not take
    them."""

    batch, maps, length, score_dim = query.shape
    if (not query.is_cuda or query.dtype not in (torch.float16, torch.bfloat16) or key.dtype != query.dtype
            or key.shape != query.shape or key.stride() != query.stride() or query.stride(3) != 1
            or score_dim % 64 or score_dim > 4096 or batch * maps > 65535 or length == 0):
        return None
    sb, ms, st = query.stride(0), query.stride(1), query.stride(2)
    if sb % 8 or ms % 8 or st % 8 or st < score_dim or query.data_ptr() % 16 or key.data_ptr() % 16:
        return None
    rows = batch * maps
    k_t = torch.empty(rows, score_dim, length, dtype=query.dtype, device=query.device)
    q_v = torch.empty(rows, length, score_dim, dtype=v_type, device=query.device)
    k_v = torch.empty_like(q_v)
    _lib.check(
        _lib.get().da_dense_attention_operands(
            query.data_ptr(), key.data_ptr(), sb, st, ms, 1, _half_code(query.dtype), batch, maps, length, score_dim,
            k_t.data_ptr(), q_v.data_ptr(), k_v.data_ptr(), _half_code(v_type), _stream(query.device),
        ),
        "dense attention operands",
    )
    return k_t, q_v, k_v


def _attention_backward_dense(
    query: Tensor, key: Tensor, value: Tensor | None, scales: Tensor, grad: Tensor, causal: bool,
    qk_grad_dtype: torch.dtype | None = None, value_t: Tensor | None = None, scales_are_log: bool = False,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Outer-attention gradients with the score matrices materialized.

    Library GEMMs form S = q k^T and dP = dO V^T (fp32 results) per
    (sequence, map); ``da_dictionary_route_backward_rows`` turns each row into
    P and gamma P (dP - sum P dP) (the gradient at q . k) with the causal row
    length and the map's gamma, plus the row's term of d gamma; GEMMs then
    give dq = dS k, dk = dS^T q and dV = sum over maps of P^T dO.  The row
    sum uses P and dP themselves, no saved output.  dS and P are stored in
    the value dtype (16-bit) between the row kernel and the GEMMs, which
    accumulate in fp32.

    ``query`` and ``key`` may be strided views (rows of unit stride: the
    score maps of the routed rows); the values come as rows ``value``
    ``[B, T, D]`` or, with ``value`` None, as the forward's V^T tiles
    ``value_t`` ``[B, Tp/32, D, 32]``, laid out as V^T by one copy.  With
    ``scales_are_log`` the scales are log gammas: the row kernel clamps and
    exponentiates them (the temperature window ``LOG_SCALE_RANGE``) and the
    scale gradient comes back at the logs (zero outside the window).
    """

    batch, maps, length, score_dim = query.shape
    rows = batch * maps
    device = query.device
    if value is None:
        if value_t is None:
            raise ValueError("value or value_t is required")
        model_dim, in_type = value_t.shape[2], value_t.dtype
    else:
        model_dim, in_type = value.shape[-1], value.dtype
    v_type = in_type if in_type in (torch.float16, torch.bfloat16) else torch.bfloat16

    def rows_of(t: Tensor) -> Tensor:
        # [rows, T, R] without a copy where the rows already have unit stride.
        t = t.detach().reshape(rows, length, score_dim)
        return t if t.stride(2) == 1 and t.stride(1) >= score_dim else t.contiguous()

    q, k = rows_of(query), rows_of(key)
    # Right operands of the products are contiguous (no transposed views):
    # K^T for S = q k^T, and q, k in the value dtype for dk and dq, written in
    # one pass over the score maps where the kernel takes their layout.
    operands = _dense_operands(query, key, v_type)
    if operands is not None:
        k_t, q_v, k_v = operands
    else:
        k_t, q_v, k_v = k.transpose(1, 2).contiguous(), None, None
    scores = torch.bmm(q, k_t, out_dtype=torch.float32)
    go = grad.detach().reshape(rows, length, model_dim).to(v_type).contiguous()
    if value is None:
        padded = value_t.shape[1] * 32
        vt = value_t.detach().to(v_type).permute(0, 2, 1, 3).reshape(batch, model_dim, padded)
        if padded != length:
            vt = vt[:, :, :length].contiguous()
    else:
        vt = value.detach().to(v_type).transpose(1, 2).contiguous()
    if maps > 1:
        vt = vt.unsqueeze(1).expand(batch, maps, model_dim, length).reshape(rows, model_dim, length)
    grad_p = torch.bmm(go, vt, out_dtype=torch.float32)
    grad_s = torch.empty(rows, length, length, dtype=v_type, device=device)
    probs = torch.empty_like(grad_s)
    dgamma_rows = torch.empty(rows * length, dtype=torch.float32, device=device)
    gamma = scales.detach().contiguous() if scales_are_log else scales.detach().float().contiguous()
    lib = _lib.get()
    _lib.check(
        lib.da_dictionary_route_backward_rows(
            scores.data_ptr(), grad_p.data_ptr(), rows * length, length, length if causal else 0, length,
            gamma.data_ptr(), dtype_code(gamma.dtype), 0.0, maps, length,
            _lib.DA_ROUTE_BETA_IS_LOG_SCALE if scales_are_log else 0, 1.0, 1.0, 0.0,
            grad_s.data_ptr(), probs.data_ptr(), length, _half_code(v_type), dgamma_rows.data_ptr(),
            _stream(device),
        ),
        "routed_attention_hip dense backward",
    )
    del scores, grad_p
    dq = torch.bmm(grad_s, k_v if k_v is not None else k.to(v_type), out_dtype=torch.float32)
    dk = torch.bmm(grad_s.transpose(1, 2), q_v if q_v is not None else q.to(v_type), out_dtype=torch.float32)
    dv = torch.bmm(probs.transpose(1, 2), go, out_dtype=torch.float32)
    dv = dv.view(batch, length, model_dim) if maps == 1 else dv.view(batch, maps, length, model_dim).sum(1)
    dgamma = dgamma_rows.view(batch, maps, length).sum(dim=(0, 2))
    shape = (batch, maps, length, score_dim)
    return (dq.view(shape).to(qk_grad_dtype or query.dtype), dk.view(shape).to(qk_grad_dtype or key.dtype),
            dv.to(in_type), dgamma.to(scales.dtype))


def attention_gradients(
    query: Tensor, key: Tensor, value: Tensor, scales: Tensor, out: Tensor, grad: Tensor, causal: bool,
    needs: tuple[bool, bool, bool, bool] = (True, True, True, True), qk_grad_dtype: torch.dtype | None = None,
) -> tuple[Tensor | None, Tensor | None, Tensor | None, Tensor | None]:
    """(dq, dk, dv, dscales) of the outer attention whose output was ``out``:
    the dense backward for long sequences, 512-wide scores and values wider
    than 512 whose score matrices fit, the flash backward kernels otherwise,
    or autograd of the fp32-softmax reference for score widths above 512 (or
    wide values whose matrices do not fit).  ``qk_grad_dtype`` (e.g. fp32) keeps dq and dk in
    that dtype on the native paths instead of rounding them to the inputs'.
    On the dense path the row kernel writes dS (the gradient at q . k) and P
    in the value dtype, so there dq and dk are fp32 sums of 16-bit dS
    entries, not products of an unrounded dS."""

    if query.numel() and value.numel() and _dense_backward_fits(query, value):
        grads = _attention_backward_dense(query, key, value, scales, grad, causal, qk_grad_dtype)
        return tuple(g if need else None for g, need in zip(grads, needs))  # type: ignore[return-value]
    if _native_backward_supported(query, value) and query.numel() and value.numel():
        grads = _attention_backward(query, key, value, scales, out, grad, causal, qk_grad_dtype)
        return tuple(g if need else None for g, need in zip(grads, needs))  # type: ignore[return-value]
    with torch.enable_grad():
        inputs = [t.detach().requires_grad_(need) for t, need in zip((query, key, value, scales), needs)]
        ref = routed_attention_reference(*inputs, causal)
        wrt = [t for t in inputs if t.requires_grad]
        grads = torch.autograd.grad(ref, wrt, grad) if wrt else ()
    it = iter(grads)
    return tuple(next(it) if t.requires_grad else None for t in inputs)  # type: ignore[return-value]


class _AttentionFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, query, key, value, scales, causal):  # type: ignore[override]
        out = _attention_forward(query, key, value, scales, causal)
        ctx.save_for_backward(query, key, value, scales, out)
        ctx.causal = causal
        return out

    @staticmethod
    def backward(ctx, grad):  # type: ignore[override]
        query, key, value, scales, out = ctx.saved_tensors
        grads = attention_gradients(query, key, value, scales, out, grad, ctx.causal, tuple(ctx.needs_input_grad[:4]))
        return (*grads, None)


def routed_attention_hip(
    query: Tensor, key: Tensor, value: Tensor, scales: Tensor, causal: bool = True, *, score_bound: float = 0.0
) -> Tensor:
    """Flash outer attention on gfx950; same contract as ``routed_attention_triton``.

    ``query``/``key`` ``[B, S, T, R]``, ``value`` ``[B, T, D]`` (shared by every
    map), ``scales`` ``[S]``; returns ``[B, S, T, D]``.  ``score_bound`` (an
    extension; 0 = unknown) is an upper bound on ``|q . k|``, e.g. 1 for
    L2-normalized rows: it lets the kernel skip online-softmax rescaling.
    """

    if not score_bound >= 0.0 or math.isinf(score_bound):
        raise ValueError("score_bound must be finite and >= 0")

    if query.ndim != 4 or key.shape != query.shape:
        raise ValueError("query and key must have matching [B, S, T, R] shapes")
    if value.ndim != 3 or value.shape[:2] != (query.shape[0], query.shape[2]):
        raise ValueError("value must have shape [B, T, D] matching query")
    if scales.shape != (query.shape[1],):
        raise ValueError(f"scales must have shape [{query.shape[1]}]")
    _require_cuda(query, key, value, scales)
    if query.dtype != key.dtype or query.dtype not in (value.dtype, torch.float16):
        raise ValueError("query, key, and value must have one matching dtype (or fp16 query/key)")
    _half_code(query.dtype)
    _half_code(value.dtype)
    if torch.is_grad_enabled() and any(t.requires_grad for t in (query, key, value, scales)):
        return _AttentionFunction.apply(query, key, value, scales, causal)
    return _attention_forward(query, key, value, scales, causal, score_bound)


# --------------------------------------------------------------------------
# Linear layers (exposed for tests and the LM path)
# --------------------------------------------------------------------------


def linear_hip(
    x: Tensor,
    weight: Tensor,
    bias: Tensor | None = None,
    *,
    activation: str | None = None,
    residual: Tensor | None = None,
) -> Tensor:
    """``act(x @ weight.T (+ bias)) (+ residual)`` with the library's MFMA GEMM.

    ``activation`` is None or ``"gelu"`` (exact, ``nn.GELU()``); ``residual``
    has the output's shape and is added to the rounded result, as the
    unfused ``residual + linear(x)`` does.
    """

    _require_cuda(x, weight)
    code = _half_code(x.dtype)
    if weight.dtype != x.dtype:
        raise ValueError("x and weight must share a dtype")
    if activation not in (None, "gelu"):
        raise ValueError(f"unsupported activation {activation!r}")
    rows = _aligned(x.reshape(-1, x.shape[-1]))
    w = _aligned(weight.detach())
    out = torch.empty(*x.shape[:-1], weight.shape[0], dtype=x.dtype, device=x.device)
    b = None if bias is None else bias.detach().contiguous()
    res = None
    if residual is not None:
        if residual.shape != out.shape or residual.dtype != x.dtype:
            raise ValueError("residual must match the output's shape and dtype")
        res = _aligned(residual.detach())
    lib = _lib.get()
    bias_code = dtype_code(b.dtype) if b is not None else _lib.DA_F32
    if activation is None and res is None:
        rc = lib.da_linear(
            rows.data_ptr(), rows.shape[0], rows.shape[1], w.data_ptr(), w.shape[0],
            _ptr(b), bias_code, code, out.data_ptr(), _stream(x.device),
        )
    else:
        rc = lib.da_linear_ex(
            rows.data_ptr(), rows.shape[0], rows.shape[1], w.data_ptr(), w.shape[0],
            _ptr(b), bias_code, code, _lib.DA_ACT_GELU if activation == "gelu" else _lib.DA_ACT_NONE,
            _ptr(res), out.data_ptr(), _stream(x.device),
        )
    _lib.check(rc, "linear_hip")
    return out


def layer_norm_hip(x: Tensor, weight: Tensor | None, bias: Tensor | None, eps: float = 1e-5) -> Tensor:
    """``F.layer_norm`` over the last dimension (fp32 statistics, one rounding)."""

    _require_cuda(x)
    code = _half_code(x.dtype)
    dim = x.shape[-1]
    xc = _aligned(x)
    w = None if weight is None else _aligned(weight.detach())
    b = None if bias is None else _aligned(bias.detach())
    params = [t for t in (w, b) if t is not None]
    if len(params) == 2 and w.dtype != b.dtype:
        raise ValueError("LayerNorm weight and bias must share a dtype")
    out = torch.empty_like(xc)
    lib = _lib.get()
    _lib.check(
        lib.da_layer_norm(
            xc.data_ptr(), xc.numel() // dim if dim else 0, dim, _ptr(w), _ptr(b),
            dtype_code(params[0].dtype) if params else _lib.DA_F32, float(eps), code, out.data_ptr(),
            _stream(x.device),
        ),
        "layer_norm_hip",
    )
    return out


# Copies of the LayerNorm backward's parameter gradients its workgroups
# spread their atomic adds over (da_layer_norm_backward).
LAYER_NORM_PARAM_COPIES = 8


def layer_norm_backward_hip(
    x: Tensor, grad: Tensor, weight: Tensor | None, eps: float = 1e-5, params_dtype: torch.dtype = torch.float32
) -> tuple[Tensor, Tensor, Tensor]:
    """The backward of ``layer_norm_hip`` (autograd of ``nn.LayerNorm``) at
    ``grad``: ``(dx, d_weight, d_bias)``, dx in x's dtype, the parameter
    gradients fp32 sums over the rows (``da_layer_norm_backward``; the
    statistics are formed again from x), rounded once to ``params_dtype``."""

    _require_cuda(x)
    dim = x.shape[-1]
    xc = _aligned(x.detach())
    g = _aligned(grad.detach().to(x.dtype))
    w = None if weight is None else _aligned(weight.detach())
    dx = torch.empty_like(xc)
    dparams = torch.zeros(LAYER_NORM_PARAM_COPIES, 2, dim, dtype=torch.float32, device=x.device)
    lib = _lib.get()
    _lib.check(
        lib.da_layer_norm_backward(
            xc.data_ptr(), g.data_ptr(), xc.numel() // dim if dim else 0, dim, _ptr(w),
            dtype_code(w.dtype) if w is not None else _lib.DA_F32, float(eps), _half_code(x.dtype), dx.data_ptr(),
            dparams.data_ptr(), _stream(x.device),
        ),
        "layer_norm_hip backward",
    )
    if params_dtype in (torch.float16, torch.bfloat16) and dim % 4 == 0:
        # The copies added up and rounded once, in one launch.
        out = torch.empty(2, dim, dtype=params_dtype, device=x.device)
        _lib.check(
            lib.da_sum_partials(dparams.data_ptr(), LAYER_NORM_PARAM_COPIES, 2 * dim, out.data_ptr(),
                                _half_code(params_dtype), _stream(x.device)),
            "layer_norm_hip backward sums",
        )
        return dx.view(x.shape), out[0], out[1]
    summed = dparams.sum(0).to(params_dtype)
    return dx.view(x.shape), summed[0], summed[1]


MAP_COMBINE_MAX_MAPS = 8


def map_combine_supported(map_output: Tensor) -> bool:
    """Whether ``map_combine`` / ``map_combine_backward`` take these per-map
    outputs (fp32 ``[B, S, T, D]``, S <= 8, D a multiple of 8)."""

    return (map_output.is_cuda and map_output.dtype == torch.float32 and map_output.dim() == 4
            and 1 <= map_output.shape[1] <= MAP_COMBINE_MAX_MAPS and map_output.shape[3] % 8 == 0)


def map_combine(map_output: Tensor, weights: Tensor, dtype: torch.dtype) -> Tensor:
    """``einsum("s,bstd->btd", weights, map_output)`` (``modules.py:265-272``)
    over fp32 per-map outputs ``[B, S, T, D]``: fp32 sum, one rounding to
    ``dtype`` (``da_map_combine``)."""

    batch, maps, length, width = map_output.shape
    o = _aligned(map_output)
    w = weights.detach().float().contiguous()
    out = torch.empty(batch, length, width, dtype=dtype, device=o.device)
    lib = _lib.get()
    _lib.check(
        lib.da_map_combine(o.data_ptr(), batch, maps, length, width, w.data_ptr(), out.data_ptr(),
                           _half_code(dtype), _stream(o.device)),
        "map combine",
    )
    return out


def map_combine_backward(map_output: Tensor, weights: Tensor, grad: Tensor) -> tuple[Tensor, Tensor]:
    """The backward of ``map_combine`` at ``grad`` ``[B, T, D]`` (16-bit):
    ``(grad_maps, weight_grad)`` with grad_maps[b, s] = weights[s] grad[b]
    rounded to grad's dtype and weight_grad[s] = <map_output[:, s], grad>
    (fp32), in one pass (``da_map_combine_backward``)."""

    batch, maps, length, width = map_output.shape
    o = _aligned(map_output)
    g = _aligned(grad)
    w = weights.detach().float().contiguous()
    grad_maps = torch.empty(batch, maps, length, width, dtype=g.dtype, device=o.device)
    sums = torch.zeros(maps, dtype=torch.float32, device=o.device)
    lib = _lib.get()
    _lib.check(
        lib.da_map_combine_backward(o.data_ptr(), batch, maps, length, width, w.data_ptr(), g.data_ptr(),
                                    _half_code(g.dtype), grad_maps.data_ptr(), sums.data_ptr(), _stream(o.device)),
        "map combine backward",
    )
    return grad_maps, sums


def qkv_projection_hip(
    x: Tensor, query_weight: Tensor, key_weight: Tensor, value_weight: Tensor, value_bias: Tensor | None
) -> tuple[Tensor, Tensor]:
    """Q/K projections ``[B, T, 2W]`` and padded V^T ``[B, Tp/32, D, 32]`` in one launch."""

    batch, length, model_dim = x.shape
    width = query_weight.shape[0]
    code = _half_code(x.dtype)
    xc = _aligned(x)
    qk = torch.empty(batch, length, 2 * width, dtype=x.dtype, device=x.device)
    padded = _round_up(length, TOKEN_PAD)
    vt = torch.empty(batch, padded // 32, value_weight.shape[0], 32, dtype=x.dtype, device=x.device)
    b = None if value_bias is None else value_bias.detach().contiguous()
    wq, wk, wv = (_aligned(w.detach()) for w in (query_weight, key_weight, value_weight))
    lib = _lib.get()
    _lib.check(
        lib.da_qkv_projection(
            xc.data_ptr(), batch * length, model_dim, length,
            wq.data_ptr(), wk.data_ptr(), width,
            wv.data_ptr(), _ptr(b), value_weight.shape[0],
            dtype_code(b.dtype) if b is not None else _lib.DA_F32, code,
            qk.data_ptr(), vt.data_ptr(), vt.stride(0), padded, _stream(x.device),
        ),
        "qkv_projection_hip",
    )
    return qk, vt


# --------------------------------------------------------------------------
# Whole-module forward
# --------------------------------------------------------------------------


class HipForwardResult(NamedTuple):
    output: Tensor
    routed: Tensor | None   # [B, T, 2, H, R] fp16: routed query branches, then key branches


def check_module_supported(config) -> None:
    """Raise ``NotImplementedError`` for variants the HIP kernels do not cover."""

    if config.dictionary_activation not in ("identity", "silu") or config.dictionary_assignment not in (
        "softmax",
        "silu",
    ):
        raise NotImplementedError(
            f"backend='hip' has no kernel for activation={config.dictionary_activation!r}, "
            f"assignment={config.dictionary_assignment!r}"
        )
    if config.routing_dim not in SUPPORTED_WIDTHS:
        raise NotImplementedError(f"backend='hip' supports routing_dim in {SUPPORTED_WIDTHS}")
    group = config.qk_branches // config.outer_maps if config.qk_branches > config.outer_maps else 1
    if group * config.routing_dim not in SUPPORTED_WIDTHS:
        raise NotImplementedError("backend='hip' supports grouped score widths up to 512")
    if config.model_dim % VALUE_WIDTH_STEP or not VALUE_WIDTH_STEP <= config.model_dim <= MAX_VALUE_WIDTH:
        raise NotImplementedError(
            f"backend='hip' supports model_dim a multiple of {VALUE_WIDTH_STEP} in [{VALUE_WIDTH_STEP}, {MAX_VALUE_WIDTH}]"
        )
    if config.outer_maps > 64:
        raise NotImplementedError("backend='hip' supports at most 64 outer maps")


def own_bank_layout(bank, key_dtype: torch.dtype) -> RouteDictionary:
    """Empty route layouts for a bank that the forward normalizes itself."""

    routing_dim, atoms = bank.raw_key.shape
    padded = _round_up(atoms, ATOM_PAD)
    device = bank.raw_key.device
    key_t = torch.empty(padded, routing_dim, dtype=key_dtype, device=device)
    value = torch.empty(padded // 32, routing_dim, 32, dtype=torch.float16, device=device)
    return RouteDictionary(key_t, value, atoms, True)


def _module_operands(module, dtype: torch.dtype):
    """The operands of ``module`` that ``shared_dictionary_attention_hip``
    passes: the Q/K/V/output weights in the compute dtype, the value bias and
    log beta in the scalars' dtype, the log score scales and the map-mix
    logits, and that dtype.  Kept on the module while the parameters are the
    same tensors at the same version (a forward then casts nothing)."""

    output = module.output.weight if isinstance(module.output, torch.nn.Linear) else None
    params = (module.query.weight, module.key.weight, module.value.weight, output, module.value.bias,
              module.log_beta, module.log_score_scales, module.map_mix_logits)
    try:
        key = (dtype, tuple(None if p is None else (p.data_ptr(), p._version) for p in params))
    except RuntimeError:   # inference tensors keep no version counter
        key = None
    cached = module.__dict__.get("_hip_operands")
    if key is not None and cached is not None and cached[0] == key:
        return cached[1]

    def cast(t: Tensor | None) -> Tensor | None:
        if t is None:
            return None
        t = t.detach()
        if t.dtype != dtype:
            t = t.to(dtype)
        return _aligned(t)

    # Scalars and the value bias share one dtype code.
    scalar_dtype = module.log_score_scales.dtype
    bv = module.value.bias
    bv = None if bv is None else bv.detach().to(scalar_dtype).contiguous()
    mix = module.map_mix_logits
    operands = (
        cast(module.query.weight), cast(module.key.weight), cast(module.value.weight), cast(output), bv,
        module.log_beta.detach().to(scalar_dtype).contiguous(), module.log_score_scales.detach().contiguous(),
        None if mix is None else mix.detach().to(scalar_dtype).contiguous(), scalar_dtype,
    )
    if key is not None:
        module.__dict__["_hip_operands"] = (key, operands)
    return operands


def shared_dictionary_attention_hip(
    module,
    x: Tensor,
    layout: RouteDictionary,
    dtype: torch.dtype,
    raw_bank: tuple[Tensor, Tensor | None] | None = None,
    residual: Tensor | None = None,
    no_alloc: bool = False,
    want_routed: bool = True,
) -> HipForwardResult:
    """One ``SharedDictionaryAttention`` forward through the fused C entry point.

    With ``raw_bank`` (the bank's raw key / value atoms) the call first
    normalizes them into ``layout`` (from ``own_bank_layout``), inside its
    projection launch.  ``residual`` ([B, T, d] of the output dtype) is added
    to the output projection's rounded result (the block's ``x + ...``).
    ``no_alloc`` runs the allocation-free entry point, whose workspace is the
    library's per-GPU scratch array: no workspace tensor is allocated, and
    ``routed`` is None (the scratch belongs to the next call), as it is
    with ``want_routed`` False.
    """

    config = module.config
    batch, length, model_dim = x.shape
    code = _half_code(dtype)
    if layout.key_t.dtype != route_key_dtype(config.normalize_routing_input, dtype):
        raise ValueError("route dictionary key dtype does not match the configuration")

    xc = x.detach()
    if xc.dtype != dtype:
        xc = xc.to(dtype)
    xc = _aligned(xc)
    wq, wk, wv, wo, bv, log_beta, log_scales, mix, scalar_dtype = _module_operands(module, dtype)

    concat = config.map_combine == "concat"
    width = config.total_qk_width
    lib = _lib.get()
    ws_bytes = lib.da_sda_workspace_bytes(batch, length, model_dim, width, config.outer_maps, int(concat), int(wo is not None))
    workspace = None if no_alloc else torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    out = torch.empty(batch, length, model_dim, dtype=dtype, device=x.device)
    flags = (
        (_lib.DA_SDA_NORMALIZE_INPUT if config.normalize_routing_input else 0)
        | (_lib.DA_SDA_NORMALIZE_OUTPUT if config.normalize_routing_output else 0)
        | (_lib.DA_SDA_CAUSAL if config.causal else 0)
        | (_lib.DA_SDA_CONCAT if concat else 0)
        | (_lib.DA_SDA_UNIT_KEYS if layout.unit or raw_bank is not None else 0)
    )
    args = _lib.SdaForwardArgs(
        xc.data_ptr(), batch, length, model_dim,
        config.qk_branches, config.outer_maps, config.routing_dim, layout.atoms,
        wq.data_ptr(), wk.data_ptr(), wv.data_ptr(), _ptr(bv), _ptr(wo),
        layout.key_t.data_ptr(), layout.value.data_ptr(),
        log_beta.data_ptr(), log_scales.data_ptr(), _ptr(mix),
        dtype_code(scalar_dtype), code, float(config.eps), flags,
        _ptr(workspace), 0 if workspace is None else ws_bytes, out.data_ptr(),
    )
    if residual is not None:
        if residual.shape != out.shape or residual.dtype != dtype:
            raise ValueError("residual must match the output's shape and dtype")
        residual = _aligned(residual.detach())
        args.residual = residual.data_ptr()
    variant = RouteVariant.of_config(config)
    args.route_variant = variant.flags()
    args.silu_gain = variant.silu_gain
    args.logit_scale = variant.logit_scale(config.routing_dim)
    if raw_bank is not None:
        raw_key = raw_bank[0].detach().contiguous()
        raw_value = None if raw_bank[1] is None else raw_bank[1].detach().to(raw_key.dtype).contiguous()
        args.raw_key = raw_key.data_ptr()
        args.raw_value = _ptr(raw_value)
        args.raw_dtype = dtype_code(raw_key.dtype)
    if no_alloc:
        # The library picks the scratch array of the stream's device; x's
        # device is also made current for the call.
        with torch.cuda.device(x.device):
            _lib.check(lib.da_shared_dictionary_attention_forward_noalloc(args, _stream(x.device)),
                       "shared_dictionary_attention_hip (no_alloc)")
        return HipForwardResult(out, None)
    _lib.check(lib.da_shared_dictionary_attention_forward(args, _stream(x.device)), "shared_dictionary_attention_hip")
    if not want_routed:
        return HipForwardResult(out, None)
    routed_bytes = batch * length * 2 * width * 2
    routed = workspace[:routed_bytes].view(torch.float16).view(
        batch, length, 2, config.qk_branches, config.routing_dim
    )
    return HipForwardResult(out, routed)


__all__ = [
    "RouteDictionary",
    "RouteVariant",
    "dictionary_normalize_hip",
    "dictionary_route_hip",
    "layer_norm_hip",
    "linear_hip",
    "qkv_projection_hip",
    "route_key_dtype",
    "route_layout",
    "routed_attention_hip",
    "shared_dictionary_attention_hip",
    "value_transposed",
]
