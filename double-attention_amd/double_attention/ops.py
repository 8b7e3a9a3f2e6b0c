"""PyTorch composition of the shared-dictionary attention math and backend dispatch.

These functions are the reference's ``backend="torch"`` path and public
helpers (reference ``src/double_attention/ops.py:16-161``), restated here so
that this package is a drop-in: same names, same arguments, same
semantics.  They run on whatever device their inputs live on and are used by
``backend="torch"`` and by the HIP path's autograd backward.  They are not
the parity oracle (that is the NumPy restatement under ``oracle/``).
"""

from __future__ import annotations

import math
from collections.abc import Sequence

import torch
import torch.nn.functional as F
from torch import Tensor

from .config import Backend

_SILU_FACTOR = 2.0  # 2*SiLU(x) has unit slope at zero (ops.py:41-43)


def dictionary_route_reference(
    x: Tensor,
    dictionary_key: Tensor,
    dictionary_value: Tensor,
    beta: Tensor | float,
    eps: float = 1e-6,
    activation: str = "identity",
    assignment: str = "softmax",
    silu_gain: float = 1.0,
    standardize_logits: bool = False,
    standardized_logit_scale: float | None = None,
    normalize_input: bool = True,
    normalize_output: bool = True,
) -> Tensor:
    """Dictionary feature map of ``x [..., R]`` against normalized ``[R, M]`` banks.

    assignment logits ``u . Dk`` (``u`` = L2-normalized ``x`` when
    ``normalize_input``), optional ``2*SiLU`` activation, optional
    standardization over the atom axis, then either ``softmax(beta * logits)``
    or the direct ``(2/g) SiLU(g * logits)`` weights, reconstruction with
    ``Dv``, and an optional output L2 normalization (``ops.py:16-62``).
    """

    u = F.normalize(x, dim=-1, eps=eps) if normalize_input else x
    logits = torch.matmul(u, dictionary_key)
    if activation == "silu":
        logits = _SILU_FACTOR * F.silu(logits)
    elif activation != "identity":
        raise ValueError(f"unsupported dictionary activation: {activation}")
    if standardize_logits:
        centered = logits - logits.mean(dim=-1, keepdim=True)
        spread = torch.rsqrt(centered.square().mean(dim=-1, keepdim=True) + eps)
        scale = x.shape[-1] ** -0.5 if standardized_logit_scale is None else standardized_logit_scale
        logits = centered * spread * scale
    if assignment == "softmax":
        weights = torch.softmax(logits * beta, dim=-1)
    elif assignment == "silu":
        weights = (_SILU_FACTOR / silu_gain) * F.silu(silu_gain * logits)
    else:
        raise ValueError(f"unsupported dictionary assignment: {assignment}")
    recon = torch.matmul(weights, dictionary_value.transpose(0, 1))
    return F.normalize(recon, dim=-1, eps=eps) if normalize_output else recon


def routed_attention_reference(
    query: Tensor,
    key: Tensor,
    value: Tensor,
    scales: Tensor,
    causal: bool = True,
) -> Tensor:
    """``softmax(scale_s * q k^T) V`` per map; ``q, k [B,S,T,R]``, ``value [B,T,D]``.

    Scores are formed in the input dtype, promoted to fp32 before scaling and
    masking (masked entries are ``-inf``), the softmax runs in fp32 and the
    probabilities are cast back to the value dtype (``ops.py:65-93``).
    """

    if query.ndim != 4 or key.shape != query.shape:
        raise ValueError("query and key must have matching [B, S, T, R] shapes")
    if value.ndim != 3 or value.shape[:2] != (query.shape[0], query.shape[2]):
        raise ValueError("value must have shape [B, T, D] matching query")
    if scales.shape != (query.shape[1],):
        raise ValueError(f"scales must have shape [{query.shape[1]}]")
    # A contiguous K^T: batched half-precision products with a transposed
    # right operand have faulted ROCm GPUs; the values are unchanged.
    scores = torch.matmul(query, key.transpose(-2, -1).contiguous()).float()
    scores = scores * scales.float()[None, :, None, None]
    if causal:
        length = query.shape[-2]
        future = torch.ones(length, length, dtype=torch.bool, device=query.device).triu(1)
        scores = scores.masked_fill(future, float("-inf"))
    probs = torch.softmax(scores, dim=-1).to(value.dtype)
    return torch.matmul(probs, value.unsqueeze(1).expand(-1, query.shape[1], -1, -1))


def assemble_score_maps(query: Tensor, key: Tensor, outer_maps: int) -> tuple[Tensor, Tensor]:
    """Turn ``[B, H, T, R]`` branches into ``[B, S, T, R']`` score-map operands.

    ``H == S``: unchanged.  ``H > S``: each map concatenates ``H/S``
    consecutive branches, each scaled by ``(H/S)^(-1/4)`` so the map's dot
    product is the branch-score sum divided by ``sqrt(H/S)``.  ``S > H``: every
    branch is repeated ``S/H`` times (``ops.py:96-139``).
    """

    if query.ndim != 4 or query.shape != key.shape:
        raise ValueError("query and key must have matching [B, H, T, R] shapes")
    branches = query.shape[1]
    if branches == outer_maps:
        return query, key
    if branches > outer_maps:
        if branches % outer_maps:
            raise ValueError("qk_branches must be divisible by outer_maps")
        group = branches // outer_maps
        factor = group ** -0.25

        def grouped(t: Tensor) -> Tensor:
            b, _, length, width = t.shape
            # [B, S, g, T, R] -> [B, S, T, g, R] -> [B, S, T, g*R]
            parts = t.reshape(b, outer_maps, group, length, width).transpose(2, 3)
            return parts.reshape(b, outer_maps, length, group * width) * factor

        return grouped(query), grouped(key)
    if outer_maps % branches:
        raise ValueError("outer_maps must be divisible by qk_branches")
    repeats = outer_maps // branches
    return query.repeat_interleave(repeats, dim=1), key.repeat_interleave(repeats, dim=1)


def _hip_supported(tensors: Sequence[Tensor]) -> bool:
    return bool(tensors) and all(
        t.is_cuda and t.dtype in (torch.float16, torch.bfloat16) for t in tensors
    )


def resolve_backend(backend: Backend, tensors: Sequence[Tensor]) -> Backend:
    """Pick the implementation for one forward (reference ``ops.py:142-157``).

    * ``"torch"``: always the PyTorch composition.
    * ``"hip"``: the gfx950 kernels; raises ``RuntimeError`` when the library
      is missing or the tensors are not fp16/bf16 on a ROCm device.
    * ``"auto"``: ``"hip"`` for fp16/bf16 device tensors, else ``"torch"``.
      On a device, a missing HIP library is an installation error and raises
      rather than silently switching implementations.
    * ``"triton"``: this build has no Triton kernels; raises like the
      reference does when Triton is unavailable.
    """

    if backend == "torch":
        return "torch"
    if backend == "triton":
        raise RuntimeError(
            "Triton backend requested but unavailable: this MI355X build ships "
            "hand-written HIP kernels instead; use backend='hip'"
        )
    wants_hip = _hip_supported(tensors)
    if backend == "auto" and not wants_hip:
        return "torch"
    from . import _lib

    if not _lib.available():
        raise RuntimeError(f"HIP backend requested but unavailable: {_lib.unavailable_reason()}")
    if not wants_hip:
        raise RuntimeError(
            "HIP backend requested but unavailable: fp16/bf16 tensors on a ROCm device are required"
        )
    return "hip"


def score_scale_from_log(log_scale: Tensor) -> Tensor:
    """Outer-map temperatures ``exp(clamp(log_scale, ln 1/4, ln 1024))`` (``ops.py:160-161``)."""

    return log_scale.clamp(math.log(0.25), math.log(1024.0)).exp()
