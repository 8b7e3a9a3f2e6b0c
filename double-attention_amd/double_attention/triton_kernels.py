"""The reference's Triton module name, kept so existing imports resolve.

This build has no Triton kernels (the GPU path is hand-written HIP for
gfx950, see ``hip_ops``).  ``TRITON_AVAILABLE`` is False and the two Triton
entry points raise the same ``RuntimeError`` the reference raises when Triton
is missing (reference ``src/double_attention/triton_kernels.py:1281-1283``).
"""

from __future__ import annotations

TRITON_AVAILABLE = False

_MESSAGE = "Triton is not available in this build; use backend='hip' (dictionary_route_hip / routed_attention_hip)"


def dictionary_route_triton(*args, **kwargs):
    raise RuntimeError(_MESSAGE)


def routed_attention_triton(*args, **kwargs):
    raise RuntimeError(_MESSAGE)
