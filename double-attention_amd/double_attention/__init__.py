"""MI355X-native shared-dictionary attention (drop-in for ``double_attention``).

Public names follow the reference package's API (reference
``src/double_attention/__init__.py:1-47``) for the attention path; the
additions are ``backend="hip"`` in the config, ``HIP_AVAILABLE`` and the
gfx950 operator functions ``dictionary_route_hip`` / ``routed_attention_hip``.
"""

from . import _lib
from .checkpoint import GraphedForward, load_model_from_checkpoint, load_training_checkpoint
from .config import DoubleAttentionConfig, experiment_config, experiment_names
from .hip_ops import dictionary_normalize_hip, dictionary_route_hip, routed_attention_hip
from .modules import (
    DoubleAttentionAux,
    DoubleAttentionBlock,
    DoubleAttentionLM,
    DoubleAttentionStack,
    SharedDictionaryAttention,
    SharedDictionaryBank,
)
from .ops import assemble_score_maps, dictionary_route_reference, routed_attention_reference
from .triton_kernels import TRITON_AVAILABLE

HIP_AVAILABLE = _lib.available()

__all__ = [
    "DoubleAttentionAux",
    "DoubleAttentionBlock",
    "DoubleAttentionConfig",
    "DoubleAttentionLM",
    "DoubleAttentionStack",
    "GraphedForward",
    "HIP_AVAILABLE",
    "SharedDictionaryAttention",
    "SharedDictionaryBank",
    "TRITON_AVAILABLE",
    "assemble_score_maps",
    "dictionary_normalize_hip",
    "dictionary_route_hip",
    "dictionary_route_reference",
    "experiment_config",
    "experiment_names",
    "load_model_from_checkpoint",
    "load_training_checkpoint",
    "routed_attention_hip",
    "routed_attention_reference",
]
