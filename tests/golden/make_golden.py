"""Write golden vectors from the reference's own PyTorch path.

Run in the build container only (the reference checkout is not available on
the GPU machines):  ``python tests/golden/make_golden.py [/path/to/reference]``.

What the fixtures pin, and why they come from the reference rather than from
a closed form:
* ``SharedDictionaryAttention.forward`` and ``DoubleAttentionLM.forward`` end
  to end (reference ``src/double_attention/modules.py:190-291, 444-460``): the
  composition of projection, pair routing, map assembly, attention, combine
  and output projection has no closed form of its own;
* the default-init parameter stream (``modules.py:79-128, 33-43, 381-396,
  430-442``): a seeded construction must reproduce the reference's weights.

Each fixture is an ``.npz`` with the config (JSON), the default-initialized
state dict in float32, a float64 input and the float64 outputs of the
reference module run in float64 (``module.double()``).  Only data is written;
no reference source is copied.
"""

from __future__ import annotations

import copy
import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
DEFAULT_REFERENCE = Path("/root/reference")

# (fixture name, preset, config overrides, batch, length, seed)
SMALL = {"model_dim": 32, "routing_dim": 8, "dictionary_size": 16}
HIP_SIZED = {"model_dim": 64, "routing_dim": 64, "dictionary_size": 64}
ATTENTION_CASES = [
    ("a1_small", "a1", SMALL, 2, 7, 101),
    ("a1_tied_small", "a1", {**SMALL, "untied_dictionary": False}, 2, 7, 102),
    ("a1_no_qnorm_small", "a1-no-qnorm", SMALL, 2, 7, 103),
    ("a1_no_dpnorm_small", "a1-no-dpnorm", SMALL, 2, 7, 104),
    ("a1_no_norm_small", "a1-no-norm", SMALL, 2, 7, 105),
    ("a1_silu_small", "a1-silu", SMALL, 2, 7, 106),
    ("a1_silu_logitnorm_small", "a1-silu-logitnorm", SMALL, 2, 7, 107),
    ("a1_silu_logitnorm_t1_small", "a1-silu-logitnorm-t1", SMALL, 2, 7, 108),
    ("a1_no_softmax_g4_small", "a1-no-softmax-g4", SMALL, 2, 7, 109),
    ("qk2_s1_small", "qk2-s1", SMALL, 2, 7, 110),
    ("qk1_s2_small", "qk1-s2", SMALL, 2, 7, 111),
    ("qk2_s2_small", "qk2-s2", SMALL, 2, 7, 112),
    ("qk4_s4_small", "qk4-s4", SMALL, 2, 7, 113),
    ("qk2_s2_concat_small", "qk2-s2", {**SMALL, "map_combine": "concat"}, 2, 7, 114),
    ("a1_noproj_nobias_small", "a1", {**SMALL, "output_projection": False, "value_bias": False}, 2, 7, 115),
    ("a1_noncausal_small", "a1", {**SMALL, "causal": False}, 2, 7, 116),
    ("a1_hip", "a1", HIP_SIZED, 2, 9, 201),
    ("qk2_s2_hip", "qk2-s2", HIP_SIZED, 1, 11, 202),
]
# (fixture name, preset, overrides, layers, group size, ffn width, vocab, max length, batch, length, seed)
LM_CASES = [
    ("lm_qk2_s2_tied_small", "qk2-s2", {**SMALL, "untied_dictionary": False}, 3, 3, 48, 41, 12, 2, 9, 301),
    ("lm_a1_stagewise_small", "a1", SMALL, 4, 2, 48, 37, 10, 2, 8, 302),
    ("lm_a1_qffn_small", "a1-d1536-qffn", {**SMALL, "dictionary_size": 48}, 2, 2, 48, 29, 8, 2, 6, 303),
]


def _import_reference(root: Path):
    sys.path.insert(0, str(root / "src"))
    import double_attention  # noqa: PLC0415

    return double_attention


def _state(module: torch.nn.Module) -> dict[str, np.ndarray]:
    return {f"param:{k}": v.detach().float().numpy() for k, v in module.state_dict().items()}


def _config_json(config) -> str:
    return json.dumps({k: getattr(config, k) for k in config.__dataclass_fields__})


def main() -> None:
    root = Path(sys.argv[1]) if len(sys.argv) > 1 else DEFAULT_REFERENCE
    ref = _import_reference(root)
    torch.set_default_dtype(torch.float32)
    for name, preset, overrides, batch, length, seed in ATTENTION_CASES:
        config = ref.experiment_config(preset, backend="torch", **overrides)
        torch.manual_seed(seed)
        module = ref.SharedDictionaryAttention(config)
        generator = torch.Generator().manual_seed(seed + 1000)
        x = torch.randn(batch, length, config.model_dim, generator=generator, dtype=torch.float64)
        module64 = copy.deepcopy(module).double().eval()
        with torch.no_grad():
            out, aux = module64(x, return_aux=True)
        np.savez_compressed(
            HERE / f"{name}.npz",
            kind="attention",
            preset=preset,
            config=_config_json(config),
            seed=seed,
            x=x.numpy(),
            out=out.numpy(),
            routing_query=aux.routing_query.numpy(),
            routing_key=aux.routing_key.numpy(),
            torch_version=torch.__version__,
            **_state(module),
        )
        print("wrote", name, tuple(out.shape))
    for name, preset, overrides, layers, group, ffn, vocab, max_len, batch, length, seed in LM_CASES:
        config = ref.experiment_config(preset, backend="torch", **overrides)
        torch.manual_seed(seed)
        model = ref.DoubleAttentionLM(
            vocab_size=vocab,
            max_sequence_length=max_len,
            config=config,
            num_layers=layers,
            dictionary_group_size=group,
            feedforward_dim=ffn,
        )
        generator = torch.Generator().manual_seed(seed + 1000)
        ids = torch.randint(0, vocab, (batch, length), generator=generator)
        model64 = copy.deepcopy(model).double().eval()
        with torch.no_grad():
            logits, _ = model64(ids)
        np.savez_compressed(
            HERE / f"{name}.npz",
            kind="lm",
            preset=preset,
            config=_config_json(config),
            seed=seed,
            layers=layers,
            group=group,
            ffn=ffn,
            vocab=vocab,
            max_len=max_len,
            ids=ids.numpy(),
            logits=logits.numpy(),
            torch_version=torch.__version__,
            **_state(model),
        )
        print("wrote", name, tuple(logits.shape))


if __name__ == "__main__":
    main()
