"""Reference-format training checkpoints and the graphed forward.

The payload mirrors ``scripts/train_screen.py:211-234`` of the reference
(model / optimizer / scaler state, step, tokens_seen, history and
``vars(args)`` with ``pathlib`` paths); the reference ships no checkpoint
file, so the tests write one in that format.
"""

from __future__ import annotations

import argparse
import pickle
from pathlib import Path

import numpy as np
import pytest
import torch

import double_attention as da
import oracle


def _payload(model: torch.nn.Module) -> dict:
    optimizer = torch.optim.AdamW(model.parameters(), lr=1e-3)
    ids = torch.randint(0, 97, (2, 16), generator=torch.Generator().manual_seed(3))
    _, loss = model(ids, ids)
    loss.backward()
    optimizer.step()
    args = argparse.Namespace(variant="qk2-s2", ids=Path("data/docs_sp2048/docs_sp2048_ids.pt"), steps=10, seed=0)
    return {
        "model": model.state_dict(),
        "optimizer": optimizer.state_dict(),
        "scaler": torch.amp.GradScaler("cuda", enabled=False).state_dict(),
        "step": 1,
        "tokens_seen": 32,
        "history": [{"step": 1, "loss": float(loss.detach())}],
        "args": vars(args),
    }


def _small_lm(backend: str = "torch") -> da.DoubleAttentionLM:
    config = da.experiment_config("qk2-s2", untied_dictionary=False, model_dim=64, routing_dim=64,
                                  dictionary_size=48, backend=backend)
    return da.DoubleAttentionLM(97, 16, config, 2, dictionary_group_size=2, feedforward_dim=96)


def test_reference_checkpoint_round_trip(tmp_path) -> None:
    torch.manual_seed(0)
    model = _small_lm()
    path = tmp_path / "checkpoint.pt"
    torch.save(_payload(model), path)
    fresh = _small_lm()
    payload = da.load_model_from_checkpoint(fresh, path)
    assert payload["step"] == 1 and payload["tokens_seen"] == 32
    assert isinstance(payload["args"]["ids"], Path)
    ids = torch.randint(0, 97, (3, 16), generator=torch.Generator().manual_seed(4))
    with torch.inference_mode():
        torch.testing.assert_close(fresh(ids)[0], model(ids)[0], rtol=0, atol=0)


class _Executes:
    def __reduce__(self):
        return (print, ("a checkpoint ran code",))


def test_checkpoint_loader_refuses_code(tmp_path) -> None:
    path = tmp_path / "bad.pt"
    torch.save({"model": {}, "extra": _Executes()}, path)
    with pytest.raises(pickle.UnpicklingError):
        da.load_training_checkpoint(path)
    plain = tmp_path / "plain.pt"
    torch.save({"weights": torch.zeros(2)}, plain)
    with pytest.raises(ValueError, match="not a training checkpoint"):
        da.load_training_checkpoint(plain)


@pytest.mark.gpu
def test_reference_checkpoint_drives_the_hip_lm(tmp_path) -> None:
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    if not da.HIP_AVAILABLE:
        raise RuntimeError("HIP library not built; run python double-attention_amd/build.py")
    torch.manual_seed(0)
    trained = _small_lm()
    path = tmp_path / "checkpoint.pt"
    torch.save(_payload(trained), path)
    hip = _small_lm("hip")
    da.load_model_from_checkpoint(hip, path)
    hip = hip.cuda().bfloat16().eval()
    ids = torch.randint(0, 97, (4, 16), generator=torch.Generator().manual_seed(5))
    with torch.inference_mode():
        logits, _ = hip(ids.cuda())
    params = {k: v.detach().float().cpu().numpy() for k, v in hip.state_dict().items()}
    expected = oracle.double_attention_lm(params, hip.stack.config, ids.numpy(), 2, 2, dtype=np.float32)
    got = logits.float().cpu().numpy().astype(np.float64)
    rel = np.linalg.norm(got - expected) / np.linalg.norm(expected)
    print(f"[parity] checkpoint lm rel_l2={rel:.3e}", flush=True)
    # bf16 activations between the layers (LayerNorm, FFN, LM head): the LM bar.
    assert rel < 2e-2


@pytest.mark.gpu
def test_graphed_lm_forward_matches_eager() -> None:
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    if not da.HIP_AVAILABLE:
        raise RuntimeError("HIP library not built; run python double-attention_amd/build.py")
    config = da.experiment_config("qk2-s2", untied_dictionary=False, backend="hip")
    torch.manual_seed(0)
    lm = da.DoubleAttentionLM(2048, 64, config, 6, dictionary_group_size=6, feedforward_dim=1536)
    lm = lm.cuda().bfloat16().eval()
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 2048, (64, 64), generator=g).cuda()
    with torch.inference_mode():
        eager = lm(ids)[0].clone()
    graphed = da.GraphedForward(lm, ids)
    other = torch.randint(0, 2048, (64, 64), generator=g).cuda()
    with torch.inference_mode():
        eager_other = lm(other)[0].clone()
        # Replays interleaved with eager work and synchronizations; every one
        # must reproduce the eager logits of its inputs.
        for inputs, expected in ((ids, eager), (other, eager_other), (ids, eager)):
            out = graphed(inputs)[0]
            torch.cuda.synchronize()
            torch.testing.assert_close(out, expected, rtol=0, atol=0)
            lm(other)
            torch.cuda.synchronize()
