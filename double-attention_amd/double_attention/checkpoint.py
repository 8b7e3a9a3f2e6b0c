"""Reading the reference's training checkpoints, and replaying a forward as a HIP graph.

``scripts/train_screen.py:211-234`` of the reference saves one payload per
checkpoint: ``{"model": state_dict, "optimizer", "scaler", "step",
"tokens_seen", "history", "args": vars(args)}``, and loads it back with
``torch.load(..., weights_only=False)`` (``train_screen.py:353-356``).  The
model state uses the reference's parameter names, which the modules here
keep, so ``model`` loads into a ``DoubleAttentionLM`` of either backend.
``load_training_checkpoint`` reads the payload with the restricted loader
(``weights_only=True``): tensors, containers and numbers only, plus the
``pathlib`` path objects that ``vars(args)`` holds; nothing in the file runs.
"""

from __future__ import annotations

import pathlib
from pathlib import Path
from typing import Any, Callable

import torch
from torch import nn

_PATH_TYPES = [pathlib.PosixPath, pathlib.PurePosixPath, pathlib.WindowsPath, pathlib.PureWindowsPath]


def load_training_checkpoint(path: str | Path, map_location: str | torch.device = "cpu") -> dict[str, Any]:
    """The checkpoint payload at ``path``, read with ``torch.load(weights_only=True)``."""

    with torch.serialization.safe_globals(_PATH_TYPES):
        payload = torch.load(path, map_location=map_location, weights_only=True)
    if not isinstance(payload, dict) or "model" not in payload:
        raise ValueError(f"{path} is not a training checkpoint (no 'model' entry)")
    return payload


def load_model_from_checkpoint(model: nn.Module, path: str | Path, *, strict: bool = True) -> dict[str, Any]:
    """Load the checkpoint's ``model`` state into ``model``; returns the payload.

    Tensors are moved to the model's device and dtype by ``load_state_dict``.
    """

    payload = load_training_checkpoint(path)
    model.load_state_dict(payload["model"], strict=strict)
    return payload


class GraphedForward:
    """A module forward captured once as a HIP graph and replayed.

    Every call copies the inputs into the captured input buffers, replays the
    graph and returns the captured output tensor (overwritten by the next
    call: clone it to keep it).  The inputs must keep the example's shapes,
    dtypes and device.  For inference only (the capture runs under
    ``torch.inference_mode``); the module's parameters may change in place
    between calls, but not be replaced.  Each replay launches the same kernels
    as an eager forward, without the per-call host work.
    """

    def __init__(self, module: Callable[..., Any], *example_inputs: torch.Tensor, warmup: int = 3) -> None:
        if not example_inputs or not all(isinstance(t, torch.Tensor) and t.is_cuda for t in example_inputs):
            raise ValueError("GraphedForward needs example inputs on the GPU")
        self.module = module
        self.inputs = tuple(t.detach().clone() for t in example_inputs)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.inference_mode():
            with torch.cuda.stream(side):
                for _ in range(warmup):
                    module(*self.inputs)
            torch.cuda.current_stream().wait_stream(side)
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph):
                self.output = module(*self.inputs)

    def __call__(self, *inputs: torch.Tensor) -> Any:
        if len(inputs) != len(self.inputs):
            raise ValueError(f"expected {len(self.inputs)} inputs, got {len(inputs)}")
        for dst, src in zip(self.inputs, inputs):
            if src.shape != dst.shape or src.dtype != dst.dtype or src.device != dst.device:
                raise ValueError("inputs must match the captured shapes, dtypes and device")
            dst.copy_(src)
        self.graph.replay()
        return self.output


__all__ = ["GraphedForward", "load_model_from_checkpoint", "load_training_checkpoint"]
