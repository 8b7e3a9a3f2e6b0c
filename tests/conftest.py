"""Shared pytest setup: import paths, the ``gpu`` marker, golden-fixture loading."""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parents[1]
PACKAGE_ROOT = REPO / "double-attention_amd"
GOLDEN = Path(__file__).resolve().parent / "golden"
for path in (str(PACKAGE_ROOT), str(REPO)):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")


class Golden:
    """One fixture written by ``tests/golden/make_golden.py``."""

    def __init__(self, name: str) -> None:
        self.name = name
        with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as data:
            self.arrays = {k: data[k] for k in data.files}
        self.config = json.loads(str(self.arrays["config"]))
        self.params = {k[len("param:"):]: v for k, v in self.arrays.items() if k.startswith("param:")}

    def __getitem__(self, key: str) -> np.ndarray:
        return self.arrays[key]


def golden_names(kind: str) -> list[str]:
    names = []
    for path in sorted(GOLDEN.glob("*.npz")):
        with np.load(path, allow_pickle=False) as data:
            if str(data["kind"]) == kind:
                names.append(path.stem)
    return names


@pytest.fixture(scope="session")
def golden_loader():
    return Golden
