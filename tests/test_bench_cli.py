"""CPU checks of bench.py's command-line contract (no GPU needed).

The driver runs ``python bench.py --gpus N --steps K --warmup W``; this build
measures one GPU, so any N above 1 must stop with a message and a non-zero
status before touching a device.
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

REPO = Path(__file__).resolve().parents[1]


def _run(*args: str) -> subprocess.CompletedProcess:
    return subprocess.run(
        [sys.executable, str(REPO / "bench.py"), *args], capture_output=True, text=True, timeout=120, cwd=REPO
    )


def test_more_than_one_gpu_is_refused() -> None:
    proc = _run("--gpus", "2", "--steps", "1", "--warmup", "0")
    assert proc.returncode == 2
    assert "one GPU" in proc.stdout + proc.stderr


def test_help_lists_the_workloads() -> None:
    proc = _run("--help")
    assert proc.returncode == 0
    for workload in ("c1", "c2", "c3", "c4", "c5"):
        assert workload in proc.stdout
