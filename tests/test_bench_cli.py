"""bench.py's command-line contract on the CPU: one GPU only, and a loud failure without one."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]


def _bench(*args: str) -> subprocess.CompletedProcess:
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                          timeout=300, cwd=ROOT)


def test_more_than_one_gpu_is_refused_with_a_message():
    result = _bench("--gpus", "2", "--steps", "1", "--warmup", "0")
    assert result.returncode == 2
    assert "one GPU" in result.stderr
    assert result.stdout == ""


@pytest.mark.skipif(torch.cuda.is_available(), reason="a GPU is visible")
def test_without_a_gpu_the_bench_fails_instead_of_measuring_the_cpu():
    result = _bench("--steps", "1", "--warmup", "0")
    assert result.returncode == 1
    assert "gfx950" in result.stderr
    assert result.stdout == ""
