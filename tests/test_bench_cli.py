"""bench.py's command-line contract on a machine without a GPU: one GPU only
(any other --gpus, or a multi-rank launch, exits with status 2 and says so
before touching a device), and without a GPU it exits with status 2 too
rather than timing a fallback."""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest
import torch

BENCH = Path(__file__).resolve().parents[1] / "bench.py"


def run(*args, env_extra=None):
    env = dict(os.environ, **(env_extra or {}))
    return subprocess.run([sys.executable, str(BENCH), *args], capture_output=True, text=True,
                          timeout=300, env=env)


def test_more_than_one_gpu_is_refused():
    for argv, extra in ((("--gpus", "2"), None), ((), {"WORLD_SIZE": "8"})):
        proc = run(*argv, env_extra=extra)
        assert proc.returncode == 2, proc.stderr[-400:]
        assert "one GPU only" in proc.stderr
        assert proc.stdout == ""


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU exit")
def test_no_gpu_exits_without_a_result_line():
    proc = run("--steps", "1", "--warmup", "0")
    assert proc.returncode == 2
    assert "needs a GPU" in proc.stderr
    assert proc.stdout == ""
