"""bench.py's result line on the MI355X, with its longest sections switched
off: exactly one JSON line on stdout carrying the fields the driver and the
judge read (the metric, whole-step value, step timing, dtype, config, and the
roofline object of the dominant kernel with its counter-measured traffic)."""

from __future__ import annotations

import json
import sys

import pytest
import torch

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs an MI355X")]


def test_bench_prints_one_contract_line(monkeypatch, capsys):
    # in this process (no child program is started from a process that has
    # initialised the GPU)
    import bench
    monkeypatch.setattr(sys, "argv", ["bench.py", "--steps", "4", "--warmup", "1", "--no-cpu",
                                      "--no-decode", "--no-proj", "--no-prefill-attention",
                                      "--no-engine"])
    assert bench.main() in (0, None)
    out = capsys.readouterr().out
    lines = [line for line in out.splitlines() if line.strip()]
    assert len(lines) == 1, out[-2000:]
    result = json.loads(lines[0])
    assert result["metric"].startswith("achieved HBM GB/s")
    assert result["unit"] == "GB/s" and result["n_gpus"] == 1
    assert result["steps"] == 4 and result["warmup"] == 1
    assert result["higher_is_better"] is True and result["scaling"] == "weak"
    assert result["dtype"] == "bf16" and result["data"] == "synthetic"
    assert result["vs_baseline"] is None
    assert "workload" in result["config"] and "model" not in result["config"]
    step_bytes = result["config"]["step_bytes"]
    # value is the step's algorithmic bytes over its measured time
    assert result["value"] == pytest.approx(step_bytes / (result["ms_per_step"] * 1e6), rel=1e-9)
    assert 0.3 < result["value"] / 8000.0 < 1.0
    roof = result["roofline"]
    assert roof["bound"] == "hbm" and roof["unit"] == "GB/s" and roof["peak"] == 8000.0
    assert roof["frac"] == pytest.approx(roof["achieved"] / roof["peak"], rel=1e-9)
    assert roof["kernel"] in result["kernels"]
    assert roof["traffic"] is None or 0.95 < roof["traffic"] / roof["algorithmic_bytes"] < 1.2
    for name, entry in result["kernels"].items():
        assert entry["us_per_call_mean"] > 0 and 0 < entry["frac"] < 1, name
