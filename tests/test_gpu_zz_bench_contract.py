"""bench.py keeps the driver's JSON contract: one line on stdout with the
required keys, a roofline object and a cpu_baseline object (a short run on
the GPT-2-small shapes)."""

from __future__ import annotations

import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_json_line():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    print("bench.py --config gpt2s (short run)", flush=True)
    out = subprocess.run(
        [sys.executable, os.path.join(ROOT, "bench.py"), "--config", "gpt2s", "--steps", "3",
         "--warmup", "1", "--no-refresh", "--sparse-steps", "0", "--phase1-steps", "0",
         "--cpu-steps", "1", "--cpu-seconds", "0"],
        cwd=ROOT, capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stderr[-2000:]
    lines = [ln for ln in out.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1, out.stdout
    d = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
                "roofline", "cpu_baseline"):
        assert key in d, key
    assert d["n_gpus"] == 1 and d["steps"] == 3 and d["warmup"] == 1
    assert d["value"] > 0 and d["ms_per_step"] > 0 and d["unit"] == "params/s"
    assert d["dtype"] == "f32" and "workload" in d["config"]
    roof = d["roofline"]
    for key in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert key in roof, key
    assert roof["bound"] in ("hbm", "mfma") and 0 < roof["frac"] < 1
    assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-9
    cpu = d["cpu_baseline"]
    for key in ("value", "unit", "cores", "kind", "sample"):
        assert key in cpu, key
    assert cpu["kind"] in ("reference", "port") and cpu["value"] > 0
