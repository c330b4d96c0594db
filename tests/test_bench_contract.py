"""bench.py's output contract: the last stdout line is one compact JSON
object with the headline fields the driver parses; more than one GPU is
refused before any device work."""

import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _baseline_metric():
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        return json.load(f)["metric"]


def test_more_than_one_gpu_is_refused():
    proc = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                          stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=120)
    assert proc.returncode == 2
    assert "one GPU only" in proc.stderr
    assert proc.stdout == ""


@pytest.mark.gpu
def test_headline_line_on_the_gpu():
    print("bench.py --no-sweep --no-cpu --steps 3 --warmup 1", flush=True)
    proc = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--no-sweep", "--no-cpu",
                           "--steps", "3", "--warmup", "1"],
                          stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr[-2000:]
    last = proc.stdout.strip().splitlines()[-1]
    assert len(last) < 2000
    line = json.loads(last)
    assert line["metric"] == _baseline_metric()
    for key in ("value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
                "vs_baseline", "dtype", "data", "config", "roofline", "native_ms", "numerics"):
        assert key in line, key
    assert line["n_gpus"] == 1 and line["steps"] == 3 and line["warmup"] == 1
    assert line["unit"] == "Gelem/s" and line["dtype"] == "bf16" and line["value"] > 0
    assert "C3" in line["config"]["workload"] and line["config"]["elements"] == 1 << 29
    roof = line["roofline"]
    assert roof["bound"] == "hbm" and roof["unit"] == "GB/s" and roof["peak"] == 8000.0
    assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3
    assert roof["traffic"] is None or roof["traffic"] > 0
    # the timed kernel is the polynomial program whose numerics are stated
    assert line["numerics"]["poly"]["max_abs"] < 0.41
