"""bench.py's contract with the round driver: one JSON line with the keys the
driver reads (metric, value, unit, n_gpus, steps, warmup, ms_per_step, ...),
the roofline and CPU-baseline objects, and a refusal of more than one GPU
(this build measures one). The refusal runs on the CPU (it is decided before
torch is imported); the JSON line needs the GPU."""
from __future__ import annotations

import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _bench(*args, timeout=600):
    env = dict(os.environ)
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], cwd=ROOT, env=env,
                          capture_output=True, text=True, timeout=timeout)


def test_more_than_one_gpu_is_refused():
    r = _bench("--gpus", "2", timeout=120)
    assert r.returncode == 2, (r.returncode, r.stdout, r.stderr)
    assert "one GPU" in r.stderr and not r.stdout.strip()


@pytest.mark.gpu
def test_json_line_carries_the_drivers_keys(torch_gpu):
    r = _bench("--steps", "5", "--warmup", "3")
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [l for l in r.stdout.splitlines() if l.startswith("{")]
    assert len(lines) == 1, r.stdout
    d = json.loads(lines[0])
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
              "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert k in d, k
    assert d["metric"] == "attention TOPS @ B2 H32 N4096 D128; % of INT8/FP8 MFMA peak"
    assert d["unit"] == "TOPS" and d["n_gpus"] == 1 and d["steps"] == 5 and d["warmup"] == 3
    # Untimed steps before the warm-up make 100 in all before the timed ones.
    assert d["clock_settle_steps"] == 97
    assert d["higher_is_better"] is True and d["vs_baseline"] is None and d["value"] > 0
    assert d["config"]["workload"].startswith("C2 ") and "model" not in d["config"]
    roof = d["roofline"]
    assert roof["bound"] == "mfma" and roof["unit"] == "TFLOP/s" and roof["peak"] == 5000.0
    assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3 and roof["traffic"] > 0
    cpu = d["cpu_baseline"]
    assert cpu["kind"] in ("port", "reference") and cpu["cores"] >= 1 and cpu["value"] > 0
    assert cpu["unit"] == "TOPS" and cpu["sample"]
    # The value is the whole step's rate over the timed steps.
    ops = 4 * 2 * 32 * 4096 * 4096 * 128
    assert abs(d["value"] - ops / (d["ms_per_step"] * 1e-3) / 1e12) <= 0.01 * d["value"]
