"""bench.py's output contract: one JSON line with the driver's fields, the
roofline of the dominant kernel and the CPU baseline (GPU), and a refusal with
a message for more than one GPU (CPU)."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, BENCH, "--gpus", "2"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


@pytest.mark.gpu
def test_bench_line_has_every_field():
    """A short config-3 run (a few steps, a 2-second CPU sample) prints the
    contract's keys with values of the right kinds."""
    print("bench contract: config 3, 3 steps", flush=True)
    r = subprocess.run([sys.executable, BENCH, "--config", "3", "--steps", "3", "--warmup", "1",
                        "--cpu-seconds", "2", "--no-gemm-ceiling"],
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [l for l in r.stdout.splitlines() if l.startswith("{")]
    assert len(lines) == 1
    d = json.loads(lines[0])
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
              "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert k in d, k
    assert d["n_gpus"] == 1 and d["steps"] == 3 and d["warmup"] == 1
    assert d["value"] > 0 and d["ms_per_step"] > 0 and d["higher_is_better"] is True
    assert d["dtype"] == "bf16" and d["vs_baseline"] is None
    assert d["config"]["workload"].startswith("cocktail B16 H12 L1024 d64")
    roof = d["roofline"]
    assert roof["bound"] in ("hbm", "mfma") and roof["unit"] in ("GB/s", "TFLOP/s")
    assert 0 < roof["achieved"] < roof["peak"] and abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3
    assert "traffic" in roof
    cpu = d["cpu_baseline"]
    assert cpu["value"] > 0 and cpu["cores"] >= 1 and cpu["kind"] in ("port", "reference")
    assert cpu["unit"] == d["unit"] and cpu["sample"]
