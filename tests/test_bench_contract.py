"""bench.py's output contract: one JSON line whose keys the round driver reads (metric,
value, unit, n_gpus, steps, warmup, ms_per_step, higher_is_better, scaling,
vs_baseline, dtype, data, config, roofline, cpu_baseline, settle), the metric named as in
BASELINE.json, and a refusal with exit status 2 for more than one GPU. The GPU case
runs bench.py as a child process at a few steps."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")

KEYS = {"metric": str, "value": float, "unit": str, "n_gpus": int, "steps": int, "warmup": int,
        "ms_per_step": float, "higher_is_better": bool, "scaling": str, "dtype": str, "data": str,
        "config": dict, "roofline": dict}
ROOF_KEYS = ("bound", "achieved", "peak", "unit", "frac", "traffic")


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, BENCH, "--gpus", "2"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def run_bench(*args):
    r = subprocess.run([sys.executable, "-u", BENCH, *args], capture_output=True, text=True, timeout=300,
                       cwd=ROOT)
    assert r.returncode == 0, r.stderr[-2000:]
    return json.loads(r.stdout.strip().splitlines()[-1])


def check_line(d, steps, warmup, rows):
    for k, t in KEYS.items():
        assert k in d, k
        assert isinstance(d[k], t) or (t is float and isinstance(d[k], int)), (k, d[k])
    assert "vs_baseline" in d and "cpu_baseline" in d
    assert d["n_gpus"] == 1 and d["steps"] == steps and d["warmup"] == warmup
    assert d["higher_is_better"] is True and d["scaling"] in ("weak", "strong")
    assert d["value"] > 0 and d["ms_per_step"] > 0
    # value is the whole job's rows per second at the timed ms_per_step
    assert abs(d["value"] - rows / (d["ms_per_step"] / 1e3)) <= 1e-3 * d["value"] + 0.1
    assert "workload" in d["config"]
    roof = d["roofline"]
    for k in ROOF_KEYS:
        assert k in roof, k
    assert roof["bound"] in ("hbm", "mfma")
    assert roof["achieved"] > 0 and roof["peak"] > 0
    assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) <= 1e-3


@pytest.mark.gpu
def test_bench_line_small_and_metric_workload():
    d = run_bench("--workload", "small_b1", "--steps", "5", "--warmup", "2", "--layers", "1",
                  "--no-cpu-baseline")
    check_line(d, 5, 2, 1)
    assert d["config"]["workload"] == "small_b1" and d["cpu_baseline"] is None
    d = run_bench("--steps", "5", "--warmup", "2", "--layers", "1", "--no-cpu-baseline", "--settle-ms", "20")
    check_line(d, 5, 2, 8)
    # the clock-settle phase ran untimed steps for at least the requested time
    assert d["settle"]["ms"] >= 20 and d["settle"]["steps"] >= 16
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        assert d["metric"] == json.load(f)["metric"]
    assert d["config"]["workload"] == "glm5_moe_decode_b8" and d["config"]["batch"] == 8
    assert d["roofline"]["bound"] == "hbm" and d["roofline"]["unit"] == "GB/s"
