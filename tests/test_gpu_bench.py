"""bench.py's JSON line on the GPU: a short run of the metric's configuration
(cfg3) and of an HBM-bound one (cfg4b) in a child process, checked against
the fields the benchmark contract names and against its own arithmetic
(Mpixel/s from the step time, roofline fraction from achieved / peak)."""
import json
import os
import subprocess
import sys

import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu


def run_bench(*args):
    print("bench.py", *args, flush=True)
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--steps", "3", "--warmup", "1",
                          "--settle-ms", "20", "--no-cpu-baseline", *args],
                         cwd=ROOT, capture_output=True, text=True, timeout=110)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-2000:]
    lines = [ln for ln in res.stdout.splitlines() if ln.startswith("{")]
    assert len(lines) == 1, res.stdout[-2000:]
    return json.loads(lines[0])


def check_common(d, pixels):
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline"):
        assert key in d, key
    assert d["n_gpus"] == 1 and d["steps"] == 3 and d["warmup"] == 1
    assert d["unit"] == "Mpixel/s" and d["higher_is_better"] is True and d["scaling"] == "weak"
    assert d["vs_baseline"] is None
    assert "workload" in d["config"]
    # whole-job throughput: the pixels of all batches per step time
    assert d["value"] == pytest.approx(pixels / (d["ms_per_step"] * 1e-3) / 1e6, rel=2e-3)
    r = d["roofline"]
    for key in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert key in r, key
    assert r["frac"] == pytest.approx(r["achieved"] / r["peak"], rel=1e-3)
    assert 0 < r["frac"] < 1


def test_bench_line_cfg3():
    d = run_bench()
    base = json.load(open(os.path.join(ROOT, "BASELINE.json")))
    assert d["metric"] == base["metric"]
    check_common(d, 4 * 256 * 256)
    assert d["dtype"] == "f32"
    r = d["roofline"]
    assert r["bound"] == "mfma" and r["unit"] == "TFLOP/s" and r["peak"] == 157.3
    assert r["traffic"] and r["traffic"] > 0
    assert "cpu_baseline" not in d


def test_bench_line_cfg4b():
    d = run_bench("--config", "cfg4b")
    assert "262144×32" in d["metric"] and "ws=63" in d["metric"]
    check_common(d, 2 * 262144)
    r = d["roofline"]
    assert r["bound"] == "hbm" and r["unit"] == "GB/s" and r["peak"] == 8000.0
