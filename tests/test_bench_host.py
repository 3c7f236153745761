"""CPU tests of bench.py's host-side parts: the CPU baseline's accounting
(FLOPs of the visible pairs, median of the passes, core counts) and the JSON
shape it contributes."""
import os
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)

import bench  # noqa: E402
from inkling_fa4 import testing  # noqa: E402


def test_cpu_baseline_accounting():
    case = testing.ragged_varlen()
    r = bench.cpu_baseline(case, repeats=3, budget_s=60.0)
    assert r["kind"] == "port" and r["unit"] == "TFLOP/s"
    assert len(r["passes_s"]) == 3
    assert r["seconds"] == sorted(r["passes_s"])[1]
    # causal, q == k lengths [64, 33, 17], 8 heads, head_dim 128
    pairs = sum(n * (n + 1) // 2 for n in (64, 33, 17))
    flops = 4.0 * 128 * pairs * 8
    assert abs(r["value"] - flops / r["seconds"] / 1e12) <= 1e-3 * r["value"] + 1e-9
    assert r["cores"] >= 1 and r["cpu_count"] >= 1
    assert r["physical_cores"] is None or 1 <= r["physical_cores"] <= r["cpu_count"]


def test_cpu_baseline_stops_at_the_budget():
    r = bench.cpu_baseline(testing.ragged_varlen(), repeats=3, budget_s=0.0)
    assert len(r["passes_s"]) == 1
