"""bench.py's bench.json record against the reference's
(examples/common/bench.cpp:145-209, examples/silhouette_optimization/
run.cpp:573-587, 676-702): key order and types, the upper median, the
warm-up split and the first-build time. CPU only."""
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402

# the reference record's keys in the order it writes them: BenchRecord's
# constructor, addPacking, then run.cpp's adds
REF_KEYS = ["example", "device", "platform", "os", "cpu", "cpu_cores", "ram_gb", "funcs",
            "substages", "stages", "technique", "screen", "views", "iters", "samples", "peels",
            "single_view", "median_ms_per_iter", "warmup_excluded", "warmup_ms",
            "first_build_ms", "mean_iou", "loss_drop"]
TYPES = {"example": str, "device": str, "platform": str, "os": str, "cpu": str, "cpu_cores": int,
         "ram_gb": float, "funcs": int, "substages": int, "stages": int, "technique": str,
         "screen": int, "views": int, "iters": int, "samples": int, "peels": int,
         "single_view": bool, "median_ms_per_iter": float, "warmup_excluded": int,
         "warmup_ms": float, "first_build_ms": float, "mean_iou": float, "loss_drop": float}


def test_upper_median():
    assert bench.median_upper([]) == 0.0
    assert bench.median_upper([5.0]) == 5.0
    assert bench.median_upper([4.0, 1.0, 3.0, 2.0]) == 3.0  # s[n / 2], not the mean of 2, 3
    assert bench.median_upper([3.0, 1.0, 2.0]) == 2.0


def test_record_keys_types_and_definitions():
    iters = 100
    ms = [50.0] + [2.0] * 19 + [1.0 + 0.01 * i for i in range(80)]
    rec = bench.bench_fields("MI355X", "cpu", 16, 31.4159, 5, "hardsoftras", 2048, 4, iters, ms,
                             0.95, 0.2, 0.05)
    assert list(rec) == REF_KEYS
    for k, t in TYPES.items():
        assert isinstance(rec[k], t), (k, type(rec[k]))
    # warm-up: the first min(20, iters / 2) iterations; the first is the build
    assert rec["warmup_excluded"] == 20
    assert rec["first_build_ms"] == 50.0
    steady = sorted(ms[20:])
    assert rec["median_ms_per_iter"] == round(steady[len(steady) // 2], 6)
    assert rec["warmup_ms"] == round(sum(ms[:20]) - 20 * rec["median_ms_per_iter"], 1)
    assert rec["loss_drop"] == 4.0
    assert rec["single_view"] is False
    # a short run: warm-up is iters / 2
    short = bench.bench_fields("d", "c", 1, 1.0, 5, "aa", 64, 1, 10, [1.0] * 10, 1.0, 1.0, 1.0)
    assert short["warmup_excluded"] == 5 and short["single_view"] is True
    json.dumps(rec)  # serialisable as written
