"""bench.py's bench.json record against the reference's
(examples/common/bench.cpp:145-209, examples/silhouette_optimization/
run.cpp:573-587, 676-702): key order and types, the upper median, the
warm-up split and the first-build time. CPU only."""
import json
import os
import re
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402

# key order, value kinds and decimals as the reference's writer and call
# site declare them (tests/golden/bench_json_keys.json, written from
# examples/common/bench.{h,cpp} and run.cpp by tests/golden/make_bench_keys.py)
with open(os.path.join(ROOT, "tests", "golden", "bench_json_keys.json")) as _f:
    GOLDEN = json.load(_f)
REF_KEYS = GOLDEN["keys"]
TYPES = {k: {"str": str, "int": int, "float": float, "bool": bool}[v]
         for k, v in GOLDEN["kinds"].items()}


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
    assert rec["median_ms_per_iter"] == steady[len(steady) // 2]
    assert rec["warmup_ms"] == sum(ms[:20]) - 20 * rec["median_ms_per_iter"]
    assert rec["loss_drop"] == 4.0
    assert rec["single_view"] is False
    # a short run: warm-up is iters / 2
    short = bench.bench_fields("d", "c", 1, 1.0, 5, "aa", 64, 1, 10, [1.0] * 10, 1.0, 1.0, 1.0)
    assert short["warmup_excluded"] == 5 and short["single_view"] is True


def test_record_text_matches_the_reference_format():
    ms = [12.345] + [1.0] * 19 + [0.123456 + 1e-4 * i for i in range(30)]
    rec = bench.bench_fields("AMD Instinct MI355X", "x86", 16, 31.4159, 5, "hardsoftras", 2048, 4,
                             50, ms, 0.955555, 0.2, 0.05)
    text = bench.bench_json_text(rec)
    assert text.endswith("}\n") and '", "' not in text and '": ' not in text
    parsed = json.loads(text)
    assert list(parsed) == REF_KEYS
    for k, t in TYPES.items():
        assert isinstance(parsed[k], t), (k, type(parsed[k]))
    # reals in fixed notation with the reference's decimals
    for k, d in GOLDEN["precision"].items():
        m = re.search(rf'"{k}":(-?\d+)\.(\d+)[,}}]', text)
        assert m and len(m.group(2)) == d, (k, text)
    assert '"median_ms_per_iter":0.1250,' in text and '"mean_iou":0.9556,' in text
    assert '"ram_gb":31.4,' in text and '"first_build_ms":12.3,' in text
    assert '"single_view":false,' in text and '"stages":1,' in text
