"""Writes tests/golden/bench_json_keys.json: the key order, value kinds and
decimal places of the silhouette example's bench.json record, read as text
from the reference's writer and call site:

  examples/common/bench.cpp:164-210   BenchRecord: example, device, platform,
                                      os, cpu, cpu_cores, ram_gb; add(key,
                                      double, precision) in fixed notation;
                                      addPacking: funcs, substages, stages
  examples/common/bench.h:32-35       the default precision of add(double)
  examples/silhouette_optimization/run.cpp:686-703   the example's keys

    python tests/golden/make_bench_keys.py
"""
from __future__ import annotations

import json
import os
import re

REF = "/root/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "bench_json_keys.json")


def main() -> None:
    bench_cpp = open(os.path.join(REF, "examples/common/bench.cpp")).read()
    bench_h = open(os.path.join(REF, "examples/common/bench.h")).read()
    run_cpp = open(os.path.join(REF, "examples/silhouette_optimization/run.cpp")).read()
    default_prec = int(re.search(r"add\(const std::string& key, double value, int precision = (\d+)\)",
                                 bench_h).group(1))
    keys, kinds, prec = [], {}, {}

    def put(k, kind, p=None):
        keys.append(k)
        kinds[k] = kind
        if p is not None:
            prec[k] = p

    ctor = bench_cpp[bench_cpp.index("BenchRecord::BenchRecord"):bench_cpp.index("void BenchRecord::add")]
    for k in re.findall(r'\\"(\w+)\\":\\"\{\}\\"', ctor):
        put(k, "str")
    for k, val in re.findall(r'add\("(\w+)",\s*([^;]+)\);', ctor):
        if "int64_t" in val:
            put(k, "int")
        elif "RamGb" in val:
            put(k, "float", int(val.rsplit(",", 1)[1].strip(" )")))
        else:
            put(k, "str")
    packing = bench_cpp[bench_cpp.index("void BenchRecord::addPacking"):]
    for k in re.findall(r'add\("(\w+)", \w+\);', packing[:packing.index("}")]):
        put(k, "int")
    block = run_cpp[run_cpp.index('BenchRecord rec("silhouette_optimization"'):]
    block = block[:block.index("rec.save")]
    for k, val in re.findall(r'rec\.add\("(\w+)",\s*(.*?)\);', block, flags=re.S):
        val = " ".join(val.split())
        if val.startswith("int64_t("):
            put(k, "int")
        elif val.startswith("double(") or val.endswith("_ms") or val.endswith(", 1") or "ms" in val:
            m = re.search(r",\s*(\d+)$", val)
            put(k, "float", int(m.group(1)) if m else default_prec)
        elif val == "opt.technique":
            put(k, "str")
        else:
            put(k, "bool")
    with open(OUT, "w") as f:
        json.dump({"keys": keys, "kinds": kinds, "precision": prec}, f, indent=1)
        f.write("\n")
    print(OUT, keys)


if __name__ == "__main__":
    main()
