"""Build recipe of the HIP library (opendressi_amd/libdressi_hip.so) for gfx950.

    python -m opendressi_amd.build

hipcc cross-compiles without a GPU. Flags:
  -ffp-contract=off                         no FMA contraction: coverage, face
                                            ids and depth decisions must be
                                            bit-identical to the reference's
                                            (unfused) CPU arithmetic
  -fhip-fp32-correctly-rounded-divide-sqrt  IEEE division / sqrt
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                            no packed FP32 instructions
"""
from __future__ import annotations

import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libdressi_hip.so")
SOURCES = ["runtime.hip", "raster.hip", "hsr.hip", "aa.hip", "tex.hip", "ds.hip", "ibl.hip", "pbr.hip",
           "graph.hip"]
HEADERS = ["internal.h", "dressi_math.h", "raster_core.h", "soft_clip.h", "hsr_chain.h",
           "aa_core.h", "plan.h", "ibl_core.h"]
ARCH = os.environ.get("DRESSI_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result", "-Wno-unused-value",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.isabs(cand) and os.path.exists(cand) or not os.path.isabs(cand)):
            return cand
    return "hipcc"


def build(verbose: bool = False) -> str:
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    tmp = LIB + ".tmp"
    cmd = [hipcc(), *FLAGS, "-I", os.path.join(ROOT, "include"), "-o", tmp, *srcs]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed building libdressi_hip.so")
    os.replace(tmp, LIB)
    return LIB


def build_graph_test(verbose: bool = False) -> str:
    """The graph-API test program (tests/graph_c1.cpp), linked against the
    library; plain C++ (the graph API header needs no HIP headers)."""
    src = os.path.join(ROOT, "tests", "graph_c1.cpp")
    out_dir = os.path.join(ROOT, "tests", "_bin")
    os.makedirs(out_dir, exist_ok=True)
    exe = os.path.join(out_dir, "graph_c1")
    cmd = ["g++", "-std=c++17", "-O2", "-ffp-contract=off", "-I", os.path.join(ROOT, "include"),
           "-o", exe + ".tmp", src, "-L", PKG, "-ldressi_hip",
           "-Wl,-rpath,$ORIGIN/../../opendressi_amd"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("g++ failed building tests/_bin/graph_c1")
    os.replace(exe + ".tmp", exe)
    return exe


if __name__ == "__main__":
    print(build(verbose=True))
    print(build_graph_test(verbose=True))
