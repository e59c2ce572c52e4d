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
           "graph.hip", "executor.hip", "builders.hip", "route.hip"]
# host-only sources (the examples' asset, geometry and PBR-graph helpers), built with g++;
# zlib is linked for their deflate streams
HOST_SOURCES = ["assets.cpp", "jpeg.cpp", "geometry.cpp", "pbr_graph.cpp"]
HEADERS = ["internal.h", "dressi_math.h", "raster_core.h", "soft_clip.h", "hsr_chain.h",
           "aa_core.h", "plan.h", "ibl_core.h", "graph_ir.h", "route.h", "libm_f32.h",
           "libm_pow5_table.h", "image_codecs.h"]
ARCH = os.environ.get("DRESSI_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result", "-Wno-unused-value",
]
OBJ_DIR = os.path.join(PKG, "_build")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.isabs(cand) and os.path.exists(cand) or not os.path.isabs(cand)):
            return cand
    return "hipcc"


def _run(cmd, verbose, what):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed building {what}")


def build(verbose: bool = False) -> str:
    """Every source compiled (in parallel, one object each), then linked."""
    from concurrent.futures import ThreadPoolExecutor
    os.makedirs(OBJ_DIR, exist_ok=True)
    inc = ["-I", os.path.join(ROOT, "include")]
    objs = [os.path.join(OBJ_DIR, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    host_objs = [os.path.join(OBJ_DIR, os.path.splitext(s)[0] + ".o") for s in HOST_SOURCES]
    jobs = min(len(SOURCES), max(1, min(os.cpu_count() or 1, 8)))
    with ThreadPoolExecutor(jobs) as ex:
        futs = [ex.submit(_run, [hipcc(), *FLAGS, *inc, "-c", os.path.join(CSRC, s), "-o", o],
                          verbose, s) for s, o in zip(SOURCES, objs)]
        futs += [ex.submit(_run, ["g++", "-O2", "-std=c++17", "-fPIC", "-ffp-contract=off", *inc,
                                  "-c", os.path.join(CSRC, s), "-o", o], verbose, s)
                 for s, o in zip(HOST_SOURCES, host_objs)]
        for f in futs:
            f.result()
    tmp = LIB + ".tmp"
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, *host_objs,
          "-lz", "-lhiprtc"], verbose, "libdressi_hip.so")
    os.replace(tmp, LIB)
    return LIB


def build_graph_test(verbose: bool = False) -> str:
    """The test programs (tests/graph_c1.cpp, graph_ops.cpp, graph_tex.cpp, graph_pbr.cpp over the
    graph API, tests/assets_cli.cpp over the examples' helpers), linked
    against the library; plain C++ (those headers need no HIP headers)."""
    out_dir = os.path.join(ROOT, "tests", "_bin")
    os.makedirs(out_dir, exist_ok=True)
    exe = ""
    for name in ("graph_c1", "graph_ops", "graph_tex", "graph_pbr", "assets_cli"):
        src = os.path.join(ROOT, "tests", name + ".cpp")
        exe = os.path.join(out_dir, name)
        cmd = ["g++", "-std=c++17", "-O2", "-ffp-contract=off", "-I", os.path.join(ROOT, "include"),
               "-o", exe + ".tmp", src, "-L", PKG, "-ldressi_hip",
               "-Wl,-rpath,$ORIGIN/../../opendressi_amd"]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            sys.stderr.write(res.stdout + res.stderr)
            raise RuntimeError(f"g++ failed building tests/_bin/{name}")
        os.replace(exe + ".tmp", exe)
    # the host build of the library's C-library-exact float functions
    # (csrc/libm_f32.h), checked against the host C library by tests/test_libm.py
    exe = os.path.join(out_dir, "libm_check")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-O2", "-std=c++17", "-ffp-contract=off",
           "-o", exe + ".tmp", os.path.join(ROOT, "tests", "libm_check.cpp")]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed building tests/_bin/libm_check")
    os.replace(exe + ".tmp", exe)
    return out_dir


if __name__ == "__main__":
    print(build(verbose=True))
    print(build_graph_test(verbose=True))
