"""The library's single-precision atanf / atan2f / acosf / pow5f
(opendressi_amd/csrc/libm_f32.h) against the host C library, on the CPU.

The reference evaluates its equirect mapping with the C library's atan2f and
acosf (src/core/ibl_math.h:41-47) and its Schlick factors with powf(x, 5)
(src/core/f_ops.cpp:3350-3409, examples/common/pbr_graph.cpp); the device
uses these restatements so that uv coordinates, bilinear weights and shading
match the reference's bits. tests/libm_check.cpp compiles the same header for
the host and compares every result bit for bit (strided sweeps of the whole
domains, random and structured atan2f pairs, every entry of the pow5f miss
table); the full sweeps (stride 1) were run when the header was written.
"""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "_bin", "libm_check")


def test_libm_f32_matches_host_c_library():
    assert os.path.exists(EXE), "tests/_bin/libm_check is not built (run __graft_entry__.build())"
    res = subprocess.run([EXE, "4"], capture_output=True, text=True, timeout=600)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "mismatches: 0" in res.stdout
