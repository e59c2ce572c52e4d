"""CPU checks of the C ABI boundary: the library loads, exports every entry
point include/dressi_hip.h declares (and the ctypes table binds exactly
those), and the host-only scene builders match the oracle and the
reference's own generators bit for bit. No GPU work is launched here."""
import ctypes as C
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            text = open(os.path.join(ROOT, "include", fn)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names |= set(re.findall(r"\b(dressi_[a-z0-9_]+)\s*\(", text))
    return names


def test_header_declares_entry_points():
    names = _declared()
    assert "dressi_hsr_step" in names and "dressi_rasterize_soft" in names
    assert len(names) > 30


def test_library_exports_every_declared_symbol():
    import opendressi_amd._lib as L
    lib = C.CDLL(L.LIB_PATH)
    missing = [n for n in sorted(_declared()) if not hasattr(lib, n)]
    assert not missing, missing
    assert set(L.EXPORTED) == _declared(), set(L.EXPORTED) ^ _declared()


def _declared_example_helpers():
    """(header, name) of every function declared at namespace scope in
    include/dressi_examples/*.h (the examples' C++ helpers)."""
    pat = re.compile(r"^(?!\s|#|struct|namespace|using|}|template|inline|enum|constexpr|static)"
                     r"[A-Za-z_:<>,\s]*?\b([A-Z][A-Za-z0-9_]*)\(([^;{]*?)\)\s*(const)?\s*;", re.M)
    out = set()
    d = os.path.join(ROOT, "include", "dressi_examples")
    for fn in sorted(os.listdir(d)):
        text = open(os.path.join(d, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        out |= {(fn, m.group(1)) for m in pat.finditer(text)}
    return out


def test_library_defines_every_example_helper():
    """The examples' helper headers (asset, geometry and PBR-graph helpers)
    are implemented in the library, not left to the example programs."""
    import shutil
    import subprocess
    import opendressi_amd._lib as L
    names = _declared_example_helpers()
    assert {n for _, n in names} >= {"LoadObjMesh", "GenerateIcosphere", "BuildPbrShade",
                                     "BuildPbrGBuffer", "BuildPbrIblMaps", "BuildPbrForward"}
    if shutil.which("nm") is None:
        pytest.skip("nm is not installed")
    syms = subprocess.run(["nm", "-DC", "--defined-only", L.LIB_PATH], capture_output=True,
                          text=True, check=True).stdout
    missing = sorted(f"{h}: {n}" for h, n in names if f"dressi_examples::{n}(" not in syms)
    assert not missing, missing


def test_library_is_built_for_gfx950():
    import opendressi_amd._lib as L
    blob = open(L.LIB_PATH, "rb").read()
    assert b"gfx950" in blob


def test_icosphere_matches_oracle(oracle):
    import opendressi_amd as od
    for lvl in range(6):
        p1, f1 = od.icosphere(lvl)
        p2, f2 = oracle.icosphere(lvl)
        assert np.array_equal(p1, p2) and np.array_equal(f1, f2), lvl


def test_icosphere_matches_reference_build():
    from oracle.pyoracle import Reference, have_reference
    if not have_reference():
        pytest.skip("oracle/_ref not built (needs the reference checkout)")
    import opendressi_amd as od
    ref = Reference()
    for lvl in (0, 3, 6):
        p1, f1 = od.icosphere(lvl)
        p2, f2 = ref.icosphere(lvl)
        assert np.array_equal(p1, p2) and np.array_equal(f1, f2), lvl


def test_vertex_faces_and_cameras_match_oracle(oracle):
    import opendressi_amd as od
    pos, faces = od.icosphere(4)
    assert np.array_equal(od.vertex_faces_tex(faces, len(pos)),
                          oracle.vertex_faces_tex(faces, len(pos)))
    eye = [0.7, 0.9, 2.6]
    assert np.array_equal(od.look_at(eye), oracle.look_at(eye))
    assert np.array_equal(od.perspective_vk(0.785398, 1.0, 0.1, 10.0),
                          oracle.perspective_vk(0.785398, 1.0, 0.1, 10.0))
    a = np.arange(16, dtype=np.float32) * 0.37
    b = np.arange(16, dtype=np.float32)[::-1].copy() * 0.11
    assert np.array_equal(od.mat4_mul(a, b), oracle.mat4_mul(a, b))


def test_scene_noise_matches_oracle(oracle):
    import opendressi_amd as od
    a = od.randn(7, 1000)
    b = oracle.randn(7, 1000)
    assert np.array_equal(a, b)
    assert abs(float(a.mean())) < 0.1 and abs(float(a.std()) - 1) < 0.1


def test_workload_shapes():
    import opendressi_amd as od
    sizes = {"c1": (642, 1280, 1), "c2": (2562, 5120, 4), "c4_hsr": (40962, 81920, 4)}
    for name, (nv, nf, nviews) in sizes.items():
        pos, faces, tgt, mvps = od.make_scene(od.WORKLOADS[name])
        assert pos.shape == (nv, 3) and faces.shape == (nf, 3) and mvps.shape == (nviews, 16)
        assert tgt.dtype == np.float32


def test_errors_are_reported_without_a_device():
    import opendressi_amd as od
    from opendressi_amd._lib import lib
    # invalid arguments fail with a status and a message, never a crash
    h = C.c_void_p()
    rc = lib.dressi_ctx_create(-1, C.byref(h))
    assert rc != 0 and lib.dressi_last_error()
    rc = lib.dressi_hsr_create(None, None, None)
    assert rc == -1 and b"bad arguments" in lib.dressi_last_error()
    with pytest.raises(od.DressiError):
        from opendressi_amd._lib import check
        check(lib.dressi_hsr_step(None, 1))


def test_kernel_expf_matches_c_library():
    """The sigmoid's exp (shared host/device code) against the C library expf
    the reference evaluator calls: random inputs over the sigmoid's range,
    special values, and the two hard-rounding inputs where a non-fused range
    reduction differs."""
    import ctypes as C
    import struct

    from opendressi_amd._lib import lib
    libm = C.CDLL("libm.so.6")
    libm.expf.restype = C.c_float
    libm.expf.argtypes = [C.c_float]
    rng = np.random.default_rng(3)
    xs = np.concatenate([rng.uniform(-110, 90, 20000), rng.uniform(-3, 3, 20000),
                         [0.0, -0.0, 88.72, 88.73, -103.9, -104.0, float("inf"), float("-inf"),
                          struct.unpack("<f", struct.pack("<I", 0x42024A2F))[0],  # 0x1.04845ep+5
                          struct.unpack("<f", struct.pack("<I", 0xC27C65D9))[0]]])  # -0x1.f8cbb2p+5
    xs = xs.astype(np.float32)
    bad = [float(x) for x in xs
           if struct.pack("<f", lib.dressi_expf(float(x))) != struct.pack("<f", libm.expf(float(x)))]
    assert not bad, bad[:5]
