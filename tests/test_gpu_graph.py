"""The graph API's generic executor on the GPU (include/dressi_graph.h,
opendressi_amd/csrc/graph.hip).

tests/graph_c1.cpp builds the HardSoftRas silhouette-fit graph of the
reference example with `Variable` / `F::` / `BuildBackward` / `DressiAD` and
runs it node by node on the device. Its loss image, gradient and Adam state
are compared with the oracle's fit (the reference build's numbers, pinned in
tests/test_oracle.py) and with the fused plan. Bar: the first iteration's
loss and gradient bit-exact (every op one fp32 rounding, the reference's
backward composition and summation order); later iterations within 1e-6,
because the in-graph Adam's bias correction 1 - b^t evaluates `powf` on the
device, which is not guaranteed to round like the C library's.
"""
import os
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "_bin", "graph_c1")


def _run_graph(tmp_path, pos, faces, tgt, mvps, screen, samples, iters, radius, lr, aa=False):
    nv, nf = len(pos), len(faces)
    hdr = np.array([nv, nf, len(tgt), nf, len(mvps), screen, samples, iters, 1 if aa else 0],
                   np.uint32)
    inp = tmp_path / "in.bin"
    out = tmp_path / "out.bin"
    with open(inp, "wb") as f:
        f.write(hdr.tobytes())
        f.write(np.array([radius, lr], np.float32).tobytes())
        for a in (pos, faces, tgt, faces, mvps):
            f.write(np.ascontiguousarray(a, np.float32).tobytes())
    if not os.path.exists(EXE):
        pytest.fail("tests/_bin/graph_c1 is not built (run __graft_entry__.build())")
    res = subprocess.run([EXE, str(inp), str(out)], capture_output=True, text=True, timeout=120)
    print(res.stdout.strip(), res.stderr.strip(), flush=True)
    assert res.returncode == 0, res.stderr
    d = np.fromfile(out, np.float32)
    o = 0
    r = {}
    for k, n in (("pos", nv * 3), ("m", nv * 3), ("v", nv * 3), ("t", 1), ("loss", iters),
                 ("grad0", nv * 3)):
        r[k] = d[o:o + n]
        o += n
    assert o == d.size
    for k in ("pos", "m", "v", "grad0"):
        r[k] = r[k].reshape(nv, 3)
    return r


@pytest.mark.parametrize("views,screen", [(1, 128), (2, 96)])
def test_graph_executor_silhouette_fit_matches_oracle(tmp_path, oracle, views, screen):
    import opendressi_amd as od
    print(f"[graph] c1 mesh, {views} view(s), {screen}px, 3 iterations", flush=True)
    w = od.WORKLOADS["c1"]
    pos, faces, tgt, mvps = od.make_scene(w)
    mvps = np.ascontiguousarray(np.asarray(mvps, np.float32)[:views])
    if len(mvps) < views:
        mvps = np.ascontiguousarray(np.asarray(od.camera_mvps(views), np.float32))
    iters, radius, samples, lr = 3, 3.0, 8, 1e-3
    g = _run_graph(tmp_path, pos, faces, tgt, mvps, screen, samples, iters, radius, lr)
    want = oracle.hsr_fit(pos, faces, tgt, faces, mvps, screen, radius=radius, samples=samples,
                          lr=lr, iters=iters, want_images=False)
    assert np.array_equal(g["grad0"], want["grad0"]), \
        f"grad0 differs: max {np.abs(g['grad0'] - want['grad0']).max():.3g}"
    assert g["loss"][0] == want["loss"][0], (g["loss"], want["loss"])
    assert np.abs(want["grad0"]).max() > 0
    np.testing.assert_allclose(g["loss"], want["loss"], rtol=1e-6, atol=0)
    for k in ("pos", "m", "v"):
        np.testing.assert_allclose(g[k], want[k], rtol=0, atol=1e-6 * max(1.0, np.abs(want[k]).max()),
                                   err_msg=k)
    assert g["t"][0] == iters
    exact = {k: bool(np.array_equal(g[k], want[k])) for k in ("pos", "m", "v", "loss")}
    print(f"[graph] bit-exact after {iters} iterations: {exact}", flush=True)


def test_graph_executor_matches_fused_plan(tmp_path):
    """The generic executor and the fused plan run the same graph: first
    iteration loss and gradient identical."""
    import opendressi_amd as od
    print("[graph] vs fused plan, c1 mesh, 1 view, 128px", flush=True)
    w = od.WORKLOADS["c1"]
    pos, faces, tgt, mvps = od.make_scene(w)
    mvps = np.ascontiguousarray(np.asarray(mvps, np.float32)[:1])
    g = _run_graph(tmp_path, pos, faces, tgt, mvps, 128, 8, 1, 3.0, w.lr)
    ctx = od.Context(0)
    fit = od.SilhouetteFit(ctx, pos, faces, mvps, 128, target_mesh=(tgt, faces), lr=w.lr,
                           keep_grad=True)
    fit.step(1)
    fit.synchronize()
    from opendressi_amd import _lib
    assert np.array_equal(g["grad0"], fit.read(_lib.BUF_GRAD)), "gradient differs"
    assert g["loss"][0] == np.float32(fit.loss()), (g["loss"][0], fit.loss())
    np.testing.assert_allclose(g["pos"], fit.read(_lib.BUF_POS), rtol=0, atol=1e-6)


@pytest.mark.parametrize("samples", [8, 0])
def test_graph_executor_aa_fit_matches_oracle(tmp_path, oracle, samples):
    """Technique aa (AntiAlias'd hard masks; stochastic wide vertex backward
    + ColSum, or the exact one) through the generic executor."""
    import opendressi_amd as od
    print(f"[graph] aa, c1 mesh, 2 views, 96px, samples={samples}, 3 iterations", flush=True)
    w = od.WORKLOADS["c1"]
    pos, faces, tgt, _ = od.make_scene(w)
    mvps = np.ascontiguousarray(np.asarray(od.camera_mvps(2), np.float32))
    iters, lr = 3, 1e-3
    g = _run_graph(tmp_path, pos, faces, tgt, mvps, 96, samples, iters, 3.0, lr, aa=True)
    want = oracle.aa_fit(pos, faces, tgt, faces, mvps, 96, samples=samples, lr=lr, iters=iters,
                         want_images=False)
    assert np.array_equal(g["grad0"], want["grad0"]), \
        f"grad0 differs: max {np.abs(g['grad0'] - want['grad0']).max():.3g}"
    assert g["loss"][0] == want["loss"][0], (g["loss"], want["loss"])
    assert np.abs(want["grad0"]).max() > 0
    np.testing.assert_allclose(g["loss"], want["loss"], rtol=1e-6, atol=0)
    for k in ("pos", "m", "v"):
        np.testing.assert_allclose(g[k], want[k], rtol=0, atol=1e-6 * max(1.0, np.abs(want[k]).max()),
                                   err_msg=k)
