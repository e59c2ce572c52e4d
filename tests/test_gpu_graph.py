"""DressiAD on the GPU through the graph API (include/dressi/dressi.h).

tests/graph_c1.cpp builds the silhouette-fit example graph of the reference
(examples/silhouette_optimization/run.cpp:229-437) with Variable / F:: /
DressiAD, sends its static images as CpuImage and steps it with
execStepWithSendsAndRecvImgsStacked. With PackingMode::RSP the executor
recognises the example graph and runs it on the fused silhouette plan
(getPlanName() "fused:hardsoftras" / "fused:aa", getStageCount() 1); with
PackingMode::Naive, or when the graph is not the example's (regulariser
weights other than 0), the generic executor runs it function by function.

Bars: the fused route reproduces the oracle's whole trajectory bit for bit
(positions, Adam moments, every loss, the first gradient, the last
predictions and the targets); the generic executor reproduces the first
iteration bit for bit (loss and gradient: every op one fp32 rounding, the
reference's backward composition and summation order) and later ones within
1e-6, because the in-graph Adam's bias correction 1 - b^t evaluates powf on
the device, which need not round like the C library's.
"""
import os
import re
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "_bin", "graph_c1")
GOLDEN = os.path.join(ROOT, "tests", "golden")


def _run_graph(tmp_path, pos, faces, tgt, mvps, screen, samples, iters, radius, lr, aa=False,
               naive=False, regs=False, w_lap=0.0, w_nrm=0.0, peels=1, no_rebuild=False,
               regrow=False, timeout=120, env=None):
    nv, nf, n = len(pos), len(faces), len(mvps)
    hdr = np.array([nv, nf, len(tgt), nf, n, screen, samples, iters, 1 if aa else 0,
                    1 if naive else 0, 1 if regs else 0, peels, 1 if no_rebuild else 0,
                    1 if regrow else 0], np.uint32)
    inp = tmp_path / "in.bin"
    out = tmp_path / "out.bin"
    with open(inp, "wb") as f:
        f.write(hdr.tobytes())
        f.write(np.array([radius, lr, w_lap, w_nrm], np.float32).tobytes())
        for a in (pos, faces, tgt, faces, mvps):
            f.write(np.ascontiguousarray(a, np.float32).tobytes())
    if not os.path.exists(EXE):
        pytest.fail("tests/_bin/graph_c1 is not built (run __graft_entry__.build())")
    res = subprocess.run([EXE, str(inp), str(out)], capture_output=True, text=True,
                         timeout=timeout, env=None if env is None else {**os.environ, **env})
    print(res.stdout.strip(), res.stderr.strip(), flush=True)
    assert res.returncode == 0, res.stderr
    m = re.search(r"plan=(\S+) stages=(\d+) substages=(\d+) funcs=(\d+)", res.stdout)
    assert m, res.stdout
    d = np.fromfile(out, np.float32)
    o = 0
    r = {"plan": m.group(1), "stages": int(m.group(2)), "substages": int(m.group(3)),
         "funcs": int(m.group(4))}
    for k, cnt in (("pos", nv * 3), ("m", nv * 3), ("v", nv * 3), ("t", 1), ("loss", iters),
                   ("grad0", nv * 3), ("pred", n * screen * screen),
                   ("target", n * screen * screen), ("kernels", iters), ("ms", iters)):
        r[k] = d[o:o + cnt]
        o += cnt
    assert o == d.size
    for k in ("pos", "m", "v", "grad0"):
        r[k] = r[k].reshape(nv, 3)
    for k in ("pred", "target"):
        r[k] = r[k].reshape(n, screen, screen)
    return r


def _scene(name, views=None):
    import opendressi_amd as od
    w = od.WORKLOADS[name]
    pos, faces, tgt, mvps = od.make_scene(w)
    if views is not None:
        mvps = np.ascontiguousarray(np.asarray(od.camera_mvps(views), np.float32))
    return w, pos, faces, tgt, mvps


def _fit(oracle, aa, pos, faces, tgt, mvps, screen, samples, lr, iters, images=True):
    fit = oracle.aa_fit if aa else oracle.hsr_fit
    kw = {} if aa else {"radius": 3.0}
    return fit(pos, faces, tgt, faces, mvps, screen, samples=samples, lr=lr, iters=iters,
               want_images=images, **kw)


@pytest.mark.parametrize("aa", [False, True], ids=["hardsoftras", "aa"])
@pytest.mark.parametrize("views,screen", [(1, 128), (2, 96)])
def test_fused_route_matches_oracle(tmp_path, oracle, aa, views, screen):
    """RSP packing: the example graph runs on the fused plan, bit-exact."""
    print(f"[graph] c1 mesh, {'aa' if aa else 'hsr'}, {views} view(s), {screen}px, RSP",
          flush=True)
    _, pos, faces, tgt, mvps = _scene("c1", views)
    iters, samples, lr = 4, 8, 1e-3
    g = _run_graph(tmp_path, pos, faces, tgt, mvps, screen, samples, iters, 3.0, lr, aa=aa)
    assert g["plan"] == ("fused:aa" if aa else "fused:hardsoftras")
    assert g["stages"] == 1 and g["substages"] == 5
    want = _fit(oracle, aa, pos, faces, tgt, mvps, screen, samples, lr, iters, images=False)
    assert np.abs(want["grad0"]).max() > 0
    for k in ("grad0", "pos", "m", "v", "loss"):
        assert np.array_equal(g[k], want[k]), \
            f"{k}: max |d| {np.abs(g[k] - want[k]).max():.3g}"
    assert g["t"][0] == iters
    # the last iteration's predictions and the targets against a one-step
    # oracle fit from the final state's predecessor: the targets are static
    one = _fit(oracle, aa, pos, faces, tgt, mvps, screen, samples, lr, 1)
    assert np.array_equal(g["target"], one["target"])


@pytest.mark.parametrize("views,screen", [(1, 128), (2, 96)])
def test_generic_executor_matches_oracle(tmp_path, oracle, views, screen):
    """Naive packing: one kernel per function, no fused plan."""
    print(f"[graph] c1 mesh, hsr, {views} view(s), {screen}px, Naive", flush=True)
    _, pos, faces, tgt, mvps = _scene("c1", views)
    iters, samples, lr = 3, 8, 1e-3
    g = _run_graph(tmp_path, pos, faces, tgt, mvps, screen, samples, iters, 3.0, lr, naive=True)
    assert g["plan"] == "generic"
    assert g["stages"] == g["substages"] > 100
    want = _fit(oracle, False, pos, faces, tgt, mvps, screen, samples, lr, iters)
    assert np.array_equal(g["grad0"], want["grad0"]), \
        f"grad0 differs: max {np.abs(g['grad0'] - want['grad0']).max():.3g}"
    assert g["loss"][0] == want["loss"][0], (g["loss"], want["loss"])
    np.testing.assert_allclose(g["loss"], want["loss"], rtol=1e-6, atol=0)
    for k in ("pos", "m", "v"):
        np.testing.assert_allclose(g[k], want[k], rtol=0,
                                   atol=1e-6 * max(1.0, np.abs(want[k]).max()), err_msg=k)
    assert g["t"][0] == iters
    assert np.array_equal(g["target"], want["target"])


def test_generic_rsp_fuses_elementwise_runs(tmp_path, oracle):
    """RSP on a graph the route does not take (regulariser weights > 0):
    the generic executor with fused elementwise stages; its first
    iteration's data gradient and loss are the oracle's (the regularisers
    change only the update)."""
    _, pos, faces, tgt, mvps = _scene("c1", 1)
    iters, samples, lr, screen = 2, 8, 1e-3, 96
    print("[graph] c1 mesh, hsr, regularisers 0.15 / 0.4, RSP", flush=True)
    g = _run_graph(tmp_path, pos, faces, tgt, mvps, screen, samples, iters, 3.0, lr, regs=True,
                   w_lap=0.15, w_nrm=0.4)
    assert g["plan"] == "generic"
    naive = _run_graph(tmp_path, pos, faces, tgt, mvps, screen, samples, iters, 3.0, lr,
                       naive=True, regs=True, w_lap=0.15, w_nrm=0.4)
    assert g["stages"] < naive["stages"] // 2, (g["stages"], naive["stages"])
    want = _fit(oracle, False, pos, faces, tgt, mvps, screen, samples, lr, 1, images=False)
    assert np.array_equal(g["grad0"], want["grad0"])
    assert g["loss"][0] == want["loss"][0]
    # fused and one-kernel-per-function runs compute the same floats
    for k in ("pos", "m", "v", "loss", "grad0"):
        assert np.array_equal(g[k], naive[k]), k
    assert np.isfinite(g["pos"]).all()
    plain = _fit(oracle, False, pos, faces, tgt, mvps, screen, samples, lr, iters, images=False)
    assert np.abs(g["pos"] - plain["pos"]).max() > 0  # the regularisers moved it


def test_example_with_zero_regulariser_weights_takes_the_route(tmp_path, oracle):
    """The reference example as run with --laplacian=0 --normal=0."""
    _, pos, faces, tgt, mvps = _scene("c1", 1)
    iters, samples, lr, screen = 3, 8, 1e-3, 96
    g = _run_graph(tmp_path, pos, faces, tgt, mvps, screen, samples, iters, 3.0, lr, regs=True)
    assert g["plan"] == "fused:hardsoftras"
    want = _fit(oracle, False, pos, faces, tgt, mvps, screen, samples, lr, iters, images=False)
    for k in ("pos", "m", "v", "loss", "grad0"):
        assert np.array_equal(g[k], want[k]), k


@pytest.mark.parametrize("peels", [2, 3])
def test_depth_peels_through_dressi_ad(tmp_path, peels):
    """The example's --peels K graph (run.cpp:302-343: K RasterizeSoft layers,
    each rejecting fragments at or in front of the previous layer's shifted
    depth, Eq. 6 composition) through DressiAD, against the reference build's
    own fit (tests/golden/hsr_peel<K>_*.npz): the first iteration's loss and
    gradient bit for bit, the predictions and targets bit for bit, the later
    iterations within 1e-6 (device powf in the in-graph Adam)."""
    with np.load(os.path.join(GOLDEN, f"hsr_peel{peels}_ico3_2view_96px_3it.npz")) as z:
        gold = {k: z[k] for k in z.files}
    screen, iters = int(gold["in_cfg"][0]), int(gold["in_cfg"][1])
    print(f"[graph] peels {peels}: ico3, 2 views, {screen}px, {iters} iterations, RSP",
          flush=True)
    g = _run_graph(tmp_path, gold["in_pos"], gold["in_faces"], gold["in_tgt_pos"],
                   gold["in_mvps"], screen, 8, iters, 3.0, 1e-3, peels=peels)
    assert g["plan"] == "generic"
    assert np.array_equal(g["grad0"], gold["out_grad0"]), \
        f"grad0 differs: max {np.abs(g['grad0'] - gold['out_grad0']).max():.3g}"
    assert g["loss"][0] == gold["out_loss"][0], (g["loss"], gold["out_loss"])
    np.testing.assert_allclose(g["loss"], gold["out_loss"], rtol=1e-6, atol=0)
    for k in ("pos", "m", "v"):
        np.testing.assert_allclose(g[k], gold["out_" + k], rtol=0,
                                   atol=1e-6 * max(1.0, np.abs(gold["out_" + k]).max()),
                                   err_msg=k)
    assert np.array_equal(g["target"], gold["out_target"])
    one = _run_graph(tmp_path, gold["in_pos"], gold["in_faces"], gold["in_tgt_pos"],
                     gold["in_mvps"], screen, 8, 1, 3.0, 1e-3, peels=1)
    assert not np.array_equal(one["grad0"], g["grad0"])  # the extra layers count


def test_compiled_fused_programs_match_the_interpreter(tmp_path):
    """The generic executor's fused elementwise programs compiled at run time
    (hipRTC, the default) and interpreted (DRESSI_NO_JIT=1) give the same
    floats: the two-peel example graph (sigmoids, square roots, divisions,
    minima, steps) over 12 iterations, through both reactive rebuilds."""
    with np.load(os.path.join(GOLDEN, "hsr_peel2_ico3_2view_96px_3it.npz")) as z:
        gold = {k: z[k] for k in z.files}
    screen = int(gold["in_cfg"][0])
    print(f"[graph] compiled vs interpreted fused programs: 2 peels, {screen}px, 12 iterations",
          flush=True)
    runs = []
    for env in ({}, {"DRESSI_NO_JIT": "1"}):
        d = tmp_path / ("jit" if not env else "interp")
        d.mkdir()
        runs.append(_run_graph(d, gold["in_pos"], gold["in_faces"], gold["in_tgt_pos"],
                               gold["in_mvps"], screen, 8, 12, 3.0, 1e-3, peels=2, env=env))
    a, b = runs
    assert a["plan"] == b["plan"] == "generic"
    for k in ("pos", "m", "v", "loss", "grad0", "pred", "target"):
        assert np.array_equal(a[k], b[k]), k


def test_reactive_cache_prunes_static_branches(tmp_path, oracle):
    """Reactive rebuilds (src/pack/reactive.cpp:10-68, driven from
    src/dressi_ad.cpp:287-308,363-372): with the default counts the per-step
    kernel count falls after the fast rebuild (2 steps with the same dirty
    pattern) and again after the full rebuild (8), as the static target
    branch is served from its cached images; every loss and the final
    parameters equal a run with setRebuildCounts(0, 0), which never prunes."""
    _, pos, faces, tgt, mvps = _scene("c1", 2)
    iters, samples, lr, screen = 12, 8, 1e-3, 96
    print("[graph] reactive rebuilds: c1 mesh, 2 views, 96px, 12 iterations, Naive", flush=True)
    g = _run_graph(tmp_path, pos, faces, tgt, mvps, screen, samples, iters, 3.0, lr, naive=True)
    flat = _run_graph(tmp_path, pos, faces, tgt, mvps, screen, samples, iters, 3.0, lr,
                      naive=True, no_rebuild=True)
    k, kf = g["kernels"].astype(int), flat["kernels"].astype(int)
    print("kernels per step:", list(k), "without rebuilds:", list(kf), flush=True)
    assert len(set(kf)) == 1, kf
    assert k[0] == kf[0]
    assert k[-1] < k[0], k
    assert (np.diff(k) <= 0).all(), k
    for key in ("pos", "m", "v", "loss", "grad0", "pred", "target"):
        assert np.array_equal(g[key], flat[key]), key
    want = _fit(oracle, False, pos, faces, tgt, mvps, screen, samples, lr, 1, images=False)
    assert np.array_equal(g["grad0"], want["grad0"])


def test_captured_graph_survives_workspace_regrow(tmp_path):
    """A per-op C-ABI call through DressiAD::context() that needs larger
    workspaces than the captured step graph frees and reallocates them; the
    next execStep notices the new workspace generation, runs eagerly and
    captures again, so the results equal a run without that call."""
    _, pos, faces, tgt, mvps = _scene("c1", 1)
    iters, samples, lr, screen = 6, 8, 1e-3, 96
    print("[graph] workspace regrow through context(): c1 mesh, 96px, 6 iterations, Naive",
          flush=True)
    g = _run_graph(tmp_path, pos, faces, tgt, mvps, screen, samples, iters, 3.0, lr, naive=True,
                   regrow=True)
    base = _run_graph(tmp_path, pos, faces, tgt, mvps, screen, samples, iters, 3.0, lr,
                      naive=True)
    for key in ("pos", "m", "v", "loss", "grad0", "pred", "target"):
        assert np.array_equal(g[key], base[key]), key


@pytest.mark.parametrize("name", ["c2", "c4"])
def test_fused_route_full_workload_final_parameters(tmp_path, name):
    """The graph API at a benchmark workload's full size and iteration count
    against the oracle's final parameters (tests/golden/final_<name>.npz)."""
    w, pos, faces, tgt, mvps = _scene(name)
    print(f"[graph] {name}: {w.iters} iterations at {w.screen}^2 x {w.views}, RSP", flush=True)
    with np.load(os.path.join(GOLDEN, f"final_{name}.npz")) as z:
        gold = {k: z[k] for k in z.files}
    g = _run_graph(tmp_path, pos, faces, tgt, mvps, w.screen, 8, w.iters, 3.0, w.lr,
                   aa=w.technique == "aa", timeout=300)
    assert g["plan"] == ("fused:aa" if w.technique == "aa" else "fused:hardsoftras")
    assert g["stages"] == 1
    assert np.array_equal(g["pos"], gold["out_pos"])
    rows = g["m"].reshape(-1, 3)[gold["out_idx_m"]]
    assert np.array_equal(rows, gold["out_smp_m"])
    assert np.array_equal(g["loss"], gold["out_loss"])
    assert g["t"][0] == w.iters


TEX_EXE = os.path.join(ROOT, "tests", "_bin", "graph_tex")


@pytest.mark.parametrize("naive", [False, True])
def test_texture_example_graph_matches_oracle(tmp_path, oracle, naive):
    """The texture fit's graph (examples/texture_optimization/run.cpp:112-145
    with TextureBilinear, the RGB L2 loss and the in-graph Adam) written with
    the graph API (tests/graph_tex.cpp) and run by DressiAD with the cameras
    sent every step -- on the fused texture plan (RSP) or the generic
    executor (Naive): the first iteration's loss and texture gradient bit for
    bit against the oracle's texture fit, the later losses and the Adam state
    within 1e-6 (the generic executor's bias correction is a device powf)."""
    import opendressi_amd as od
    w = od.TexWorkload("graph", 16, 8, 64, 32, 2, 3, 1e-2, 3, 7)
    pos, uv, faces, mvps, gt, tex0 = od.make_tex_scene(w)
    iters = 3
    print(f"[graph tex] uv sphere 16x8, {w.views} views, {w.screen}px, tex {w.tex}, "
          f"naive={naive}", flush=True)
    nv, nf = len(pos), len(faces)
    hdr = np.array([nv, nf, w.views, w.screen, w.tex, w.tex, iters, w.sets, 1 if naive else 0],
                   np.uint32)
    inp, out = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(inp, "wb") as f:
        f.write(hdr.tobytes())
        f.write(np.float32(w.lr).tobytes())
        for a in (pos, uv, faces, mvps, gt, tex0):
            f.write(np.ascontiguousarray(a, np.float32).tobytes())
    res = subprocess.run([TEX_EXE, str(inp), str(out)], capture_output=True, text=True,
                         timeout=120)
    assert res.returncode == 0, res.stderr
    print(" ", res.stdout.strip(), flush=True)
    # RSP packing: the graph runs on the fused texture plan (one stage of its
    # five kernels), the cameras' clip and ScreenAttr images sent each step
    want_plan = "plan=generic" if naive else "plan=fused:texture stages=1 substages=5"
    assert want_plan in res.stdout, res.stdout
    d = np.fromfile(out, np.float32)
    t_n = w.tex * w.tex * 4
    got = {}
    o = 0
    for k, cnt in (("tex", t_n), ("m", t_n), ("v", t_n), ("t", 1), ("loss", iters),
                   ("grad0", t_n)):
        got[k] = d[o:o + cnt]
        o += cnt
    assert o == d.size
    ref = oracle.tex_fit(pos, uv, faces, mvps, w.screen, gt, tex0, lr=w.lr, iters=iters,
                         want_images=False)
    assert np.abs(got["grad0"]).max() > 0
    assert np.array_equal(got["grad0"], ref["grad0"].reshape(-1)), \
        f"grad0: max |d| {np.abs(got['grad0'] - ref['grad0'].reshape(-1)).max():.3g}"
    assert got["loss"][0] == ref["loss"][0], (got["loss"], ref["loss"])
    if not naive:
        # the fused plan: every iteration bit for bit
        for k in ("tex", "m", "v", "loss"):
            assert np.array_equal(got[k], ref[k].reshape(-1)), k
    np.testing.assert_allclose(got["loss"], ref["loss"], rtol=1e-6, atol=0)
    for k in ("tex", "m", "v"):
        want = ref[k].reshape(-1)
        np.testing.assert_allclose(got[k], want, rtol=0,
                                   atol=1e-6 * max(1.0, np.abs(want).max()), err_msg=k)
    assert got["t"][0] == iters


PBR_EXE = os.path.join(ROOT, "tests", "_bin", "graph_pbr")


@pytest.mark.parametrize("name,naive", [("pbr_ico2_48px_2view_3it.npz", False),
                                        ("pbr_ico2_48px_2view_3it.npz", True),
                                        ("pbr_ico3_96px_3view_2it.npz", False)])
def test_pbr_example_graph_matches_reference_fixture(tmp_path, golden, name, naive):
    """The PBR material + environment fit's graph written with the graph API
    and the examples' PBR graph builders (tests/graph_pbr.cpp over
    dressi_examples/pbr_graph.h) and run by DressiAD, against the reference's
    own outputs for the ico2 48 px 2-view and ico3 96 px 3-view scenes: the first loss 1e-5, the
    first-iteration albedo / mr / env gradients 1e-4 (relative to the largest
    entry) and the parameters after the fixture's iterations 1e-3 absolute --
    the bars of the fused PBR plan on the same fixture (the executor's
    reductions and the device's atan2 / acos / pow round differently from the
    reference's CPU evaluation)."""
    g = golden(name)
    keys = ("pos", "normal", "uv", "faces", "mvps", "frames", "light", "gt_albedo", "gt_mr",
            "gt_env", "albedo0", "mr0", "env0")
    a = {k: np.ascontiguousarray(g["in_" + k], np.float32) for k in keys}
    iters = len(g["out_loss"])
    th, tw = a["gt_albedo"].shape[:2]
    eh, ew = a["gt_env"].shape[:2]
    nv, nf, n = len(a["pos"]), len(a["faces"]), len(a["mvps"])
    s, levels = int(g["in_screen"]), int(g["in_levels"])
    print(f"[graph pbr] {name}: {s}px {n} views, tex {tw}x{th}, env {ew}x{eh}, naive={naive}",
          flush=True)
    hdr = np.array([nv, nf, n, s, tw, th, ew, eh, levels, iters, 1 if naive else 0], np.uint32)
    inp, out = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(inp, "wb") as f:
        f.write(hdr.tobytes())
        f.write(np.float32(g["in_lr"]).tobytes())
        for k in keys:
            f.write(a[k].tobytes())
    res = subprocess.run([PBR_EXE, str(inp), str(out)], capture_output=True, text=True,
                         timeout=120)
    assert res.returncode == 0, res.stderr
    print(" ", res.stdout.strip(), flush=True)
    d = np.fromfile(out, np.float32)
    t_n, e_n = tw * th * 3, ew * eh * 3
    got = {}
    o = 0
    for k, cnt in (("albedo", t_n), ("mr", t_n), ("env", e_n), ("t", 1), ("loss", iters),
                   ("g_albedo0", t_n), ("g_mr0", t_n), ("g_env0", e_n)):
        got[k] = d[o:o + cnt]
        o += cnt
    assert o == d.size
    assert got["t"][0] == iters

    def close(x, want, tol, what):
        want = np.asarray(want, np.float64).reshape(-1)
        diff = np.abs(x.astype(np.float64) - want).max()
        m = float(np.abs(want).max())
        assert m > 0, what
        assert diff <= tol * m, f"{what}: max diff {diff:.3g} vs max {m:.3g} (tol {tol})"

    close(got["loss"][:1], g["out_loss"][:1], 1e-5, "loss")
    for k in ("g_albedo0", "g_mr0", "g_env0"):
        close(got[k], g["out_" + k], 1e-4, k)
    if not naive:
        # RSP: the graph runs on the fused PBR plan (the route), and gives
        # the plan's own results bit for bit
        assert "plan=fused:pbr stages=1" in res.stdout, res.stdout
        import opendressi_amd as od
        from opendressi_amd import _lib
        ctx = od.Context(0)
        sc = {k: a[k] for k in keys}
        sc.update(screen=s, levels=levels, lr=float(g["in_lr"]))
        fit = od.PbrFit(ctx, sc, keep_grad=True)
        fit.step(1, graph=False)
        for k, which in (("g_albedo0", _lib.PBR_G_ALBEDO), ("g_mr0", _lib.PBR_G_MR),
                         ("g_env0", _lib.PBR_G_ENV)):
            assert np.array_equal(got[k], fit.read(which)[..., :3].reshape(-1)), k
        fit.step(iters - 1)
        alb, mr, env, t = fit.state()
        for k, want in (("albedo", alb), ("mr", mr), ("env", env)):
            assert np.array_equal(got[k], want[..., :3].reshape(-1)), k
        fit.close()
        ctx.close()
    for k in ("albedo", "mr", "env"):
        diff = float(np.abs(got[k].astype(np.float64) - g["out_" + k].reshape(-1)).max())
        assert diff <= 1e-3, f"{k}: max diff {diff:.3g} (tol 1e-3)"
