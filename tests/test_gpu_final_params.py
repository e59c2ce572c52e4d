"""Every benchmark workload run for its full iteration count on the GPU,
against the oracle's final parameters (tests/golden/final_<workload>.npz,
written by tests/golden/make_final_params.py; the oracle is pinned to the
reference's own CPU build by the unit and trajectory fixtures).

The reference example optimises for a fixed iteration count and reports the
parameters it ends with (examples/silhouette_optimization/run.cpp:574-637);
the bar for them is 1e-3. Every plan reproduces the oracle's arithmetic
operation for operation, so the whole trajectory -- every loss and the final
parameters (and, for the silhouette and texture fits, the Adam moments) --
must be identical to the oracle's bit for bit.
"""
import hashlib
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def ctx():
    import opendressi_amd as od
    c = od.Context(0)
    yield c
    c.close()


def _load(name):
    path = os.path.join(GOLDEN, f"final_{name}.npz")
    with np.load(path) as z:
        return {k: z[k] for k in z.files}


def _sha(a):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest(), np.uint8)


def _check_inputs(g, arrays):
    for k, a in arrays.items():
        assert np.array_equal(_sha(a), g["in_sha_" + k]), f"scene input {k} differs"


def _param(g, name, got):
    """(max |got - want|, bit-identical?) over the stored full array or the
    stored sample rows, plus the whole-array hash and |.| sum."""
    if "out_" + name in g:
        want = g["out_" + name]
        d = np.abs(got.astype(np.float64) - want)
    else:
        rows = got.reshape(-1, got.shape[-1])[g["out_idx_" + name]]
        d = np.abs(rows.astype(np.float64) - g["out_smp_" + name])
    same = bool(np.array_equal(_sha(got), g["out_sha_" + name]))
    s = float(np.abs(got.astype(np.float64)).sum())
    sum_rel = abs(s - float(g["out_sum_" + name][0])) / max(abs(float(g["out_sum_" + name][0])),
                                                            1e-30)
    return float(d.max()), same, sum_rel


def _run_losses(fit, iters, loss_fn):
    losses = []
    for _ in range(iters):
        fit.step(1)
        fit.synchronize()
        losses.append(loss_fn())
    return np.array(losses, np.float64)


@pytest.mark.parametrize("name", ["c2", "c4_hsr", "c4"])
def test_silhouette_final_parameters(ctx, name):
    import opendressi_amd as od
    g = _load(name)
    w = od.WORKLOADS[name]
    pos, faces, tgt, mvps = od.make_scene(w)
    _check_inputs(g, {"pos": pos, "faces": faces, "tgt": tgt, "mvps": mvps})
    print(f"[final params] {name}: {w.iters} iterations at {w.screen}^2 x {w.views}", flush=True)
    fit = od.SilhouetteFit(ctx, pos, faces, mvps, w.screen, target_mesh=(tgt, faces), lr=w.lr,
                           technique=w.technique)
    losses = _run_losses(fit, w.iters, fit.loss)
    p, m, v, t = fit.state()
    fit.close()
    assert t == float(g["out_t"][0]) == float(w.iters)
    lrel = np.abs(losses.astype(np.float32) - g["out_loss"]) / np.abs(g["out_loss"])
    res = {k: _param(g, k, a) for k, a in (("pos", p), ("m", m), ("v", v))}
    print(f"  loss rel err max {lrel.max():.3g}; pos/m/v max |d| "
          f"{[f'{r[0]:.3g}' for r in res.values()]}, identical {[r[1] for r in res.values()]}",
          flush=True)
    assert res["pos"][0] <= 1e-3
    assert lrel.max() <= 1e-6
    for k, (d, same, _) in res.items():
        assert same and d == 0.0, f"{name}: final {k} not bit-identical (max |d| {d:.3g})"


def test_texture_final_parameters(ctx):
    import opendressi_amd as od
    g = _load("c3")
    w = od.TEX_WORKLOADS["c3"]
    pos, uv, faces, mvps, gt, tex0 = od.make_tex_scene(w)
    _check_inputs(g, {"pos": pos, "uv": uv, "faces": faces, "mvps": mvps, "gt": gt,
                      "tex0": tex0})
    print(f"[final params] c3: {w.iters} iterations at {w.screen}^2 x {w.views}", flush=True)
    fit = od.TextureFit(ctx, pos, uv, faces, mvps, w.screen, gt, tex0, lr=w.lr)
    losses = _run_losses(fit, w.iters, fit.loss)
    tex, m, v, t = fit.state()
    fit.close()
    assert t == float(g["out_t"][0]) == float(w.iters)
    lrel = np.abs(losses.astype(np.float32) - g["out_loss"]) / np.abs(g["out_loss"])
    res = {k: _param(g, k, a) for k, a in (("tex", tex), ("m", m), ("v", v))}
    print(f"  loss rel err max {lrel.max():.3g}; tex/m/v max |d| "
          f"{[f'{r[0]:.3g}' for r in res.values()]}, identical {[r[1] for r in res.values()]}",
          flush=True)
    assert res["tex"][0] <= 1e-3
    assert lrel.max() <= 1e-6
    for k, (d, same, _) in res.items():
        assert same and d == 0.0, f"c3: final {k} not bit-identical (max |d| {d:.3g})"


def test_pbr_final_parameters(ctx):
    """C5 after its 100 iterations against the oracle: every loss and every
    sampled entry of the final albedo, metallic-roughness and env identical
    bit for bit. The plan adds every sum of the fit in the oracle's order
    (map gradients by band and view, the loss by F::Mean's Reduce2x2Sum
    pyramid) with the C library's transcendentals."""
    import opendressi_amd as od
    from opendressi_amd.pbr import workload_scene
    g = _load("c5")
    w = od.PBR_WORKLOADS["c5"]
    sc = workload_scene(w)
    _check_inputs(g, {k: v for k, v in sc.items() if isinstance(v, np.ndarray)})
    print(f"[final params] c5: {w.iters} iterations at {w.screen}^2 x {w.views}", flush=True)
    fit = od.PbrFit(ctx, sc)
    losses = _run_losses(fit, w.iters, fit.loss)
    alb, mr, env, _ = fit.state()
    fit.close()
    lbad = int((np.asarray(losses, np.float32) != np.asarray(g["out_loss"], np.float32)).sum())
    report = {}
    for k, a in (("albedo", alb), ("mr", mr), ("env", env)):
        x, y = _rows(g, k, a)
        d = np.abs(x - y)
        report[k] = (float(d.max()), int((d != 0).sum()), d.size)
    print(f"  losses not identical: {lbad}/{len(losses)}; (max |d|, entries not identical / "
          "sampled): " + ", ".join(f"{k} {r[0]:.3g} {r[1]}/{r[2]}" for k, r in report.items()),
          flush=True)
    assert lbad == 0, "c5: losses differ"
    for k, (dmax, nbad, _) in report.items():
        assert nbad == 0, f"c5: final {k}: {nbad} entries differ (max |d| {dmax:.3g})"


def _rows(g, name, got):
    got = np.ascontiguousarray(got)
    return got.reshape(-1, got.shape[-1])[g["out_idx_" + name]].astype(np.float64), \
        g["out_smp_" + name].astype(np.float64)


def test_pbr_c5_first_iterations(ctx):
    """C5 at its full size (1024^2 x 6 views, icosphere L5, 512^2 textures,
    512 x 256 env, 6 prefilter levels) against the oracle, entry by entry and
    bit for bit: target and prediction of the first iteration, its loss and
    albedo / metallic-roughness / env gradients, the parameters after two
    iterations."""
    import opendressi_amd as od
    from opendressi_amd import _lib as L
    from opendressi_amd.pbr import workload_scene
    if not os.path.exists(os.path.join(GOLDEN, "final_c5_first.npz")):
        pytest.skip("final_c5_first.npz not generated")
    g = _load("c5_first")
    w = od.PBR_WORKLOADS["c5"]
    sc = workload_scene(w)
    _check_inputs(g, {k: v for k, v in sc.items() if isinstance(v, np.ndarray)})
    print("[c5 first iterations] set-up", flush=True)
    fit = od.PbrFit(ctx, sc, keep_pred=True, keep_grad=True)
    got = {"target0": fit.read(L.PBR_TARGET)[..., :3]}
    fit.step(1, graph=False)
    fit.synchronize()
    loss0 = fit.loss()
    got.update(pred0=fit.read(L.PBR_PRED)[..., :3], g_albedo0=fit.read(L.PBR_G_ALBEDO)[..., :3],
               g_mr0=fit.read(L.PBR_G_MR)[..., :3], g_env0=fit.read(L.PBR_G_ENV)[..., :3])
    fit.step(1, graph=False)
    alb, mr, env, t = fit.state()
    fit.close()
    got.update(albedo=alb, mr=mr, env=env)
    assert t == 2.0
    report = {}
    fails = []
    for k, a in got.items():
        x, y = _rows(g, k, a)
        d = np.abs(x - y)
        report[k] = (float(d.max()), int((d != 0).sum()), d.size)
        if report[k][1]:
            fails.append(f"{k}: {report[k][1]} entries differ (max |d| {d.max():.3g})")
    same_loss = np.float32(loss0) == np.float32(g["out_loss"][0])
    print(f"  loss identical: {bool(same_loss)}; (max |d|, entries not identical / sampled): "
          + ", ".join(f"{k} {r[0]:.3g} {r[1]}/{r[2]}" for k, r in report.items()), flush=True)
    assert same_loss, f"c5: loss {loss0} vs {float(g['out_loss'][0])}"
    assert not fails, "; ".join(fails)
