"""GPU parity of the screen-space antialiasing path (technique aa) against
the reference's own outputs (golden fixtures from oracle/_ref) and the oracle
at full size, through the C ABI.

Bars: face-id buffers bit-exact; rendered images within 1e-5
relative; vertex gradients within 1e-4 relative; optimised parameters within
1e-3 after the fixed iteration count. The kernels replay the reference's
float operations in its order, so the fixture cases are checked bit-exactly.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

S = 16


@pytest.fixture(scope="module")
def ctx():
    import opendressi_amd as od
    c = od.Context(0)
    yield c
    c.close()


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _exact(a, b, what):
    assert a.shape == b.shape, (what, a.shape, b.shape)
    if not np.array_equal(a, b):
        d = np.abs(a.astype(np.float64) - b)
        idx = np.unravel_index(d.argmax(), d.shape)
        raise AssertionError(f"{what}: {int((d > 0).sum())} values differ, max {d.max():.3g} at "
                             f"{idx}: got {a[idx]} want {b[idx]}")


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


@pytest.mark.parametrize("name", ["generic", "w13", "occlusion"])
def test_aa_ops_match_reference_fixtures(ctx, golden, name):
    from opendressi_amd import ops
    g = golden("aa_unit.npz")
    print(f"[aa op fixture] {name}", flush=True)
    clip, faces = dev(g[f"in_{name}_clip"]), dev(g[f"in_{name}_faces"])
    img, tri, vf, gy = (dev(g[f"in_{name}_{k}"]) for k in ("img", "tri", "vf", "gy"))
    _exact(host(ops.rasterize_face_id(ctx, clip, faces, S, S)), g[f"in_{name}_tri"], "face id")
    _exact(host(ops.antialias(ctx, img, tri, clip, faces)), g[f"out_{name}_aa"], "fwd")
    _exact(host(ops.antialias_bwd_img(ctx, gy, tri, clip, faces)), g[f"out_{name}_bwd_img"],
           "bwd img")
    seed = dev(np.array([7.0], np.float32))
    wide = ops.antialias_bwd_vtx(ctx, gy, img, tri, clip, faces, vf, seed, 8, wide=True)
    _exact(host(wide), g[f"out_{name}_bwd_vtx_wide_n8_seed7"], "bwd vtx wide")
    _exact(host(ops.col_sum(ctx, wide)), g[f"out_{name}_bwd_vtx_n8_seed7"], "colsum")
    _exact(host(ops.antialias_bwd_vtx(ctx, gy, img, tri, clip, faces, vf, None, 0)),
           g[f"out_{name}_bwd_vtx_n0"], "bwd vtx n0")


def _random_scene(oracle, seed, level, s):
    """An icosphere seen from a random orbit camera (clip, faces)."""
    import math
    rng = np.random.default_rng(seed)
    pos, faces = oracle.icosphere(level)
    pos = (pos * (1.0 + 0.05 * rng.standard_normal(len(pos)))[:, None]).astype(np.float32)
    yaw, pitch = rng.uniform(0, 2 * math.pi), rng.uniform(-0.6, 0.6)
    eye = [3 * math.cos(pitch) * math.sin(yaw), 3 * math.sin(pitch),
           3 * math.cos(pitch) * math.cos(yaw)]
    proj = oracle.perspective_vk(45 * math.pi / 180, 1.0, 0.1, 10.0)
    mvp = oracle.mat4_mul(proj, oracle.look_at(eye))
    return oracle.transform_to_clip(pos, mvp), faces


@pytest.mark.parametrize("seed,level,s", [(1, 3, 64), (2, 4, 97), (3, 3, 257)])
def test_aa_ops_match_oracle(ctx, oracle, seed, level, s):
    from opendressi_amd import ops
    print(f"[aa op parity] seed={seed} level={level} screen={s}", flush=True)
    clip, faces = _random_scene(oracle, seed, level, s)
    ones = np.ones(len(clip), np.float32)
    img = oracle.rasterize(clip, ones, faces, s, s)[..., 0]
    tri = oracle.rasterize_face_id(clip, faces, s, s)
    vf = oracle.vertex_faces_tex(faces, len(clip))
    rng = np.random.default_rng(seed)
    gy = rng.standard_normal((s, s)).astype(np.float32)
    _exact(host(ops.rasterize(ctx, dev(clip), dev(ones), dev(faces), s, s))[..., 0], img, "mask")
    d_img, d_tri, d_clip, d_faces = dev(img), dev(tri), dev(clip), dev(faces)
    _exact(host(ops.antialias(ctx, d_img, d_tri, d_clip, d_faces)),
           oracle.antialias(img, tri, clip, faces), "fwd")
    _exact(host(ops.antialias_bwd_img(ctx, dev(gy), d_tri, d_clip, d_faces)),
           oracle.antialias_bwd_img(gy, tri, clip, faces), "bwd img")
    for n, seed_v in ((8, 3.0), (0, 0.0)):
        got = host(ops.antialias_bwd_vtx(ctx, dev(gy), d_img, d_tri, d_clip, d_faces, dev(vf),
                                         dev(np.array([seed_v], np.float32)), n))
        want = oracle.antialias_bwd_vtx(gy, img, tri, clip, faces, vf, seed_v, n)
        _exact(got, want, f"bwd vtx n={n}")


def test_aa_batch_ops_match_oracle(ctx, oracle):
    """The batched AntiAlias / AntiAliasBwdImg / AntiAliasBwdVtx / ColSum
    entry points: three items (own cameras; per-item clips, and one clip
    shared by all), 2-channel images at an odd screen size, each item equal
    to the oracle's single-image op; the stochastic backward with a seed per
    item, the exact one, and ColSum of the wide partials."""
    import torch

    from opendressi_amd import ops
    s = 97
    print(f"[aa batch ops] 3 items screen={s}", flush=True)
    scenes = [_random_scene(oracle, seed, 3, s) for seed in (11, 12, 13)]
    faces = scenes[0][1]
    vf = oracle.vertex_faces_tex(faces, len(scenes[0][0]))
    rng = np.random.default_rng(4)
    for shared in (False, True):
        clips = [scenes[0][0] if shared else sc[0] for sc in scenes]
        ones = np.ones(len(clips[0]), np.float32)
        masks = [oracle.rasterize(c, ones, faces, s, s)[..., 0] for c in clips]
        tris = np.stack([oracle.rasterize_face_id(c, faces, s, s) for c in clips])
        img = np.stack([np.stack([m, m * rng.uniform(0.2, 1.0)], -1) for m in masks]).astype(
            np.float32)
        gy = rng.standard_normal(img.shape).astype(np.float32)
        seeds = np.array([3.0, 4.0, 9.0], np.float32)
        d_clip = dev(clips[0]) if shared else dev(np.stack(clips))
        d_img, d_tri, d_gy, d_faces = dev(img), dev(tris), dev(gy), dev(faces)
        fwd = host(ops.antialias_batch(ctx, d_img, d_tri, d_clip, d_faces))
        bimg = host(ops.antialias_bwd_img_batch(ctx, d_gy, d_tri, d_clip, d_faces))
        wide = ops.antialias_bwd_vtx_batch(ctx, d_gy, d_img, d_tri, d_clip, d_faces, dev(vf),
                                           dev(seeds), 8, wide=True)
        summed = host(ops.col_sum_batch(ctx, wide))
        wide = host(wide)
        exact = host(ops.antialias_bwd_vtx_batch(ctx, d_gy, d_img, d_tri, d_clip, d_faces,
                                                 dev(vf), None, 0))
        for i in range(3):
            what = f"item {i} shared={shared}"
            _exact(fwd[i], oracle.antialias(img[i], tris[i], clips[i], faces), f"{what} fwd")
            _exact(bimg[i], oracle.antialias_bwd_img(gy[i], tris[i], clips[i], faces),
                   f"{what} bwd img")
            want = oracle.antialias_bwd_vtx(gy[i], img[i], tris[i], clips[i], faces, vf,
                                            float(seeds[i]), 8)
            _exact(wide[i], want, f"{what} bwd vtx n=8")
            _exact(summed[i], oracle.col_sum(want), f"{what} col sum")
            _exact(exact[i], oracle.antialias_bwd_vtx(gy[i], img[i], tris[i], clips[i], faces,
                                                      vf, 0.0, 0), f"{what} bwd vtx exact")
        assert (tris > 0).sum() > 300
    ctx.synchronize()


def _fit(ctx, g, keep=True):
    import opendressi_amd as od
    screen = int(g["in_cfg"][0])
    return od.SilhouetteFit(ctx, g["in_pos"], g["in_faces"], g["in_mvps"], screen,
                            target_mesh=(g["in_tgt_pos"], g["in_faces"]),
                            samples=int(g["in_cfg"][2]), lr=float(g["in_cfg"][3]),
                            keep_pred=keep, keep_grad=keep, technique="aa")


@pytest.mark.parametrize("name", ["aa_ico3_64px_5it.npz", "aa_ico4_4view_128px_3it.npz"])
def test_aa_first_iteration_matches_reference(ctx, golden, name):
    from opendressi_amd import _lib as L
    g = golden(name)
    print(f"[aa fixture] {name}", flush=True)
    fit = _fit(ctx, g)
    _exact(fit.read(L.BUF_TARGET), g["out_target"], "target")
    fit.step(1)
    ctx.synchronize()
    _exact(fit.read(L.BUF_FACE_ID).astype(np.float32), g["out_tri0"], "face ids")
    _exact(fit.read(L.BUF_PRED), g["out_pred0"], "pred")
    _exact(fit.read(L.BUF_LOSS), g["out_lossimg0"], "loss image")
    grad = fit.read(L.BUF_GRAD)
    print(f"  grad rel err {rel_err(grad, g['out_grad0']):.3g}", flush=True)
    _exact(grad, g["out_grad0"], "grad")
    fit.close()


@pytest.mark.parametrize("name", ["aa_ico3_64px_5it.npz", "aa_ico4_4view_128px_3it.npz",
                                  "aa_c1_256px_50it.npz"])
def test_aa_trajectory_matches_reference(ctx, golden, name):
    g = golden(name)
    iters = int(g["in_cfg"][1])
    print(f"[aa trajectory] {name} iters={iters}", flush=True)
    fit = _fit(ctx, g, keep=False)
    losses = []
    for _ in range(iters):
        fit.step(1)
        losses.append(fit.loss())
    pos, m, v, t = fit.state()
    assert t == float(iters)
    err = float(np.abs(pos - g["out_pos"]).max())
    print(f"  final pos max abs err {err:.3g}, loss rel err {rel_err(losses, g['out_loss']):.3g}",
          flush=True)
    assert err <= 1e-3 and rel_err(losses, g["out_loss"]) <= 1e-4
    assert np.array_equal(pos, g["out_pos"]) and np.array_equal(m, g["out_m"])
    assert np.array_equal(v, g["out_v"])
    fit.close()


@pytest.mark.parametrize("screen,dist", [(97, 3.0), (301, 3.0), (130, 2.2), (128, 2.2)])
def test_aa_odd_screen_matches_oracle(ctx, oracle, screen, dist):
    """Screens that are not a multiple of 4 px (scalar row path, a partial
    last lane), wider than one 256-px forward workgroup, and cameras close
    enough (distance 2.2) for the silhouette to cross every image border: ids,
    pred, loss image and gradient of the first iteration, then 3 iterations
    of state."""
    import opendressi_amd as od
    from opendressi_amd import _lib as L
    print(f"[aa odd screen] {screen} camera distance {dist}", flush=True)
    w = od.Workload("odd", 3, screen, 4, 0.05, 0.1, 1e-3, 3, 7, "aa")
    pos, faces, tgt, _ = od.make_scene(w)
    mvps = od.camera_mvps(4, dist=dist)
    fit = od.SilhouetteFit(ctx, pos, faces, mvps, screen, target_mesh=(tgt, faces), lr=w.lr,
                           keep_pred=True, keep_grad=True, technique="aa")
    fit.step(1)
    ctx.synchronize()
    got = {k: fit.read(b) for k, b in (("tri0", L.BUF_FACE_ID), ("pred0", L.BUF_PRED),
                                       ("lossimg0", L.BUF_LOSS), ("grad0", L.BUF_GRAD))}
    fit.step(2)
    pos_g, m_g, v_g, t_g = fit.state()
    fit.close()
    ref = oracle.aa_fit(pos, faces, tgt, faces, mvps, screen, lr=w.lr, iters=3)
    _exact(got["tri0"].astype(np.float32), ref["tri0"], "face ids")
    for k in ("pred0", "lossimg0", "grad0"):
        _exact(got[k], ref[k], k)
    assert t_g == 3.0
    _exact(pos_g, ref["pos"], "pos")
    _exact(m_g, ref["m"], "m")
    _exact(v_g, ref["v"], "v")


def test_aa_graph_replay_equals_eager(ctx):
    import opendressi_amd as od
    from opendressi_amd import _lib as L
    a = od.SilhouetteFit.from_workload(ctx, "c1", keep_grad=True, technique="aa")
    b = od.SilhouetteFit.from_workload(ctx, "c1", keep_grad=True, technique="aa")
    for i in range(3):
        a.step(1, graph=True)
        b.step(1, graph=False)
        ctx.synchronize()
        pa, _, va, ta = a.state()
        pb, _, vb, tb = b.state()
        assert np.array_equal(pa, pb) and np.array_equal(va, vb) and ta == tb, i
        assert np.array_equal(a.read(L.BUF_FACE_ID), b.read(L.BUF_FACE_ID))
        assert np.array_equal(a.read(L.BUF_GRAD), b.read(L.BUF_GRAD))
    a.close()
    b.close()


def test_aa_c4_full_size_matches_oracle(ctx, oracle):
    """2048^2 x 4 views, icosphere L6, technique aa (the C4 workload): face
    ids, pred, loss image and the gradient of one iteration, bit for bit."""
    import opendressi_amd as od
    from opendressi_amd import _lib as L
    w = od.WORKLOADS["c4"]
    pos, faces, tgt, mvps = od.make_scene(w)
    print("[aa full-size] c4 1 iteration", flush=True)
    fit = od.SilhouetteFit(ctx, pos, faces, mvps, w.screen, target_mesh=(tgt, faces), lr=w.lr,
                           keep_pred=True, keep_grad=True, technique="aa")
    fit.step(1)
    ctx.synchronize()
    ids, pred, loss, grad = (fit.read(b) for b in (L.BUF_FACE_ID, L.BUF_PRED, L.BUF_LOSS,
                                                   L.BUF_GRAD))
    target = fit.read(L.BUF_TARGET)
    fit.close()
    ref = oracle.aa_fit(pos, faces, tgt, faces, mvps, w.screen, lr=w.lr, iters=1)
    _exact(target, ref["target"], "target")
    _exact(ids.astype(np.float32), ref["tri0"], "face ids")
    e = rel_err(grad, ref["grad0"])
    print(f"  grad rel err {e:.3g}, exact {np.array_equal(grad, ref['grad0'])}", flush=True)
    _exact(pred, ref["pred0"], "pred")
    _exact(loss, ref["lossimg0"], "loss image")
    _exact(grad, ref["grad0"], "grad")
