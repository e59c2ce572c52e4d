"""GPU parity of the per-op kernels (C ABI through opendressi_amd.ops) against
the reference's own outputs (golden fixtures) and the oracle.

Bar: bit-exact for every raster / id / gather output (integer-valued
decisions and gathers of identical float values in the reference's order).
"""
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


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


def _soft_inputs(clip, faces, s, r, ops, ctx):
    nf = len(faces)
    soft = host(ops.soft_clip(ctx, dev(clip), dev(faces), s, s, r))
    fid = np.repeat(np.arange(nf, dtype=np.float32), 3)
    fsoft = np.arange(3 * nf, dtype=np.float32).reshape(nf, 3)
    return soft, fid, fsoft


def test_ops_match_reference_fixtures(ctx, golden):
    from opendressi_amd import ops
    g = golden("ops_unit.npz")
    s = 16
    for name in ("profile", "depth", "generic"):
        clip, faces = g[f"in_{name}_clip"], g[f"in_{name}_faces"]
        print(f"[ops fixture] scene={name}", flush=True)
        soft, fid, fsoft = _soft_inputs(clip, faces, s, 3.0, ops, ctx)
        _exact(soft, g[f"out_{name}_soft_clip"], f"{name} soft_clip")
        rs = host(ops.rasterize_soft(ctx, dev(soft), dev(fid), dev(fsoft), dev(clip), dev(faces),
                                     s, s, 3.0))
        _exact(rs, g[f"out_{name}_rasterize_soft"], f"{name} rasterize_soft")
        hard = host(ops.rasterize(ctx, dev(clip), dev(np.ones((len(clip), 1))), dev(faces), s, s))
        _exact(hard, g[f"out_{name}_rasterize"], f"{name} rasterize")
        ids = host(ops.rasterize_face_id(ctx, dev(clip), dev(faces), s, s))
        _exact(ids, g[f"out_{name}_face_id"], f"{name} face_id")
    clip, faces, ids = g["in_generic_clip"], g["in_generic_faces"], g["out_generic_face_id"]
    tri = [ops.lookup_faces(ctx, dev(clip), dev(faces), k) for k in range(3)]
    seed = dev(np.array([7.0]))
    ffb = host(ops.face_fetch_bwd(ctx, dev(g["in_ffb_gy"]), dev(ids), *tri, seed, 3.0, 8))
    _exact(ffb, g["out_ffb_n8_seed7"], "face_fetch_bwd n=8 seed=7")
    ffb0 = host(ops.face_fetch_bwd(ctx, dev(g["in_ffb_gy"]), dev(ids), *tri, seed, 3.0, 0))
    _exact(ffb0, g["out_ffb_n0"], "face_fetch_bwd exact")
    import opendressi_amd as od
    vf = od.vertex_faces_tex(faces, len(clip))
    for k in range(3):
        lfb = host(ops.lookup_faces_bwd(ctx, dev(g["in_lfb_gy"]), dev(faces), dev(vf), k))
        _exact(lfb, g[f"out_lfb_k{k}"], f"lookup_faces_bwd k={k}")
    _exact(host(ops.face_fetch(ctx, tri[1], dev(ids))), g["out_face_fetch"], "face_fetch")
    ctx.synchronize()


def _random_scene(seed, level, s):
    import opendressi_amd as od
    rng = np.random.default_rng(seed)
    pos, faces = od.icosphere(level)
    pos = pos * (1 + 0.1 * rng.standard_normal((len(pos), 1))).astype(np.float32)
    yaw, pitch = rng.uniform(0, 2 * math.pi), rng.uniform(-1.0, 1.0)
    dist = rng.uniform(2.2, 4.0)
    eye = [dist * math.cos(pitch) * math.sin(yaw), dist * math.sin(pitch),
           dist * math.cos(pitch) * math.cos(yaw)]
    mvp = od.mat4_mul(od.perspective_vk(math.radians(rng.uniform(30, 70)), 1.0, 0.1, 10.0),
                      od.look_at(eye))
    clip = np.zeros((len(pos), 4), np.float32)
    for row in range(4):
        acc = np.zeros(len(pos), np.float32)
        for k in range(3):
            acc = acc + mvp[k * 4 + row] * pos[:, k]
        clip[:, row] = acc + mvp[12 + row]
    return clip, faces


@pytest.mark.parametrize("seed,level,s", [(1, 3, 64), (2, 4, 100), (3, 3, 257), (4, 5, 320)])
def test_rasterizers_match_oracle(ctx, oracle, seed, level, s):
    from opendressi_amd import ops
    print(f"[raster parity] seed={seed} level={level} screen={s}", flush=True)
    clip, faces = _random_scene(seed, level, s)
    r = 3.0
    soft, fid, fsoft = _soft_inputs(clip, faces, s, r, ops, ctx)
    _exact(soft, oracle.soft_clip(clip, faces, s, s, r), "soft_clip")
    rs = host(ops.rasterize_soft(ctx, dev(soft), dev(fid), dev(fsoft), dev(clip), dev(faces),
                                 s, s, r))
    want = oracle.rasterize_soft(soft, fid, fsoft, clip, faces, s, s, r)
    _exact(rs, want, "rasterize_soft")
    assert (want[..., 3] > 0).sum() > 100  # the scene is actually on screen
    # peel overload: previous layer's shifted depth rebuilt from the channels
    # (examples/silhouette_optimization/run.cpp:320-330)
    ge = (want[..., 0] >= 0).astype(np.float32)
    prev = want[..., 3] * (ge * (np.clip(want[..., 2], 0, 1) * 0.5) +
                           (1 - ge) * (np.clip(-want[..., 0] * (1 / r), 0, 1) * 0.5 + 0.5))
    prev = prev.astype(np.float32)
    rs2 = host(ops.rasterize_soft(ctx, dev(soft), dev(fid), dev(fsoft), dev(clip), dev(faces),
                                  s, s, r, prev_shifted_depth=dev(prev)))
    _exact(rs2, oracle.rasterize_soft(soft, fid, fsoft, clip, faces, s, s, r, prev=prev),
           "rasterize_soft peel")
    attr = np.random.default_rng(seed).standard_normal((len(clip), 3)).astype(np.float32)
    _exact(host(ops.rasterize(ctx, dev(clip), dev(attr), dev(faces), s, s)),
           oracle.rasterize(clip, attr, faces, s, s), "rasterize attr3")
    _exact(host(ops.rasterize_face_id(ctx, dev(clip), dev(faces), s, s)),
           oracle.rasterize_face_id(clip, faces, s, s), "face_id")
    ctx.synchronize()


def test_rasterize_batch_matches_per_item(ctx, oracle):
    """dressi_rasterize_batch: three items (different cameras, per-item and
    shared attributes) in one pass equal the oracle's per-item Rasterize and
    RasterizeFaceId, including an odd screen size."""
    import torch

    from opendressi_amd import ops
    s = 97
    items = [_random_scene(seed, 3, s) for seed in (5, 6, 7)]
    faces = items[0][1]
    assert all(np.array_equal(it[1], faces) for it in items)
    clip = np.stack([it[0] for it in items])
    rng = np.random.default_rng(9)
    attr_items = rng.standard_normal((3, clip.shape[1], 2)).astype(np.float32)
    attr_shared = attr_items[0]
    print(f"[raster batch] 3 items screen={s}", flush=True)
    out, ids = ops.rasterize_batch(ctx, dev(clip), dev(attr_items), dev(faces), s, s,
                                   with_face_id=True)
    out2 = ops.rasterize_batch(ctx, dev(clip), dev(attr_shared), dev(faces), s, s)
    out, ids, out2 = host(out), host(ids), host(out2)
    for i in range(3):
        _exact(out[i], oracle.rasterize(clip[i], attr_items[i], faces, s, s), f"item {i} attr")
        _exact(out2[i], oracle.rasterize(clip[i], attr_shared, faces, s, s), f"item {i} shared")
        _exact(ids[i], oracle.rasterize_face_id(clip[i], faces, s, s), f"item {i} face id")
    assert (ids > 0).sum() > 100
    ctx.synchronize()


def test_lookup_and_fetch_batches_match_per_item(ctx, oracle):
    """The batched LookupFaces / FaceFetch and their backwards: three items
    (own cameras; per-item and shared attributes / clips; the exact and the
    stochastic FaceFetchBwd with a seed per item) equal the single-item entry
    points item by item, bit for bit."""
    import torch

    from opendressi_amd import ops
    s = 61
    items = [_random_scene(seed, 3, s) for seed in (21, 22, 23)]
    faces = items[0][1]
    clip = np.stack([it[0] for it in items])
    nv = clip.shape[1]
    rng = np.random.default_rng(5)
    attr = rng.standard_normal((3, nv, 3)).astype(np.float32)
    ids = np.stack([oracle.rasterize_face_id(c, faces, s, s) for c in clip])
    gy = rng.standard_normal((3, s, s, 3)).astype(np.float32)
    vf = oracle.vertex_faces_tex(faces, nv)
    seeds = np.array([0.0, 5.0, 11.0], np.float32)
    print(f"[fetch batch] 3 items screen={s}", flush=True)
    d_faces, d_ids, d_vf, d_gy = dev(faces), dev(ids), dev(vf), dev(gy)
    for k in range(3):
        lf = host(ops.lookup_faces_batch(ctx, dev(attr), d_faces, k, 3))
        lf_shared = host(ops.lookup_faces_batch(ctx, dev(attr[1]), d_faces, k, 3))
        prj = [ops.lookup_faces_batch(ctx, dev(clip), d_faces, q, 3) for q in range(3)]
        ff = host(ops.face_fetch_batch(ctx, dev(lf), d_ids))
        ff_shared = host(ops.face_fetch_batch(ctx, dev(lf_shared[0]), d_ids))
        bwd = {n: host(ops.face_fetch_bwd_batch(ctx, d_gy, d_ids, prj[0], prj[1], prj[2],
                                                dev(seeds), 2.0, n)) for n in (0, 8)}
        lb = host(ops.lookup_faces_bwd_batch(ctx, dev(bwd[0]), d_faces, d_vf, k))
        for i in range(3):
            what = f"corner {k} item {i}"
            _exact(lf[i], host(ops.lookup_faces(ctx, dev(attr[i]), d_faces, k)), what + " lookup")
            _exact(lf_shared[i], host(ops.lookup_faces(ctx, dev(attr[1]), d_faces, k)),
                   what + " lookup shared")
            _exact(ff[i], host(ops.face_fetch(ctx, dev(lf[i]), dev(ids[i]))), what + " fetch")
            _exact(ff_shared[i], host(ops.face_fetch(ctx, dev(lf_shared[0]), dev(ids[i]))),
                   what + " fetch shared")
            pi = [p[i].contiguous() for p in prj]
            for n in (0, 8):
                one = ops.face_fetch_bwd(ctx, dev(gy[i]), dev(ids[i]), pi[0], pi[1], pi[2],
                                         dev(seeds[i:i + 1]), 2.0, n)
                _exact(bwd[n][i], host(one), f"{what} fetch bwd n={n}")
            _exact(lb[i], host(ops.lookup_faces_bwd(ctx, dev(bwd[0][i]), d_faces, d_vf, k)),
                   what + " lookup bwd")
    assert (ids > 0).sum() > 300
    ctx.synchronize()


def test_raster_edge_cases(ctx, oracle):
    """Empty mesh, a screen-filling triangle (its bins overflow the list
    capacity and take the full-scan path), faces behind the camera, a
    degenerate face, and a screen size that is not a multiple of the tile."""
    from opendressi_amd import ops
    s = 1100  # 69 x 69 tiles: more bin entries than the default list capacity
    clip = np.array([[-3, -3, .5, 1], [9, -3, .5, 1], [-3, 9, .5, 1],      # covers all
                     [0, 0, .2, 1], [.5, 0, .2, 1], [0, .5, .2, 1],         # small, in front
                     [.1, .1, .3, -1], [.6, .1, .3, 1], [.1, .6, .3, 1],    # w < 0
                     [.2, .2, .1, 1], [.2, .2, .1, 1], [.7, .7, .1, 1]],    # degenerate
                    np.float32)
    faces = np.arange(12, dtype=np.float32).reshape(4, 3)
    _exact(host(ops.rasterize_face_id(ctx, dev(clip), dev(faces), s, s)),
           oracle.rasterize_face_id(clip, faces, s, s), "face_id edge")
    soft, fid, fsoft = _soft_inputs(clip, faces, s, 3.0, ops, ctx)
    _exact(soft, oracle.soft_clip(clip, faces, s, s, 3.0), "soft_clip edge")
    _exact(host(ops.rasterize_soft(ctx, dev(soft), dev(fid), dev(fsoft), dev(clip), dev(faces),
                                   s, s, 3.0)),
           oracle.rasterize_soft(soft, fid, fsoft, clip, faces, s, s, 3.0), "rasterize_soft edge")
    empty = np.zeros((0, 3), np.float32)
    import torch
    out = ops.rasterize_face_id(ctx, dev(clip), torch.zeros((0, 3), device="cuda"), 40, 24)
    assert float(host(out).sum()) == 0.0
    ctx.synchronize()


def test_bad_indices_are_reported(ctx):
    import opendressi_amd as od
    from opendressi_amd import ops
    clip = np.zeros((3, 4), np.float32)
    faces = np.array([[0, 1, 7]], np.float32)  # vertex 7 does not exist
    ops.rasterize_face_id(ctx, dev(clip), dev(faces), 16, 16)
    with pytest.raises(od.DressiError, match="out of range"):
        ctx.synchronize()
    ctx.synchronize()  # the error word is cleared after being reported


def test_device_sqrt_div_exp_agree_with_host(ctx, oracle):
    """The fused kernels rely on IEEE division and sqrt on the device; a
    rasterize_soft over many random sub-pixel triangles exercises both in the
    depth decisions. expf is not required to be bit-exact (see the HSR tests)."""
    from opendressi_amd import ops
    rng = np.random.default_rng(11)
    n = 400
    s = 96
    clip = np.zeros((3 * n, 4), np.float32)
    clip[:, :2] = rng.uniform(-1, 1, (3 * n, 2))
    clip[:, 2] = rng.uniform(0.05, 0.95, 3 * n)
    clip[:, 3] = rng.uniform(0.5, 2.0, 3 * n)
    clip[:, :3] *= clip[:, 3:4]
    faces = np.arange(3 * n, dtype=np.float32).reshape(n, 3)
    soft, fid, fsoft = _soft_inputs(clip, faces, s, 3.0, ops, ctx)
    _exact(soft, oracle.soft_clip(clip, faces, s, s, 3.0), "soft_clip random")
    _exact(host(ops.rasterize_soft(ctx, dev(soft), dev(fid), dev(fsoft), dev(clip), dev(faces),
                                   s, s, 3.0)),
           oracle.rasterize_soft(soft, fid, fsoft, clip, faces, s, s, 3.0),
           "rasterize_soft random overlap")
    ctx.synchronize()
