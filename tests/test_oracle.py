"""Pins the CPU oracle (oracle/dressi_oracle.c) before it is trusted as the
checker of the HIP path:

* against the reference's own CPU evaluator through the committed golden
  fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py from
  oracle/_ref): bit-exact for every array;
* against closed forms the reference's tests state (tests/test_softras.cpp:92-139:
  distance profile 3/sqrt(2) and -0.5, hard z, coverage, depth-shift winner);
* against central finite differences of the loss (the reference's
  test_backward / test_softras FD pattern) for the per-pixel chain;
* against invariants (coverage of the hard raster is a subset of the soft
  raster; image-loss gradient equals the sum of per-pixel gradients).
"""
import math

import numpy as np
import pytest


def _exact(a, b, what=""):
    assert a.shape == b.shape, (what, a.shape, b.shape)
    if not np.array_equal(a, b):
        d = np.abs(a.astype(np.float64) - b)
        raise AssertionError(f"{what}: not bit-exact, max diff {d.max():.3g} at "
                             f"{np.unravel_index(d.argmax(), d.shape)}, {int((d > 0).sum())} differ")


# ---------------------------------------------------------------- fixtures --
def test_ops_match_reference_fixtures(oracle, golden):
    g = golden("ops_unit.npz")
    s = 16
    for name in ("profile", "depth", "generic"):
        clip, faces = g[f"in_{name}_clip"], g[f"in_{name}_faces"]
        nf = len(faces)
        soft = oracle.soft_clip(clip, faces, s, s, 3.0)
        _exact(soft, g[f"out_{name}_soft_clip"], f"{name} soft_clip")
        fid = np.repeat(np.arange(nf, dtype=np.float32), 3)
        fsoft = np.arange(3 * nf, dtype=np.float32).reshape(nf, 3)
        rs = oracle.rasterize_soft(soft, fid, fsoft, clip, faces, s, s, 3.0)
        _exact(rs, g[f"out_{name}_rasterize_soft"], f"{name} rasterize_soft")
        hard = oracle.rasterize(clip, np.ones((len(clip), 1), np.float32), faces, s, s)
        _exact(hard, g[f"out_{name}_rasterize"], f"{name} rasterize")
        ids = oracle.rasterize_face_id(clip, faces, s, s)
        _exact(ids, g[f"out_{name}_face_id"], f"{name} face_id")
    clip, faces = g["in_generic_clip"], g["in_generic_faces"]
    ids = g["out_generic_face_id"]
    tri = [oracle.lookup_faces(clip, faces, k) for k in range(3)]
    ffb8 = oracle.face_fetch_bwd(g["in_ffb_gy"], ids, *tri, 7.0, 3.0, 8)
    _exact(ffb8, g["out_ffb_n8_seed7"], "face_fetch_bwd n=8 seed=7")
    assert np.abs(ffb8).max() > 0, "stochastic samples all missed"
    _exact(oracle.face_fetch_bwd(g["in_ffb_gy"], ids, *tri, 7.0, 3.0, 0), g["out_ffb_n0"],
           "face_fetch_bwd exact")
    vf = oracle.vertex_faces_tex(faces, len(clip))
    for k in range(3):
        _exact(oracle.lookup_faces_bwd(g["in_lfb_gy"], faces, vf, k), g[f"out_lfb_k{k}"],
               f"lookup_faces_bwd k={k}")
    _exact(oracle.face_fetch(tri[1], ids), g["out_face_fetch"], "face_fetch")


@pytest.mark.parametrize("name", ["hsr_ico3_64px_5it.npz", "hsr_ico4_4view_128px_3it.npz",
                                  "hsr_c1_256px_50it.npz"])
def test_fit_matches_reference_fixture(oracle, golden, name):
    g = golden(name)
    screen, iters, radius, samples, lr = g["in_cfg"]
    images = "out_pred0" in g
    res = oracle.hsr_fit(g["in_pos"], g["in_faces"], g["in_tgt_pos"], g["in_faces"], g["in_mvps"],
                         int(screen), radius=float(radius), samples=int(samples), lr=float(lr),
                         iters=int(iters), want_images=images)
    for k, v in res.items():
        _exact(v, g["out_" + k], f"{name}:{k}")


# ------------------------------------------------------------ closed forms --
def _scene_rs(oracle, clip, faces, s=16, r=3.0):
    clip = np.asarray(clip, np.float32)
    faces = np.asarray(faces, np.float32)
    nf = len(faces)
    soft = oracle.soft_clip(clip, faces, s, s, r)
    fid = np.repeat(np.arange(nf, dtype=np.float32), 3)
    fsoft = np.arange(3 * nf, dtype=np.float32).reshape(nf, 3)
    return oracle.rasterize_soft(soft, fid, fsoft, clip, faces, s, s, r)


def _clip(sx, sy, z, s=16, w=1.0):
    return [(sx / s * 2 - 1) * w, (sy / s * 2 - 1) * w, z * w, w]


def test_distance_profile_closed_form(oracle):
    # right triangle (4,4),(12,4),(4,12): pixel (6,6) is 3/sqrt(2) from x+y=16,
    # pixel (3,6) lies 0.5 px outside x=4 (reference tests/test_softras.cpp:92-121)
    rs = _scene_rs(oracle, [_clip(4, 4, .5), _clip(12, 4, .5), _clip(4, 12, .5)], [[0, 1, 2]])
    assert abs(rs[6, 6, 0] - 3 / math.sqrt(2)) < 1e-4
    assert rs[6, 6, 1] == 0.0 and rs[6, 6, 3] == 1.0
    assert abs(rs[6, 6, 2] - 0.5) < 1e-5
    assert abs(rs[6, 3, 0] + 0.5) < 1e-4 and rs[6, 3, 3] == 1.0
    assert np.all(rs[14, 14] == 0.0)


def test_depth_shift_near_wins(oracle):
    rs = _scene_rs(oracle, [_clip(4, 4, .2), _clip(12, 4, .2), _clip(4, 12, .2),
                            _clip(4, 4, .8), _clip(12, 4, .8), _clip(4, 12, .8)],
                   [[3, 4, 5], [0, 1, 2]])
    assert rs[6, 6, 1] == 1.0 and abs(rs[6, 6, 2] - 0.2) < 1e-5


def test_hard_coverage_subset_of_soft(oracle):
    clip = np.array([_clip(4.3, 3.8, .5), _clip(12.4, 5.2, .5, 1.3), _clip(5.1, 12.6, .5),
                     _clip(11.2, 12.1, .5)], np.float32)
    faces = np.array([[0, 1, 2], [1, 3, 2]], np.float32)
    rs = _scene_rs(oracle, clip, faces)
    ids = oracle.rasterize_face_id(clip, faces, 16, 16)
    assert np.all(rs[..., 3][ids > 0] == 1.0)
    # dist >= 0 exactly where the hard raster covers (generic position)
    assert np.array_equal(rs[..., 0] >= 0, (ids > 0) | (rs[..., 3] == 0))


def test_wang_hash_known_values(oracle):
    # integer recurrence (src/core/f_ops.cpp:1473-1480), recomputed here
    def wang(x):
        m = 0xFFFFFFFF
        x = ((x ^ 61) ^ (x >> 16)) & m
        x = (x * 9) & m
        x ^= x >> 4
        x = (x * 0x27D4EB2D) & m
        x ^= x >> 15
        return x

    for x in (0, 1, 7, 12345, 0xDEADBEEF, 0xFFFFFFFF):
        assert oracle.wang_hash(x) == wang(x)
    u = oracle.hash_to_unit(3, 5, 7, 1)
    assert 0.0 <= u < 1.0


def test_camera_closed_forms(oracle):
    # LookAt from (0,0,3) toward the origin is a pure -3 z translation
    m = oracle.look_at([0, 0, 3])
    expect = np.eye(4, dtype=np.float32)
    expect[2, 3] = -3.0
    assert np.allclose(m.reshape(4, 4).T, expect, atol=1e-7)
    p = oracle.perspective_vk(math.pi / 2, 1.0, 0.1, 10.0)
    assert abs(p[0] - 1.0) < 1e-6 and abs(p[5] + 1.0) < 1e-6 and p[11] == -1.0
    assert abs(p[10] - 10.0 / (0.1 - 10.0)) < 1e-6


def test_icosphere_counts_and_unit_radius(oracle):
    for lvl in range(5):
        pos, faces = oracle.icosphere(lvl)
        assert len(pos) == 10 * 4 ** lvl + 2 and len(faces) == 20 * 4 ** lvl
        assert np.allclose(np.linalg.norm(pos, axis=1), 1.0, atol=1e-6)
        # every edge shared by exactly two faces (closed manifold)
        f = faces.astype(np.int64)
        e = np.sort(np.concatenate([f[:, [0, 1]], f[:, [1, 2]], f[:, [2, 0]]]), axis=1)
        _, cnt = np.unique(e, axis=0, return_counts=True)
        assert np.all(cnt == 2)


# ------------------------------------------------------ finite differences --
def test_pixel_chain_matches_finite_differences(oracle):
    """d loss / d corner clip of the per-pixel chain vs central differences in
    float64-rounded steps (the reference's FD pattern, tolerance as
    tests/test_softras.cpp:44-88: abs 2e-3 + rel 2e-2)."""
    s, r = 16, 3.0
    clip = np.array([_clip(4.3, 3.8, .5), _clip(12.4, 5.2, .5, 1.3), _clip(5.1, 12.6, .5)],
                    np.float32)
    faces = np.array([[0, 1, 2]], np.float32)
    rs = _scene_rs(oracle, clip, faces, s, r)
    target = (0.2 + 0.5 * (np.arange(s * s) % 3)).reshape(s, s).astype(np.float32)
    tri = [oracle.lookup_faces(clip, faces, k) for k in range(3)]
    gys = oracle.hsr_backward(rs, *tri, target, r)
    # analytic d(sum loss)/d tri_k: every pixel the ID buffer gives to face 0
    # (the n = 0 gather only scans the hard bbox +-1 px and misses soft-rim
    # pixels, so sum the gradient images directly)
    idx = (rs[..., 1] + 1) * rs[..., 3]
    own = idx > 0.5

    def loss(tris):
        _, vl = oracle.hsr_forward(rs, *tris, target, r)
        return float(vl.astype(np.float64).sum())

    h = 1e-3
    for k in range(3):
        analytic = gys[k][own].astype(np.float64).sum(axis=0)
        for c in (0, 1, 3):
            tp = [t.copy() for t in tri]
            tm = [t.copy() for t in tri]
            tp[k][0, c] += h
            tm[k][0, c] -= h
            num = (loss(tp) - loss(tm)) / (2 * h)
            assert abs(analytic[c] - num) <= 2e-3 + 2e-2 * abs(num), (k, c, analytic[c], num)
        assert analytic[2] == 0.0  # clip z never reaches the distance chain
