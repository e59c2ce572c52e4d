"""Pins the oracle's screen-space antialiasing (technique aa:
oracle/dressi_oracle.c or_eval_aa_pair / or_antialias / or_antialias_bwd_img /
or_antialias_bwd_vtx / or_col_sum / or_aa_fit) before it is trusted as the
checker of the HIP path:

* bit-exact against the reference's own CPU evaluator through the committed
  fixtures (tests/golden/aa_*.npz from tests/golden/make_golden.py): the three
  scenes of tests/test_antialias.cpp:153-273 (fwd, bwd img, bwd vtx n = 0 and
  n = 8 seed 7 with its wide partials) and the AA silhouette fit (1 view / 4
  views, and the 256^2 x 50-iteration trajectory);
* against what the mathematics fixes: AntiAlias is linear in the image, so
  its backward w.r.t. the image is its exact adjoint (<A x, y> = <x, A^T y>);
  pixels whose 3x3 neighbourhood shares one triangle id keep their value
  (tests/test_antialias.cpp:183-186); the exact vertex backward matches
  central finite differences of the forward w.r.t. the clip positions with
  the id buffers frozen (tests/test_antialias.cpp:219-236); the back
  triangle of the occlusion scene gets exactly zero gradient
  (tests/test_antialias.cpp:238-272); ColSum is the row sum.
"""
import numpy as np
import pytest

S = 16


def _exact(a, b, what=""):
    assert a.shape == b.shape, (what, a.shape, b.shape)
    if not np.array_equal(a, b):
        d = np.abs(a.astype(np.float64) - b)
        raise AssertionError(f"{what}: not bit-exact, max diff {d.max():.3g}, "
                             f"{int((d > 0).sum())} differ")


def _clip(sx, sy, z, w=1.0):
    return [(sx / S * 2 - 1) * w, (sy / S * 2 - 1) * w, z * w, w]


GENERIC = ([_clip(4.3, 3.8, .5), _clip(12.4, 5.2, .5), _clip(5.1, 12.6, .5)], [[0, 1, 2]])
W13 = ([_clip(4.3, 3.8, .5), _clip(12.4, 5.2, .5, 1.3), _clip(5.1, 12.6, .5)], [[0, 1, 2]])


def _scene(oracle, clip, faces, shade=None):
    clip = np.array(clip, np.float32)
    faces = np.array(faces, np.float32)
    attr = np.ones(len(clip), np.float32) if shade is None else np.array(shade, np.float32)
    img = oracle.rasterize(clip, attr, faces, S, S)[..., 0]
    tri = oracle.rasterize_face_id(clip, faces, S, S)
    vf = oracle.vertex_faces_tex(faces, len(clip))
    return clip, faces, img, tri, vf


# ---------------------------------------------------------------- fixtures --
@pytest.mark.parametrize("name", ["generic", "w13", "occlusion"])
def test_aa_ops_match_reference_fixtures(oracle, golden, name):
    g = golden("aa_unit.npz")
    clip, faces = g[f"in_{name}_clip"], g[f"in_{name}_faces"]
    img, tri, vf, gy = g[f"in_{name}_img"], g[f"in_{name}_tri"], g[f"in_{name}_vf"], g[f"in_{name}_gy"]
    _exact(oracle.rasterize_face_id(clip, faces, S, S), tri, "face id")
    _exact(oracle.antialias(img, tri, clip, faces), g[f"out_{name}_aa"], "fwd")
    _exact(oracle.antialias_bwd_img(gy, tri, clip, faces), g[f"out_{name}_bwd_img"], "bwd img")
    wide = oracle.antialias_bwd_vtx(gy, img, tri, clip, faces, vf, 7.0, 8, wide=True)
    _exact(wide, g[f"out_{name}_bwd_vtx_wide_n8_seed7"], "bwd vtx wide")
    _exact(oracle.col_sum(wide.transpose(0, 1, 2)), g[f"out_{name}_bwd_vtx_n8_seed7"], "colsum")
    _exact(oracle.antialias_bwd_vtx(gy, img, tri, clip, faces, vf, 7.0, 0),
           g[f"out_{name}_bwd_vtx_n0"], "bwd vtx n0")


@pytest.mark.parametrize("name", ["aa_ico3_64px_5it.npz", "aa_ico4_4view_128px_3it.npz",
                                  "aa_c1_256px_50it.npz"])
def test_aa_fit_matches_reference_fixture(oracle, golden, name):
    g = golden(name)
    screen, iters, samples, lr = g["in_cfg"]
    images = "out_pred0" in g
    res = oracle.aa_fit(g["in_pos"], g["in_faces"], g["in_tgt_pos"], g["in_faces"],
                        g["in_mvps"], int(screen), samples=int(samples), lr=float(lr),
                        iters=int(iters), want_images=images)
    for k, v in res.items():
        _exact(v, g["out_" + k], f"{name}:{k}")
    assert np.abs(res["grad0"]).max() > 0  # the gather reaches the mesh


# ------------------------------------------------------------ closed forms --
def test_uniform_neighbourhoods_keep_their_value(oracle):
    clip, faces, img, tri, _ = _scene(oracle, *GENERIC)
    out = oracle.antialias(img, tri, clip, faces)
    n_uniform = n_mixed = 0
    for y in range(1, S - 1):
        for x in range(1, S - 1):
            nb = tri[y - 1:y + 2, x - 1:x + 2]
            if np.all(nb == tri[y, x]):
                # (c + 8 c) / 9 in float: within one rounding of c
                assert abs(out[y, x] - img[y, x]) <= 1e-6
                n_uniform += 1
            else:
                assert 0.0 <= out[y, x] <= 1.0
                n_mixed += 1
    assert n_uniform > 0 and n_mixed > 0


@pytest.mark.parametrize("scene", [GENERIC, W13])
def test_bwd_img_is_the_adjoint(oracle, scene):
    clip, faces, _, tri, _ = _scene(oracle, *scene)
    rng = np.random.default_rng(0)
    for _ in range(3):
        x = rng.standard_normal((S, S)).astype(np.float32)
        y = rng.standard_normal((S, S)).astype(np.float32)
        lhs = float((oracle.antialias(x, tri, clip, faces).astype(np.float64) * y).sum())
        rhs = float((x.astype(np.float64) * oracle.antialias_bwd_img(y, tri, clip, faces)).sum())
        assert abs(lhs - rhs) <= 1e-5 * (abs(lhs) + abs(rhs) + 1.0), (lhs, rhs)


def test_exact_vtx_gradient_matches_finite_differences(oracle):
    """loss = mean((t - AA(img))^2) with img / tri frozen; d loss / d clip of
    the exact (n = 0) gather vs central differences (tolerance of
    tests/test_antialias.cpp:233-235: rel 2e-2, abs 2e-3); z gets none."""
    clip, faces, img, tri, vf = _scene(oracle, *W13)
    target = np.full((S, S), 0.35, np.float32)

    def loss(c):
        a = oracle.antialias(img, tri, c, faces).astype(np.float64)
        return float(((target - a) ** 2).mean())

    a = oracle.antialias(img, tri, clip, faces)
    gy = (-2.0 * (target - a) / (S * S)).astype(np.float32)
    g = oracle.antialias_bwd_vtx(gy, img, tri, clip, faces, vf, 0.0, 0)
    h = 1e-3
    for v in range(3):
        for c in range(4):
            cp, cm = clip.copy(), clip.copy()
            cp[v, c] += h
            cm[v, c] -= h
            num = (loss(cp) - loss(cm)) / (2 * h)
            if c == 2:
                assert g[v, c] == 0.0
            else:
                assert abs(g[v, c] - num) <= 2e-3 + 2e-2 * abs(num), (v, c, g[v, c], num)


def test_occlusion_back_triangle_gets_no_gradient(oracle):
    clip, faces, img, tri, vf = _scene(
        oracle, [_clip(-40, -40, .8), _clip(100, -40, .8), _clip(-40, 100, .8),
                 _clip(5.2, 4.7, .2), _clip(11.6, 6.3, .2), _clip(6.4, 11.8, .2)],
        [[0, 1, 2], [3, 4, 5]], [0.2, 0.2, 0.2, 0.9, 0.9, 0.9])
    gy = np.full((S, S), 1.0 / (S * S), np.float32)  # d mean(AA) / d AA
    g = oracle.antialias_bwd_vtx(gy, img, tri, clip, faces, vf, 0.0, 0)
    assert np.abs(g[:3]).sum() == 0.0
    assert np.abs(g[3:]).sum() > 1e-4


def test_col_sum_is_the_row_sum(oracle):
    x = np.random.default_rng(1).standard_normal((5, 7, 4)).astype(np.float32)
    want = np.zeros((7, 4), np.float32)
    for r in range(5):
        want = want + x[r]
    _exact(oracle.col_sum(x), want, "col_sum")
