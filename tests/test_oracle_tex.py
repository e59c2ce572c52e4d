"""Pins the oracle's texture path (oracle/dressi_oracle.c or_uv_sphere /
or_texture_bilinear / or_gather_inv_uv_bilinear / or_screen_attr /
or_uv_as_clip / or_tex_fit) before it is trusted as the checker of the HIP
path:

* bit-exact against the reference's own CPU evaluator through the committed
  fixtures (tests/golden/tex_*.npz from tests/golden/make_golden.py): per-op
  scenes (TextureBilinear with 1 / 3 / 4 components in and out of the clamp
  region, GatherByInverseUVBilinear with covered and uncovered inverse-UV
  entries, the UV-sphere generator) and the C3-shaped texture fit (3 and 8
  views, first-iteration images and gradient, a 20-iteration trajectory);
* against what the mathematics fixes: the exact interpolation values of
  tests/test_cpu_eval.cpp:534-561; on the clamp-free scene of
  tests/test_backward.cpp:415-456 (every contributing pixel inside its
  texel's +-3 window) the gather is the exact adjoint of TextureBilinear,
  <B t, g> = <t, G g>, and the texture gradient of a quadratic loss matches
  central finite differences; the UV-sphere counts (stacks + 1)(slices + 1)
  and 2 stacks slices - 2 slices; UvAsClip / ScreenAttr closed forms.
"""
import numpy as np
import pytest


def _exact(a, b, what=""):
    assert a.shape == b.shape, (what, a.shape, b.shape)
    if not np.array_equal(a, b):
        d = np.abs(a.astype(np.float64) - b)
        raise AssertionError(f"{what}: not bit-exact, max diff {d.max():.3g}, "
                             f"{int((d > 0).sum())} differ")


def test_texture_ops_match_reference_fixtures(oracle, golden):
    g = golden("tex_unit.npz")
    for nc in (1, 3, 4):
        _exact(oracle.texture_bilinear(g[f"in_bl{nc}_tex"], g[f"in_bl{nc}_uv"]),
               g[f"out_bl{nc}"], f"bilinear n={nc}")
    for name in ("g_small", "g_sparse"):
        _exact(oracle.gather_inv_uv_bilinear(g[f"in_{name}_gy"], g[f"in_{name}_iv"],
                                             g[f"in_{name}_uv"]), g[f"out_{name}"], name)
    pos, uv, faces = oracle.uv_sphere(16, 8)
    _exact(pos, g["out_uvs16_pos"], "uv sphere pos")
    _exact(uv, g["out_uvs16_uv"], "uv sphere uv")
    _exact(faces, g["out_uvs16_faces"], "uv sphere faces")
    p2, _, f2 = oracle.uv_sphere(128, 64)
    assert [len(p2), len(f2)] == list(g["out_uvs128_counts"])


@pytest.mark.parametrize("name", ["tex_uvs16_64px_3view_3it.npz", "tex_uvs32_8view_128px_3it.npz",
                                  "tex_uvs16_64px_20it.npz"])
def test_tex_fit_matches_reference(oracle, golden, name):
    g = golden(name)
    screen, iters = int(g["in_cfg"][0]), int(g["in_cfg"][1])
    images = "out_pred0" in g
    r = oracle.tex_fit(g["in_pos"], g["in_uv"], g["in_faces"], g["in_mvps"], screen, g["in_gt"],
                       g["in_tex0"], lr=float(g["in_cfg"][2]), iters=iters, want_images=images)
    for k, v in r.items():
        _exact(v, g["out_" + k], k)


def test_texture_bilinear_exact_interpolation(oracle):
    """tests/test_cpu_eval.cpp:534-561: texel centres, the centre of all four,
    the midpoint of the top row."""
    tex = np.array([0, 1, 2, 3], np.float32).reshape(2, 2, 1)
    uv = np.array([[.25, .25], [.75, .75], [.5, .5], [.5, .25]], np.float32)
    out = oracle.texture_bilinear(tex, uv)[:, 0]
    assert list(out) == [0.0, 3.0, 1.5, 0.5]


def _clamp_free_scene():
    """tests/test_backward.cpp:415-456: an 8x8 screen sampling a 4x4 texture
    inside the clamp-free region, each texel anchored at its nearest pixel."""
    uv = np.zeros((8, 8, 2), np.float32)
    for py in range(8):
        for px in range(8):
            uv[py, px] = [0.125 + 0.75 * (px + 0.5) / 8, 0.125 + 0.75 * (py + 0.5) / 8]

    def anchor(t):
        p = np.float32(t) / np.float32(0.375)
        return min(p, np.float32(7.0))

    iv = np.zeros((4, 4, 4), np.float32)
    for ty in range(4):
        for tx in range(4):
            iv[ty, tx] = [np.floor(anchor(tx)) + 0.5, np.floor(anchor(ty)) + 0.5, 1, 0]
    return uv, iv


def test_gather_is_the_adjoint_on_the_clamp_free_scene(oracle):
    uv, iv = _clamp_free_scene()
    rng = np.random.default_rng(0)
    for _ in range(3):
        t = rng.standard_normal((4, 4, 1)).astype(np.float32)
        gy = rng.standard_normal((8, 8, 1)).astype(np.float32)
        lhs = float((oracle.texture_bilinear(t, uv).astype(np.float64) * gy).sum())
        rhs = float((t.astype(np.float64) * oracle.gather_inv_uv_bilinear(gy, iv, uv)).sum())
        assert abs(lhs - rhs) <= 1e-5 * (abs(lhs) + 1.0), (lhs, rhs)


def test_texture_gradient_matches_finite_differences(oracle):
    """d/d tex of L = mean(B(tex)^2 + B(tex)) (the loss of
    tests/test_backward.cpp:415-456) by the gather, against central
    differences in float64 of the same forward."""
    uv, iv = _clamp_free_scene()
    tex = np.array([0.2 + 0.11 * ((i * 5) % 7) for i in range(16)], np.float32).reshape(4, 4, 1)
    out = oracle.texture_bilinear(tex, uv)
    gy = ((2.0 * out + 1.0) / out.size).astype(np.float32)
    g = oracle.gather_inv_uv_bilinear(gy, iv, uv)

    def loss(t):
        o = oracle.texture_bilinear(t, uv).astype(np.float64)
        return float((o * o + o).mean())

    h = 1e-2
    for i in range(16):
        tp, tm = tex.copy(), tex.copy()
        tp.flat[i] += h
        tm.flat[i] -= h
        fd = (loss(tp) - loss(tm)) / (2 * h)
        assert abs(fd - g.flat[i]) <= 2e-4 + 1e-3 * abs(fd), (i, fd, g.flat[i])


def test_uv_sphere_counts_and_uv_layout(oracle):
    for st, sl in ((2, 3), (16, 8), (128, 64)):
        pos, uv, faces = oracle.uv_sphere(st, sl)
        assert len(pos) == (st + 1) * (sl + 1)
        assert len(faces) == 2 * st * sl - 2 * sl
        assert np.allclose(np.linalg.norm(pos, axis=1), 1.0, atol=1e-6)
        assert uv.min() == 0.0 and uv.max() == 1.0
    clip = oracle.uv_as_clip(uv)
    assert np.array_equal(clip[:, :2], uv * 2 - 1) and (clip[:, 2] == 0.5).all()
    assert (clip[:, 3] == 1).all()


def test_screen_attr_closed_form(oracle):
    clip = np.array([[0.5, -0.25, 0.3, 2.0], [-1.0, 1.0, 0.0, 1.0]], np.float32)
    a = oracle.screen_attr(clip, 64, 32)
    assert np.array_equal(a, np.array([[40.0, 14.0, 1, 0], [0.0, 32.0, 1, 0]], np.float32))


def test_texture_nearest_closed_forms(oracle):
    """Nearest, clamp-to-edge: pixel (x, y) of an identity uv grid reads
    texel (x, y); uv outside [0, 1) clamps to the edge texels; u = k / tw
    exactly reads texel k."""
    tex = np.arange(6 * 5 * 2, dtype=np.float32).reshape(5, 6, 2)
    ys, xs = np.mgrid[0:5, 0:6]
    uv = np.stack([(xs + 0.5) / 6, (ys + 0.5) / 5], -1).astype(np.float32)
    assert np.array_equal(oracle.texture_nearest(tex, uv), tex)
    uv = np.array([[-0.1, -3.0], [1.0, 1.0], [1.5, 0.2], [2 / 6, 3 / 5], [0.0, 0.999]],
                  np.float32)
    want = np.stack([tex[0, 0], tex[4, 5], tex[1, 5], tex[3, 2], tex[4, 0]])
    assert np.array_equal(oracle.texture_nearest(tex, uv), want)


def _identity_scene(n=8):
    ys, xs = np.mgrid[0:n, 0:n]
    uv = np.stack([(xs + 0.5) / n, (ys + 0.5) / n], -1).astype(np.float32)
    iv = np.zeros((n, n, 4), np.float32)
    iv[..., 0], iv[..., 1], iv[..., 2] = xs + 0.5, ys + 0.5, 1.0
    return uv, iv


def test_gather_inv_uv_is_the_adjoint_on_a_one_to_one_map(oracle):
    """Screen pixel p samples exactly texel p: the gather is the exact
    transpose of the sampling, so <T(t), g> == <t, G(g)> and G(g) == g."""
    uv, iv = _identity_scene()
    rng = np.random.default_rng(3)
    for _ in range(3):
        t = rng.standard_normal((8, 8, 3)).astype(np.float32)
        gy = rng.standard_normal((8, 8, 3)).astype(np.float32)
        g = oracle.gather_inv_uv(gy, iv, uv)
        assert np.array_equal(g, gy)
        lhs = float((oracle.texture_nearest(t, uv).astype(np.float64) * gy).sum())
        rhs = float((t.astype(np.float64) * g).sum())
        assert abs(lhs - rhs) <= 1e-9 * (abs(lhs) + 1.0)


def test_gather_inv_uv_many_to_one_takes_the_first_sampling_pixel(oracle):
    """16x16 screen over a 4x4 texture (each texel sampled by a 4x4 pixel
    block), anchors at the block centres: the 7x7 window's first sampling
    pixel in row order is the block's top-left pixel; a texel whose table
    entry is empty borrows the first covered entry of its +-4 neighbourhood in
    row order (dilation): found for texel (1, 0), whose borrowed window still
    reaches its block, zero for texel (2, 1), whose does not; a texel no pixel
    samples gets zero."""
    n, t = 16, 4
    ys, xs = np.mgrid[0:n, 0:n]
    uv = np.stack([(xs + 0.5) / n, (ys + 0.5) / n], -1).astype(np.float32)
    tys, txs = np.mgrid[0:t, 0:t]
    iv = np.zeros((t, t, 4), np.float32)
    iv[..., 0], iv[..., 1], iv[..., 2] = txs * 4 + 2, tys * 4 + 2, 1.0
    gy = np.random.default_rng(5).standard_normal((n, n, 2)).astype(np.float32)
    g = oracle.gather_inv_uv(gy, iv, uv)
    assert np.array_equal(g, gy[0::4, 0::4])
    iv2 = iv.copy()
    iv2[0, 1, 2] = 0.0  # texel (1, 0) borrows texel (0, 0)'s anchor (2, 2)
    iv2[1, 2, 2] = 0.0  # texel (2, 1) borrows texel (0, 0)'s anchor too
    g2 = oracle.gather_inv_uv(gy, iv2, uv)
    assert np.array_equal(g2[0, 1], gy[0, 4])
    assert (g2[1, 2] == 0).all()
    keep = np.ones((t, t), bool)
    keep[0, 1] = keep[1, 2] = False
    assert np.array_equal(g2[keep], g[keep])
    uv3 = uv.copy()
    uv3[0:4, 0:4] = uv3[0:4, 4:8]  # nobody samples texel (0, 0) any more
    g3 = oracle.gather_inv_uv(gy, iv, uv3)
    assert (g3[0, 0] == 0).all() and np.array_equal(g3[1:, 1:], g[1:, 1:])
