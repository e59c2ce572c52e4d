"""Pins the oracle's split-sum PBR / IBL path (oracle/pbr_oracle.c) before it
is trusted as the checker of the HIP path:

* bit-exact against the reference's own CPU evaluator through the committed
  fixtures (tests/golden/ibl_unit.npz, pbr_*.npz from
  tests/golden/make_golden.py): EquirectSample and its map VJP (1 / 3 / 4
  components; zero-length, pole and seam directions), AvgPool2x2 and its VJP
  (odd and even sizes), IrradianceConv / PrefilterConv at roughness 0, 0.5, 1
  and their transposes, PrefilterEnv, the BRDF LUT;
* the C5-shaped fit (BuildPbrGBuffer + BuildPbrShade, IBL maps of the
  optimised env, L1 loss, Adam on albedo / mr / env): first-iteration images
  bit-exact; gradients within 1e-4 of the largest entry and parameters within
  1e-5 after 2-3 iterations (the reference's autodiff adds the same terms in
  another order);
* against what the mathematics fixes: every backward is the exact adjoint of
  its forward (<A x, y> = <x, A^T y> in double), a constant environment L0
  prefilters to L0 at every roughness (up to the float sums) and irradiates to L0 up to the
  quadrature error, the LUT's A + B lies in [0, 1] and tends to 1 for smooth
  surfaces seen head-on, and the fit's env gradient matches central finite
  differences of its loss.
"""
import numpy as np
import pytest


def _exact(a, b, what=""):
    assert a.shape == b.shape, (what, a.shape, b.shape)
    if not np.array_equal(a, b):
        d = np.abs(a.astype(np.float64) - b)
        raise AssertionError(f"{what}: not bit-exact, max diff {d.max():.3g}, "
                             f"{int((d > 0).sum())} differ")


def _close(a, b, tol, what=""):
    """|a - b| <= tol * max|b| everywhere."""
    assert a.shape == b.shape, (what, a.shape, b.shape)
    d = np.abs(a.astype(np.float64) - b).max()
    m = np.abs(b).max()
    assert d <= tol * max(m, 1e-30), f"{what}: max diff {d:.3g} vs max {m:.3g} (tol {tol})"


def test_ibl_ops_match_reference_fixtures(oracle, golden):
    g = golden("ibl_unit.npz")
    for nc in (1, 3, 4):
        m, d, gy = g[f"in_eq{nc}_map"], g[f"in_eq{nc}_dir"], g[f"in_eq{nc}_gy"]
        _exact(oracle.equirect_sample(m, d), g[f"out_eq{nc}"], f"equirect n={nc}")
        _exact(oracle.equirect_sample(m, d, gy), g[f"out_eq{nc}_bwd"], f"equirect bwd n={nc}")
    for name in ("pool_odd", "pool_even"):
        x, gy = g[f"in_{name}_x"], g[f"in_{name}_gy"]
        _exact(oracle.avg_pool2x2(x), g[f"out_{name}"], name)
        _exact(oracle.avg_pool2x2(x, gy), g[f"out_{name}_bwd"], name + " bwd")
    env, g84, g168 = g["in_env"], g["in_g84"], g["in_g168"]
    _exact(oracle.irradiance_conv(env, 8, 4), g["out_irr"], "irradiance")
    _exact(oracle.irradiance_conv(env, 8, 4, g84), g["out_irr_bwd"], "irradiance bwd")
    for i, rough in enumerate((0.0, 0.5, 1.0)):
        _exact(oracle.prefilter_conv(env, 16, 8, rough), g[f"out_pref{i}_16"], f"pref {rough}")
        _exact(oracle.prefilter_conv(env, 8, 4, rough), g[f"out_pref{i}_8"], f"pref {rough}")
        _exact(oracle.prefilter_conv(env, 16, 8, rough, g168), g[f"out_pref{i}_16_bwd"],
               f"pref bwd {rough}")
        _exact(oracle.prefilter_conv(env, 8, 4, rough, g84), g[f"out_pref{i}_8_bwd"],
               f"pref bwd {rough}")
    _exact(oracle.prefilter_env(env, 8, 4, 0.5, 64), g["out_prefenv"], "prefilter env")
    _exact(oracle.brdf_lut(16, 16, 64), g["out_lut16"], "lut 16")
    _exact(oracle.brdf_lut(64, 64, 512), g["out_lut64"], "lut 64")


def _scene(g):
    keys = ("pos", "normal", "uv", "faces", "mvps", "frames", "light", "gt_albedo", "gt_mr",
            "gt_env", "albedo0", "mr0", "env0")
    sc = {k: g["in_" + k] for k in keys}
    sc.update(screen=int(g["in_screen"]), levels=int(g["in_levels"]), lr=float(g["in_lr"]))
    return sc


@pytest.mark.parametrize("name", ["pbr_ico2_48px_2view_3it.npz", "pbr_ico3_96px_3view_2it.npz"])
def test_pbr_fit_matches_reference(oracle, golden, name):
    g = golden(name)
    iters = len(g["out_loss"])
    images = "out_pred0" in g
    r = oracle.pbr_fit(_scene(g), iters=iters, want_images=images)
    for k in ("pred0", "target0", "mask0"):
        if images:
            _exact(r[k], g["out_" + k], k)
    # the loss is F::Mean's Reduce2x2Sum pyramid, CompSum and the views'
    # SumPixelWise tree in the reference's order: bit for bit
    _exact(np.asarray(r["loss"], np.float32), g["out_loss"], "loss")
    for k in ("g_albedo0", "g_mr0", "g_env0"):
        _close(r[k], g["out_" + k], 1e-4, k)
    for k in ("albedo", "mr", "env"):
        _close(r[k], g["out_" + k], 1e-5, k)


def test_ibl_backwards_are_adjoints(oracle):
    """<A x, y> = <x, A^T y> for every linear IBL op and its VJP."""
    rng = np.random.default_rng(3)

    def dot(a, b):
        return float(np.sum(a.astype(np.float64) * b))

    m = rng.random((8, 16, 3)).astype(np.float32)
    d = rng.standard_normal((10, 12, 3)).astype(np.float32)
    y = rng.standard_normal((10, 12, 3)).astype(np.float32)
    lhs, rhs = dot(oracle.equirect_sample(m, d), y), dot(m, oracle.equirect_sample(m, d, y))
    assert abs(lhs - rhs) <= 1e-5 * abs(lhs)
    x = rng.random((16, 32, 3)).astype(np.float32)
    y = rng.standard_normal((8, 16, 3)).astype(np.float32)
    lhs, rhs = dot(oracle.avg_pool2x2(x), y), dot(x, oracle.avg_pool2x2(x, y))
    assert abs(lhs - rhs) <= 1e-5 * abs(lhs)
    env = rng.random((8, 16, 3)).astype(np.float32)
    y = rng.standard_normal((4, 8, 3)).astype(np.float32)
    lhs = dot(oracle.irradiance_conv(env, 8, 4), y)
    rhs = dot(env, oracle.irradiance_conv(env, 8, 4, y))
    assert abs(lhs - rhs) <= 1e-5 * abs(lhs)
    for rough in (0.0, 0.3, 1.0):
        lhs = dot(oracle.prefilter_conv(env, 8, 4, rough), y)
        rhs = dot(env, oracle.prefilter_conv(env, 8, 4, rough, y))
        assert abs(lhs - rhs) <= 1e-5 * abs(lhs), rough


def test_constant_environment_closed_forms(oracle):
    """A constant environment L0: every prefiltered level is L0 (normalised
    convolution); the irradiance map E(N)/pi is L0 up to the midpoint
    quadrature of the cosine lobe; PrefilterEnv returns L0."""
    L0 = np.full((32, 64, 3), 0.7, np.float32)
    for rough in (0.0, 0.25, 1.0):
        p = oracle.prefilter_conv(L0, 16, 8, rough)
        assert np.allclose(p, 0.7, rtol=2e-5, atol=0), (rough, np.abs(p - 0.7).max())
    irr = oracle.irradiance_conv(L0, 16, 8)
    assert np.allclose(irr, 0.7, rtol=5e-3, atol=0), np.abs(irr - 0.7).max()
    pe = oracle.prefilter_env(L0, 8, 4, 0.5, 64)
    assert np.allclose(pe, 0.7, rtol=1e-5, atol=0)


def test_brdf_lut_bounds(oracle):
    lut = oracle.brdf_lut(32, 32, 256).astype(np.float64)
    s = lut[..., 0] + lut[..., 1]
    assert (lut >= 0).all() and (s <= 1.0 + 1e-5).all()
    # smooth surface seen head-on: A + B -> 1 (all samples reflect to V)
    assert s[0, -1] > 0.98


def test_pbr_env_gradient_matches_finite_differences(oracle, golden):
    """The fit's iteration-0 env gradient (shading chain -> EquirectSample
    VJPs of the background, irradiance and prefilter maps -> conv transposes
    -> pooling VJPs) against central differences of its loss on the texels
    with the largest gradient per channel (the L1 loss is piecewise smooth:
    steps small enough to keep every pixel's sign). The material gradients
    come from GatherByInverseUVBilinear, which is the reference's tent-weighted
    approximation of TextureBilinear's transpose, not its exact adjoint: they
    are pinned by the reference fixtures above."""
    g = golden("pbr_ico2_48px_2view_3it.npz")
    sc = _scene(g)
    base = oracle.pbr_fit(sc, iters=1, want_images=False)
    for ch in range(3):
        gg = np.abs(base["g_env0"][..., ch])
        idx = np.unravel_index(np.argmax(gg), gg.shape) + (ch,)
        h = 1e-2
        vals = []
        for s in (+1, -1):
            sc2 = dict(sc)
            arr = sc["env0"].copy()
            arr[idx] += s * h
            sc2["env0"] = arr
            vals.append(float(oracle.pbr_fit(sc2, iters=1, want_images=False)["loss"][0]))
        fd = (vals[0] - vals[1]) / (2 * h)
        an = float(base["g_env0"][idx])
        assert abs(fd - an) <= 0.02 * abs(an) + 1e-7, (idx, fd, an)
