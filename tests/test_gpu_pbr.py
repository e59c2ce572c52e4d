"""GPU parity of the split-sum IBL ops (C5) against the reference fixtures and
the oracle, through the C ABI per-op entry points.

Bit-exact: AvgPool2x2 and its VJP, IrradianceConv / PrefilterConvNorm /
PrefilterConv and their transposes (one thread per output texel, the
reference's loop order, the reference's texel-centre direction tables).
Within tolerance (written per test): the ops that map per-direction uv with
atan2 / acos on the device (EquirectSample, PrefilterEnv: the reference's
float library calls differ from correctly rounded results by an ulp on some
inputs), EquirectSample's VJP (exact fixed-point sum vs the reference's float
sums) and the BRDF LUT (pow).
"""
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _exact(a, b, what):
    assert a.shape == b.shape, (what, a.shape, b.shape)
    if not np.array_equal(a, b):
        d = np.abs(a.astype(np.float64) - b)
        idx = np.unravel_index(d.argmax(), d.shape)
        raise AssertionError(f"{what}: {int((d > 0).sum())} values differ, max {d.max():.3g} at "
                             f"{idx}: got {a[idx]} want {b[idx]}")


def _close(a, b, tol, what):
    """|a - b| <= tol * max|b|."""
    assert a.shape == b.shape, (what, a.shape, b.shape)
    d = np.abs(a.astype(np.float64) - b).max()
    m = float(np.abs(b).max())
    assert d <= tol * max(m, 1e-30), f"{what}: max diff {d:.3g} vs max {m:.3g} (tol {tol})"


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


def smooth_map(h, w, nc, seed):
    """A smooth positive equirect map (low-frequency sinusoids, periodic in u)."""
    rng = np.random.default_rng(seed)
    yy, xx = np.meshgrid((np.arange(h) + 0.5) / h, (np.arange(w) + 0.5) / w, indexing="ij")
    out = np.zeros((h, w, nc))
    for c in range(nc):
        a, b, p = rng.integers(1, 3), rng.integers(1, 3), rng.random() * 6.28
        out[..., c] = 1.0 + 0.5 * np.sin(2 * math.pi * a * xx + p) * np.sin(math.pi * b * yy)
    return out.astype(np.float32)


def test_ibl_ops_match_reference_fixtures(ctx, golden):
    from opendressi_amd import ops
    g = golden("ibl_unit.npz")
    print("[ibl ops] fixtures: pool / irradiance / prefilter", flush=True)
    for name in ("pool_odd", "pool_even"):
        x, gy = g[f"in_{name}_x"], g[f"in_{name}_gy"]
        _exact(host(ops.avg_pool2x2(ctx, dev(x))), g[f"out_{name}"], name)
        _exact(host(ops.avg_pool2x2_bwd(ctx, dev(gy), x.shape[1], x.shape[0])),
               g[f"out_{name}_bwd"], name + " bwd")
    env, g84, g168 = dev(g["in_env"]), dev(g["in_g84"]), dev(g["in_g168"])
    _exact(host(ops.irradiance_conv(ctx, env, 8, 4)), g["out_irr"], "irradiance")
    _exact(host(ops.irradiance_conv_bwd(ctx, g84, 16, 8)), g["out_irr_bwd"], "irradiance bwd")
    for i, rough in enumerate((0.0, 0.5, 1.0)):
        _exact(host(ops.prefilter_conv(ctx, env, 16, 8, rough)), g[f"out_pref{i}_16"],
               f"pref {rough}")
        _exact(host(ops.prefilter_conv(ctx, env, 8, 4, rough)), g[f"out_pref{i}_8"],
               f"pref {rough}")
        _exact(host(ops.prefilter_conv_bwd(ctx, g168, 16, 8, rough)), g[f"out_pref{i}_16_bwd"],
               f"pref bwd {rough}")
        _exact(host(ops.prefilter_conv_bwd(ctx, g84, 16, 8, rough)), g[f"out_pref{i}_8_bwd"],
               f"pref bwd {rough}")
    print("[ibl ops] fixtures: equirect / prefilter env / lut", flush=True)
    for nc in (1, 3, 4):
        m, d, gy = g[f"in_eq{nc}_map"], g[f"in_eq{nc}_dir"], g[f"in_eq{nc}_gy"]
        # random (non-smooth) maps: an ulp of u moves a tap weight by ~w * 1e-7
        _close(host(ops.equirect_sample(ctx, dev(m), dev(d))), g[f"out_eq{nc}"], 1e-5,
               f"equirect n={nc}")
        _close(host(ops.equirect_sample_bwd(ctx, dev(gy), dev(d), m.shape[1], m.shape[0])),
               g[f"out_eq{nc}_bwd"], 1e-5, f"equirect bwd n={nc}")
    _close(host(ops.prefilter_env(ctx, env, 8, 4, 0.5, 64)), g["out_prefenv"], 1e-5,
           "prefilter env")
    _close(host(ops.brdf_lut(ctx, 16, 16, 64)), g["out_lut16"], 1e-6, "lut 16")
    _close(host(ops.brdf_lut(ctx, 64, 64, 512)), g["out_lut64"], 1e-6, "lut 64")


@pytest.mark.parametrize("shape", [(64, 128, 128, 64), (32, 64, 32, 16)])
def test_ibl_convs_match_oracle_at_map_sizes(ctx, oracle, shape):
    """The C5 map sizes: prefilter levels from a 128 x 64 source, the
    irradiance map 32 x 16 from 64 x 32 (bit-exact)."""
    from opendressi_amd import ops
    sh, sw, oh, ow = shape
    print(f"[ibl convs] src {sw}x{sh} -> {ow}x{oh}", flush=True)
    env = smooth_map(sh, sw, 3, 5)
    rng = np.random.default_rng(6)
    gy = rng.standard_normal((oh, ow, 3)).astype(np.float32)
    for rough in (0.0, 0.6):
        _exact(host(ops.prefilter_conv(ctx, dev(env), ow, oh, rough)),
               oracle.prefilter_conv(env, ow, oh, rough), f"pref {rough}")
        _exact(host(ops.prefilter_conv_bwd(ctx, dev(gy), sw, sh, rough)),
               oracle.prefilter_conv(env, ow, oh, rough, gy), f"pref bwd {rough}")
    _exact(host(ops.irradiance_conv(ctx, dev(env), ow // 2, oh // 2)),
           oracle.irradiance_conv(env, ow // 2, oh // 2), "irradiance")


def test_equirect_sample_smooth_map_and_vjp(ctx, oracle):
    """A 512 x 256 smooth map sampled at 96 x 80 random directions (images
    1e-5), and the map VJP of 1024 x 8 directions (gradients 1e-5)."""
    from opendressi_amd import ops
    print("[equirect] 512x256 smooth map", flush=True)
    m = smooth_map(256, 512, 3, 7)
    rng = np.random.default_rng(8)
    d = rng.standard_normal((80, 96, 3)).astype(np.float32)
    _close(host(ops.equirect_sample(ctx, dev(m), dev(d))), oracle.equirect_sample(m, d), 1e-5,
           "equirect")
    d2 = rng.standard_normal((8, 1024, 3)).astype(np.float32)
    gy = rng.standard_normal((8, 1024, 3)).astype(np.float32)
    got = host(ops.equirect_sample_bwd(ctx, dev(gy), dev(d2), 64, 32))
    _close(got, oracle.equirect_sample(np.zeros((32, 64, 3), np.float32), d2, gy), 1e-5,
           "equirect vjp")
    # determinism: the fixed-point sum does not depend on the atomics' order
    again = host(ops.equirect_sample_bwd(ctx, dev(gy), dev(d2), 64, 32))
    _exact(again, got, "equirect vjp rerun")
