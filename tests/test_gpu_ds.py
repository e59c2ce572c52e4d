"""GPU parity of GatherDistGrad (dressi_gather_dist_grad) against the
reference fixture and the oracle, through the C ABI: bit-exact wide partials
and {V,1} sums."""
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


def test_gather_dist_grad_matches_reference_fixture(ctx, golden, oracle):
    from opendressi_amd import ops
    g = golden("ds_unit.npz")
    r = float(g["in_cfg"][1])
    for i in range(3):
        print(f"[dist grad] fixture scene {i}", flush=True)
        args = (dev(g[f"in_gy{i}"]), dev(g[f"in_rs{i}"]), dev(g[f"in_clip{i}"]), dev(g["in_faces"]),
                dev(g["in_vf"]), r)
        _exact(host(ops.gather_dist_grad(ctx, *args, wide=True)), g[f"out_wide{i}"], f"wide {i}")
        flat = oracle.gather_dist_grad(g[f"in_gy{i}"], g[f"in_rs{i}"], g[f"in_clip{i}"],
                                       g["in_faces"], g["in_vf"], wide=False)
        _exact(host(ops.gather_dist_grad(ctx, *args, wide=False)), flat, f"flat {i}")
    ctx.synchronize()


@pytest.mark.parametrize("level,s,seed", [(2, 64, 0), (3, 97, 1)])
def test_gather_dist_grad_matches_oracle(ctx, oracle, level, s, seed):
    from opendressi_amd import ops
    print(f"[dist grad] random level={level} s={s} seed={seed}", flush=True)
    rng = np.random.default_rng(seed)
    pos, faces = oracle.icosphere(level)
    proj = oracle.perspective_vk(45.0 * 3.14159265 / 180.0, 1.0, 0.1, 10.0)
    eye = [rng.standard_normal() * 0.6, rng.standard_normal() * 0.6, 2.5]
    clip = oracle.transform_to_clip(pos, oracle.mat4_mul(proj, oracle.look_at(eye)))
    nf = len(faces)
    fid = np.repeat(np.arange(nf, dtype=np.float32), 3)[:, None]
    fs = np.arange(3 * nf, dtype=np.float32).reshape(nf, 3)
    vf = oracle.vertex_faces_tex(faces, len(pos))
    soft = oracle.soft_clip(clip, faces, s, s, 3.0)
    rs = oracle.rasterize_soft(soft, fid, fs, clip, faces, s, s, 3.0)
    gy = rng.standard_normal((s, s, 4)).astype(np.float32)
    gy[rng.random((s, s)) < 0.3, 0] = 0.0
    for wide in (True, False):
        got = host(ops.gather_dist_grad(ctx, dev(gy), dev(rs), dev(clip), dev(faces), dev(vf),
                                        3.0, wide=wide))
        _exact(got, oracle.gather_dist_grad(gy, rs, clip, faces, vf, wide=wide),
               f"wide={wide}")
    ctx.synchronize()
