"""The nvdiffrast-compatible surface (opendressi_amd.torch) on the GPU.

Two kinds of checks, following the reference's tests/python suite:
  * behaviour: analytic barycentrics and depth order, finite differences of
    the linear ops, gradient direction of the geometric ops against central
    differences, small end-to-end optimizations with torch's Adam;
  * parity: each op's forward and backward equal the oracle's per-op
    functions composed the way the reference's graph composes them, bit for
    bit (the surface only adds fp32 elementwise torch ops, replayed here in
    numpy float32 with the same operation order).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dr():
    import opendressi_amd.torch as dr
    return dr


@pytest.fixture(scope="module")
def ctx(dr):
    return dr.RasterizeHipContext()


def _np(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def _exact(a, b, what):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    if not np.array_equal(a, b):
        d = np.abs(a.astype(np.float64) - b)
        idx = np.unravel_index(d.argmax(), d.shape)
        raise AssertionError(f"{what}: {int((d > 0).sum())} values differ, max {d.max():.3g} "
                             f"at {idx}: got {a[idx]} want {b[idx]}")


def _bary(pts, px, py):
    (x0, y0), (x1, y1), (x2, y2) = pts
    area = (x1 - x0) * (y2 - y0) - (y1 - y0) * (x2 - x0)
    l0 = ((x1 - px) * (y2 - py) - (y1 - py) * (x2 - px)) / area
    l1 = ((x2 - px) * (y0 - py) - (y2 - py) * (x0 - px)) / area
    return l0, l1, 1.0 - l0 - l1


def _screen(pos, h, w):
    return [((v[0] / v[3] * 0.5 + 0.5) * w, (v[1] / v[3] * 0.5 + 0.5) * h) for v in pos]


def _gl_to_vk(p):
    q = np.array(p, np.float32, copy=True)
    q[..., 2] = np.float32(0.5) * (p[..., 2] + p[..., 3])
    return q


def _grad_vk_to_gl(g):
    q = np.array(g, np.float32, copy=True)
    q[..., 2] = np.float32(0.5) * g[..., 2]
    q[..., 3] = g[..., 3] + np.float32(0.5) * g[..., 2]
    return q


# ------------------------------- rasterize ---------------------------------


def test_rasterize_single_triangle_barycentrics(dr, ctx):
    print("[torch] rasterize single triangle", flush=True)
    h, w = 8, 8
    pos = torch.tensor([[-0.5, -0.5, 0.2, 1.0], [0.5, -0.5, 0.2, 1.0], [-0.5, 0.5, 0.2, 1.0]])
    tri = torch.tensor([[0, 1, 2]], dtype=torch.int32)
    rast, rast_db = dr.rasterize(ctx, pos, tri, resolution=[h, w])
    assert rast.shape == (1, h, w, 4) and rast.device == pos.device
    assert torch.count_nonzero(rast_db) == 0
    pts = _screen(pos.tolist(), h, w)
    covered = 0
    for iy in range(h):
        for ix in range(w):
            l0, l1, l2 = _bary(pts, ix + 0.5, iy + 0.5)
            got = rast[0, iy, ix]
            if min(l0, l1, l2) > 1e-4:
                covered += 1
                assert got[3].item() == 1.0
                assert got[0].item() == pytest.approx(l0, abs=1e-3)
                assert got[1].item() == pytest.approx(l1, abs=1e-3)
                assert got[2].item() == pytest.approx(0.2, abs=1e-4)
            elif min(l0, l1, l2) < -1e-4:
                assert torch.count_nonzero(got).item() == 0
    assert covered > 0


def test_rasterize_perspective_correct(dr, ctx):
    print("[torch] rasterize perspective", flush=True)
    h, w = 16, 16
    pos = torch.tensor([[-0.8, -0.8, 0.0, 1.0], [1.6, -1.6, 1.0, 2.0], [-1.6, 1.6, 1.0, 2.0]])
    tri = torch.tensor([[0, 1, 2]], dtype=torch.int32)
    rast, _ = dr.rasterize(ctx, pos, tri, resolution=[h, w])
    pts = _screen(pos.tolist(), h, w)
    ws = [1.0, 2.0, 2.0]
    zs = [0.0, 1.0, 1.0]
    checked = 0
    for iy in range(h):
        for ix in range(w):
            if rast[0, iy, ix, 3].item() == 0.0:
                continue
            ls = _bary(pts, ix + 0.5, iy + 0.5)
            if min(ls) < 1e-3:
                continue
            q = [l / wk for l, wk in zip(ls, ws)]
            den = sum(q)
            assert rast[0, iy, ix, 0].item() == pytest.approx(q[0] / den, abs=2e-3)
            assert rast[0, iy, ix, 1].item() == pytest.approx(q[1] / den, abs=2e-3)
            z_pc = sum(qk * zk for qk, zk in zip(q, zs)) / den
            w_pc = sum(ls) / den
            assert rast[0, iy, ix, 2].item() == pytest.approx(z_pc / w_pc, abs=2e-3)
            checked += 1
    assert checked > 10


def test_rasterize_depth_order(dr, ctx):
    print("[torch] rasterize depth", flush=True)
    pos = torch.tensor([[-0.9, -0.9, 0.5, 1.0], [0.9, -0.9, 0.5, 1.0], [0.0, 0.9, 0.5, 1.0],
                        [-0.4, -0.4, -0.5, 1.0], [0.4, -0.4, -0.5, 1.0], [0.0, 0.4, -0.5, 1.0]])
    tri = torch.tensor([[0, 1, 2], [3, 4, 5]], dtype=torch.int32)
    rast, _ = dr.rasterize(ctx, pos.cuda(), tri, resolution=[8, 8])
    assert rast.is_cuda
    tid = rast[0, :, :, 3]
    assert (tid == 2.0).any() and (tid == 1.0).any()
    assert tid[3, 3].item() == 2.0
    assert rast[0, 3, 3, 2].item() == pytest.approx(-0.5, abs=1e-4)


def test_engine_cache_reuse(dr, ctx):
    print("[torch] engine cache", flush=True)
    tri = torch.tensor([[0, 1, 2]], dtype=torch.int32)
    p1 = torch.tensor([[-0.5, -0.5, 0.0, 1.0], [0.5, -0.5, 0.0, 1.0], [-0.5, 0.5, 0.0, 1.0]])
    p2 = p1 * torch.tensor([1.5, 1.5, 1.0, 1.0])
    n0 = len(ctx._engines)
    r1, _ = dr.rasterize(ctx, p1, tri, resolution=[6, 6])
    n1 = len(ctx._engines)
    r2, _ = dr.rasterize(ctx, p2, tri, resolution=[6, 6])
    assert len(ctx._engines) == n1 == n0 + 1
    assert not torch.equal(r1, r2)
    dr.rasterize(ctx, p1, tri, resolution=[12, 12])
    assert len(ctx._engines) == n1 + 1


def test_rasterize_batch(dr, ctx):
    print("[torch] rasterize batch", flush=True)
    tri = torch.tensor([[0, 1, 2]], dtype=torch.int32)
    base = torch.tensor([[-0.5, -0.5, 0.0, 1.0], [0.5, -0.5, 0.0, 1.0], [-0.5, 0.5, 0.0, 1.0]])
    pos = torch.stack([base, base * torch.tensor([0.2, 0.2, 1.0, 1.0])])
    rast, _ = dr.rasterize(ctx, pos, tri, resolution=[4, 4])
    assert rast.shape == (2, 4, 4, 4)
    assert (rast[1, :, :, 3] > 0).sum() < (rast[0, :, :, 3] > 0).sum()


def _sphere(level=2, seed=0, jitter=0.03):
    import opendressi_amd as od
    p, f = od.icosphere(level)
    rng = np.random.default_rng(seed)
    p = p * (1.0 + jitter * rng.standard_normal((len(p), 1))).astype(np.float32)
    clip = np.concatenate([p[:, :2] * 0.7, p[:, 2:3] * 0.5, np.ones((len(p), 1))], 1)
    clip[:, 3] += 0.1 * p[:, 2]
    return clip.astype(np.float32), f.astype(np.int64)


def test_rasterize_matches_oracle(dr, ctx, oracle):
    """rast = (u, v, z/w, id+1) from the oracle's Rasterize of the unwelded
    corners (barycentric constants, z, w) and RasterizeFaceId."""
    print("[torch] rasterize parity", flush=True)
    clip_gl, faces = _sphere()
    h, w = 48, 40
    rast, _ = dr.rasterize(ctx, torch.from_numpy(clip_gl).cuda(),
                           torch.from_numpy(faces).cuda(), resolution=[h, w])
    nf = len(faces)
    unweld = faces.reshape(-1)
    clip3 = _gl_to_vk(clip_gl)[unweld]
    corner = np.tile(np.array([[1, 0], [0, 1], [0, 0]], np.float32), (nf, 1))
    attr4 = np.concatenate([corner, clip_gl[unweld][:, 2:4]], 1)
    seq = np.arange(3 * nf, dtype=np.float32).reshape(nf, 3)
    g = oracle.rasterize(clip3, attr4, seq, w, h)
    tid = oracle.rasterize_face_id(clip3, seq, w, h)
    mask = (tid > 0.5).astype(np.float32)
    zw = g[..., 2] / (g[..., 3] + (np.float32(1.0) - mask))
    want = np.stack([g[..., 0], g[..., 1], zw, tid], -1)[None]
    _exact(_np(rast), want, "rast")
    assert (tid > 0).sum() > 300


# ------------------------------ interpolate --------------------------------


def _quad_scene():
    pos = torch.tensor([[-0.8, -0.8, 0.2, 1.0], [0.8, -0.6, 0.2, 1.0], [-0.6, 0.8, 0.2, 1.0],
                        [0.9, 0.9, 0.2, 1.0]])
    tri = torch.tensor([[0, 1, 2], [1, 3, 2]], dtype=torch.int32)
    return pos, tri


def test_interpolate_forward_matches_barycentrics(dr, ctx):
    print("[torch] interpolate forward", flush=True)
    pos, tri = _quad_scene()
    attr = torch.tensor([[1.0, 10.0, -1.0], [2.0, 20.0, -2.0], [3.0, 30.0, -3.0],
                         [4.0, 40.0, -4.0]])
    rast, _ = dr.rasterize(ctx, pos, tri, resolution=[16, 16])
    out, none = dr.interpolate(attr, rast, tri)
    assert none is None and out.shape == (1, 16, 16, 3)
    covered = 0
    for iy in range(16):
        for ix in range(16):
            u, v, _, tid = rast[0, iy, ix].tolist()
            if tid == 0.0:
                assert torch.count_nonzero(out[0, iy, ix]).item() == 0
                continue
            covered += 1
            i0, i1, i2 = tri[int(tid) - 1].tolist()
            want = u * attr[i0] + v * attr[i1] + (1 - u - v) * attr[i2]
            assert torch.allclose(out[0, iy, ix], want, atol=2e-3)
    assert covered > 20


def test_interpolate_grad_matches_fd(dr, ctx):
    print("[torch] interpolate fd", flush=True)
    pos, tri = _quad_scene()
    attr0 = torch.tensor([[0.5], [1.5], [-0.7], [2.2]])
    weight = torch.linspace(-1.0, 1.0, 144).reshape(1, 12, 12, 1)
    rast, _ = dr.rasterize(ctx, pos, tri, resolution=[12, 12])

    def loss_of(a):
        out, _ = dr.interpolate(a, rast, tri)
        return (out * weight).sum()

    attr = attr0.clone().requires_grad_(True)
    loss_of(attr).backward()
    for i in range(4):
        d = torch.zeros_like(attr0)
        d[i, 0] = 1e-2
        with torch.no_grad():
            fd = (loss_of(attr0 + d) - loss_of(attr0 - d)) / 2e-2
        assert attr.grad[i, 0].item() == pytest.approx(fd.item(), abs=1e-2, rel=1e-3)


def test_interpolate_batched_attr(dr, ctx):
    print("[torch] interpolate batched", flush=True)
    pos, tri = _quad_scene()
    rast, _ = dr.rasterize(ctx, torch.stack([pos, pos]), tri, resolution=[8, 8])
    attr = torch.rand(2, 4, 2)
    out, _ = dr.interpolate(attr, rast, tri)
    assert out.shape == (2, 8, 8, 2)
    assert not torch.equal(out[0], out[1])


@pytest.mark.parametrize("shared", [True, False])
def test_interpolate_matches_oracle(dr, ctx, oracle, shared):
    """Forward: u p0 + v p1 + ((1 - u) - v) p2 with p_k = FaceFetch(
    LookupFaces(attr, k)); backward: per item and corner k = 2, 1, 0,
    LookupFacesBwd(FaceFetchBwd(gy * weight_k, exact)), summed in that order
    (and over items, last first, when attr is shared)."""
    print(f"[torch] interpolate parity shared={shared}", flush=True)
    clip_gl, faces = _sphere(seed=1)
    nv, nf = len(clip_gl), len(faces)
    h, w, n = 40, 44, 2
    rng = np.random.default_rng(7)
    pos = np.stack([clip_gl, clip_gl * np.float32(0.9)])
    attr_np = rng.standard_normal((nv, 3) if shared else (n, nv, 3)).astype(np.float32)
    gy = rng.standard_normal((n, h, w, 3)).astype(np.float32)
    tri = torch.from_numpy(faces).cuda()
    rast, _ = dr.rasterize(ctx, torch.from_numpy(pos).cuda(), tri, resolution=[h, w])
    attr = torch.from_numpy(attr_np).cuda().requires_grad_(True)
    out, _ = dr.interpolate(attr, rast, tri)
    out.backward(torch.from_numpy(gy).cuda())
    r = _np(rast)
    ff = faces.astype(np.float32)
    vft = oracle.vertex_faces_tex(ff, nv)
    want_out, contribs = [], []
    for i in range(n):
        a = attr_np if shared else attr_np[i]
        u, v, tid = r[i, ..., 0:1], r[i, ..., 1:2], r[i, ..., 3]
        p = [oracle.face_fetch(oracle.lookup_faces(a, ff, k), tid) for k in range(3)]
        want_out.append(u * p[0] + v * p[1] + ((np.float32(1.0) - u) - v) * p[2])
        prj = [oracle.lookup_faces(_gl_to_vk(pos[i]), ff, k) for k in range(3)]
        wk = [u, v, (np.float32(1.0) - u) - v]
        item = []
        for k in (2, 1, 0):
            gf = oracle.face_fetch_bwd(gy[i] * wk[k], tid, prj[0], prj[1], prj[2], 0.0, 1.0, 0)
            item.append(oracle.lookup_faces_bwd(gf, ff, vft, k))
        contribs.append(item)
    _exact(_np(out), np.stack(want_out), "interpolate")
    if shared:
        flat = [c for item in reversed(contribs) for c in item]  # 6 -> (4 summed) + (2 summed)
        s0 = ((flat[0] + flat[1]) + flat[2]) + flat[3]
        want_g = s0 + (flat[4] + flat[5])
    else:
        want_g = np.stack([(c[0] + c[1]) + c[2] for c in contribs])
    _exact(_np(attr.grad), want_g, "interpolate grad")
    assert np.abs(want_g).max() > 0


# -------------------------------- texture ----------------------------------


def _fullscreen_quad():
    pos = torch.tensor([[-1.0, -1.0, 0.0, 1.0], [1.0, -1.0, 0.0, 1.0], [-1.0, 1.0, 0.0, 1.0],
                        [1.0, 1.0, 0.0, 1.0]])
    uv = torch.tensor([[0.0, 0.0], [1.0, 0.0], [0.0, 1.0], [1.0, 1.0]])
    tri = torch.tensor([[0, 1, 2], [1, 3, 2]], dtype=torch.int32)
    return pos, uv, tri


def test_texture_nearest_identity(dr, ctx):
    print("[torch] texture identity", flush=True)
    pos, uv, tri = _fullscreen_quad()
    tex = torch.arange(64, dtype=torch.float32).reshape(8, 8, 1)
    rast, _ = dr.rasterize(ctx, pos, tri, resolution=[8, 8])
    uv_img, _ = dr.interpolate(uv, rast, tri)
    out = dr.texture(tex, uv_img)
    assert out.shape == (1, 8, 8, 1)
    assert torch.equal(out[0], tex)


def test_texture_grad_matches_fd(dr, ctx):
    print("[torch] texture fd", flush=True)
    pos, uv, tri = _fullscreen_quad()
    tex0 = torch.rand(8, 8, 2)
    weight = torch.rand(1, 8, 8, 2) - 0.5
    rast, _ = dr.rasterize(ctx, pos, tri, resolution=[8, 8])
    uv_img, _ = dr.interpolate(uv, rast, tri)

    def loss_of(t):
        return (dr.texture(t, uv_img) * weight).sum()

    tex = tex0.clone().requires_grad_(True)
    loss_of(tex).backward()
    flat0 = tex0.reshape(-1)
    for i in range(0, flat0.numel(), 7):
        d = torch.zeros_like(flat0)
        d[i] = 1e-2
        d = d.reshape(tex0.shape)
        with torch.no_grad():
            fd = (loss_of(tex0 + d) - loss_of(tex0 - d)) / 2e-2
        assert tex.grad.reshape(-1)[i].item() == pytest.approx(fd.item(), abs=1e-2, rel=1e-3)


def test_texture_no_grad_and_errors(dr, ctx):
    print("[torch] texture no-grad", flush=True)
    pos, uv, tri = _fullscreen_quad()
    rast, _ = dr.rasterize(ctx, pos, tri, resolution=[8, 8])
    uv_img, _ = dr.interpolate(uv, rast, tri)
    with torch.no_grad():
        out = dr.texture(torch.rand(4, 4, 3), uv_img)
    assert out.shape == (1, 8, 8, 3)
    with pytest.raises(RuntimeError):
        dr.texture(torch.rand(4, 4, 3), uv_img.clone())  # no provenance
    with pytest.raises(NotImplementedError):
        dr.texture(torch.rand(4, 4, 3), uv_img, filter_mode="linear")


def test_texture_matches_oracle(dr, ctx, oracle):
    """Forward = nearest sampling of the interpolated uv; backward =
    GatherByInverseUV through the table Rasterize(UvAsClip(uv),
    ScreenAttr(clip), T), items summed last first."""
    print("[torch] texture parity", flush=True)
    clip_gl, faces = _sphere(seed=2)
    nv = len(clip_gl)
    rng = np.random.default_rng(11)
    uv_v = rng.random((nv, 2)).astype(np.float32)
    h, w, th, tw = 36, 40, 24, 20
    pos = np.stack([clip_gl, clip_gl * np.float32(1.1)])
    tri = torch.from_numpy(faces).cuda()
    rast, _ = dr.rasterize(ctx, torch.from_numpy(pos).cuda(), tri, resolution=[h, w])
    uv_img, _ = dr.interpolate(torch.from_numpy(uv_v).cuda(), rast, tri)
    tex_np = rng.random((th, tw, 3)).astype(np.float32)
    tex = torch.from_numpy(tex_np).cuda().requires_grad_(True)
    out = dr.texture(tex, uv_img)
    gy = rng.standard_normal((2, h, w, 3)).astype(np.float32)
    out.backward(torch.from_numpy(gy).cuda())
    uvi = _np(uv_img)
    _exact(_np(out), np.stack([oracle.texture_nearest(tex_np, uvi[i]) for i in range(2)]),
           "texture")
    ff = faces.astype(np.float32)
    uvc = oracle.uv_as_clip(uv_v)
    contribs = []
    for i in (1, 0):
        iv = oracle.rasterize(uvc, oracle.screen_attr(_gl_to_vk(pos[i]), w, h), ff, tw, th)
        contribs.append(oracle.gather_inv_uv(gy[i], iv, uvi[i]))
    want = contribs[0] + contribs[1]
    _exact(_np(tex.grad), want, "texture grad")
    assert (want != 0).sum() > 50


def test_texture_fit_converges(dr, ctx):
    print("[torch] texture fit", flush=True)
    torch.manual_seed(0)
    s = 0.8
    pos = torch.tensor([[-s, -s, 0.0, 1.0], [s, -s, 0.0, 1.0], [-s, s, 0.0, 1.0], [s, s, 0.0, 1.0]])
    uv = torch.tensor([[0.0, 0.0], [1.0, 0.0], [0.0, 1.0], [1.0, 1.0]])
    tri = torch.tensor([[0, 1, 2], [1, 3, 2]], dtype=torch.int32)
    gt = torch.rand(8, 8, 3)
    rast, _ = dr.rasterize(ctx, pos, tri, resolution=[24, 24])
    uv_img, _ = dr.interpolate(uv, rast, tri)
    with torch.no_grad():
        target = dr.texture(gt, uv_img)
    tex = torch.full((8, 8, 3), 0.5, requires_grad=True)
    opt = torch.optim.Adam([tex], lr=5e-2)

    def loss_fn():
        return ((dr.texture(tex, uv_img) - target) ** 2).mean()

    l0 = loss_fn().item()
    for _ in range(60):
        opt.zero_grad()
        loss_fn().backward()
        opt.step()
    assert loss_fn().item() < l0 * 0.05


# ------------------------------- antialias ---------------------------------


def _tri(dx=0.0, dy=0.0):
    pos = torch.tensor([[-0.55 + dx, -0.45 + dy, 0.2, 1.0], [0.62 + dx, -0.38 + dy, 0.2, 1.0],
                        [-0.35 + dx, 0.58 + dy, 0.2, 1.0]])
    return pos, torch.tensor([[0, 1, 2]], dtype=torch.int32)


def _mask(dr, ctx, pos, tri, res, n_samples=0):
    rast, _ = dr.rasterize(ctx, pos, tri, resolution=res)
    m, _ = dr.interpolate(torch.ones(pos.shape[0], 1), rast, tri)
    return dr.antialias(m, rast, pos, tri, n_samples=n_samples)


def test_antialias_blends_boundary_only(dr, ctx):
    print("[torch] antialias boundary", flush=True)
    pos, tri = _tri()
    rast, _ = dr.rasterize(ctx, pos, tri, resolution=[32, 32])
    m, _ = dr.interpolate(torch.ones(3, 1), rast, tri)
    aa = dr.antialias(m, rast, pos, tri)
    tid = rast[0, :, :, 3]
    same = torch.ones_like(tid, dtype=torch.bool)
    for dy in (-1, 0, 1):
        for dx in (-1, 0, 1):
            same &= torch.roll(tid, shifts=(dy, dx), dims=(0, 1)) == tid
    same[0, :] = same[-1, :] = False
    same[:, 0] = same[:, -1] = False
    diff = (aa[0, :, :, 0] - m[0, :, :, 0]).abs()
    assert torch.all(diff[same] < 1e-6)
    assert diff[~same].max() > 1e-3


def test_antialias_color_grad_matches_fd(dr, ctx):
    print("[torch] antialias color fd", flush=True)
    pos, tri = _tri()
    rast, _ = dr.rasterize(ctx, pos, tri, resolution=[16, 16])
    a0 = torch.full((3, 1), 0.8)
    weight = torch.rand(1, 16, 16, 1) - 0.5

    def loss_of(a):
        m, _ = dr.interpolate(a, rast, tri)
        return (dr.antialias(m, rast, pos, tri) * weight).sum()

    a = a0.clone().requires_grad_(True)
    loss_of(a).backward()
    for i in range(3):
        d = torch.zeros_like(a0)
        d[i, 0] = 1e-2
        with torch.no_grad():
            fd = (loss_of(a0 + d) - loss_of(a0 - d)) / 2e-2
        assert a.grad[i, 0].item() == pytest.approx(fd.item(), abs=2e-2, rel=2e-2)


def test_antialias_pos_grad_direction(dr, ctx):
    print("[torch] antialias pos direction", flush=True)
    pos0, tri = _tri()
    with torch.no_grad():
        target = _mask(dr, ctx, _tri(0.08, -0.05)[0], tri, [32, 32])

    def loss_of(p):
        return ((_mask(dr, ctx, p, tri, [32, 32]) - target) ** 2).sum()

    p = pos0.clone().requires_grad_(True)
    loss_of(p).backward()
    an = p.grad[:, :2].reshape(-1)
    assert an.abs().max() > 0
    fd = torch.zeros_like(an)
    for k in range(6):
        d = torch.zeros_like(pos0)
        d[k // 2, k % 2] = 2e-3
        with torch.no_grad():
            fd[k] = (loss_of(pos0 + d) - loss_of(pos0 - d)) / 4e-3
    cos = torch.dot(an, fd) / (an.norm() * fd.norm() + 1e-12)
    assert cos.item() > 0.9, (cos.item(), an, fd)


def test_antialias_silhouette_optimization(dr, ctx):
    print("[torch] antialias optimization", flush=True)
    pos0, tri = _tri()
    with torch.no_grad():
        target = _mask(dr, ctx, _tri(0.15, -0.1)[0], tri, [32, 32])
    offset = torch.zeros(1, 2, requires_grad=True)
    opt = torch.optim.Adam([offset], lr=2e-2)

    def loss_fn():
        p = torch.cat([pos0[:, :2] + offset, pos0[:, 2:]], dim=1)
        return ((_mask(dr, ctx, p, tri, [32, 32], n_samples=8) - target) ** 2).sum()

    l0 = loss_fn().item()
    for _ in range(150):
        opt.zero_grad()
        loss_fn().backward()
        opt.step()
    assert loss_fn().item() < l0 * 0.1
    assert offset[0, 0].item() == pytest.approx(0.15, abs=0.03)
    assert offset[0, 1].item() == pytest.approx(-0.1, abs=0.03)


@pytest.mark.parametrize("n_samples", [0, 8])
def test_antialias_matches_oracle(dr, ctx, oracle, n_samples):
    """Forward = AntiAlias(img, id, clip_vk); backward: AntiAliasBwdImg for
    the colour, AntiAliasBwdVtx (exact, or wide + ColSum with the per-item
    seed iteration * N + i) for the clip, mapped back to GL clip space."""
    print(f"[torch] antialias parity n={n_samples}", flush=True)
    clip_gl, faces = _sphere(seed=3)
    nv = len(clip_gl)
    h, w, n = 40, 36, 2
    rng = np.random.default_rng(13)
    pos_np = np.stack([clip_gl, clip_gl * np.float32(0.95)])
    col_np = rng.random((n, h, w, 3)).astype(np.float32)
    gy = rng.standard_normal((n, h, w, 3)).astype(np.float32)
    tri = torch.from_numpy(faces).cuda()
    pos = torch.from_numpy(pos_np).cuda()
    rast, _ = dr.rasterize(ctx, pos, tri, resolution=[h, w])
    pos_g = pos.clone().requires_grad_(True)
    col = torch.from_numpy(col_np).cuda().requires_grad_(True)
    out = dr.antialias(col, rast, pos_g, tri, n_samples=n_samples)
    key = ("antialias", h, w, len(faces), nv, 3, n, n_samples)
    it = ctx._engines[key].iter_seed + 1 if key in ctx._engines else 1
    out.backward(torch.from_numpy(gy).cuda())
    r = _np(rast)
    ff = faces.astype(np.float32)
    vft = oracle.vertex_faces_tex(ff, nv)
    wo, wc, wp = [], [], []
    for i in range(n):
        clip = _gl_to_vk(pos_np[i])
        tid = r[i, ..., 3]
        wo.append(oracle.antialias(col_np[i], tid, clip, ff))
        wc.append(oracle.antialias_bwd_img(gy[i], tid, clip, ff))
        if n_samples:
            wide = oracle.antialias_bwd_vtx(gy[i], col_np[i], tid, clip, ff, vft,
                                            float(it * n + i), n_samples, True)
            wp.append(oracle.col_sum(wide))
        else:
            wp.append(oracle.antialias_bwd_vtx(gy[i], col_np[i], tid, clip, ff, vft, 0.0, 0,
                                               False))
    _exact(_np(out), np.stack(wo), "antialias")
    _exact(_np(col.grad), np.stack(wc), "antialias colour grad")
    want_p = _grad_vk_to_gl(np.stack(wp)) * np.float32(1.0)
    _exact(_np(pos_g.grad), want_p, "antialias pos grad")
    assert np.abs(want_p).max() > 0


# ------------------------------ rasterize_soft -----------------------------


def _soft_tri(dx=0.0, dy=0.0):
    pos = torch.tensor([[-0.5 + dx, -0.42 + dy, 0.2, 1.0], [0.58 + dx, -0.35 + dy, 0.2, 1.0],
                        [-0.32 + dx, 0.55 + dy, 0.2, 1.0]])
    return pos, torch.tensor([[0, 1, 2]], dtype=torch.int32)


def _soft_mask(dr, ctx, pos, tri, res):
    rs = dr.rasterize_soft(ctx, pos, tri, res, radius_px=3.0)
    return rs[..., 3] * torch.sigmoid(rs[..., 0])


def test_rasterize_soft_channels(dr, ctx):
    print("[torch] soft channels", flush=True)
    pos, tri = _soft_tri()
    rs = dr.rasterize_soft(ctx, pos, tri, [32, 32], radius_px=3.0)
    assert rs.shape == (1, 1, 32, 32, 4)
    dist, fid, cov = rs[0, 0, ..., 0], rs[0, 0, ..., 1], rs[0, 0, ..., 3]
    assert ((cov > 0.5) & (dist > 0.5)).sum() > 20
    assert ((cov > 0.5) & (dist < -0.5)).sum() > 10
    assert (cov < 0.5).sum() > 200
    assert torch.all(fid[cov > 0.5] == 0.0)
    assert torch.count_nonzero(rs[0, 0, 0, -1]) == 0


def test_rasterize_soft_two_layers(dr, ctx):
    print("[torch] soft two layers", flush=True)
    pos = torch.tensor([[-0.7, -0.7, 0.2, 1.0], [0.7, -0.7, 0.2, 1.0], [0.0, 0.7, 0.2, 1.0],
                        [-0.5, -0.5, 0.6, 1.0], [0.5, -0.5, 0.6, 1.0], [0.0, 0.5, 0.6, 1.0]])
    tri = torch.tensor([[0, 1, 2], [3, 4, 5]], dtype=torch.int32)
    rs = dr.rasterize_soft(ctx, pos, tri, [24, 24], radius_px=2.0, peels=2)
    assert rs.shape == (1, 2, 24, 24, 4)
    assert ((rs[0, 0, ..., 3] > 0.5) & (rs[0, 0, ..., 1] == 0.0)).sum() > 10
    assert ((rs[0, 1, ..., 3] > 0.5) & (rs[0, 1, ..., 1] == 1.0)).sum() > 5


def test_rasterize_soft_grad_direction(dr, ctx):
    print("[torch] soft direction", flush=True)
    pos0, tri = _soft_tri()
    with torch.no_grad():
        target = _soft_mask(dr, ctx, _soft_tri(0.06, -0.04)[0], tri, [32, 32])

    def loss_of(p):
        return ((_soft_mask(dr, ctx, p, tri, [32, 32]) - target) ** 2).sum()

    p = pos0.clone().requires_grad_(True)
    loss_of(p).backward()
    an = p.grad[:, :2].reshape(-1)
    assert an.abs().max() > 0
    fd = torch.zeros_like(an)
    for k in range(6):
        d = torch.zeros_like(pos0)
        d[k // 2, k % 2] = 2e-3
        with torch.no_grad():
            fd[k] = (loss_of(pos0 + d) - loss_of(pos0 - d)) / 4e-3
    cos = torch.dot(an, fd) / (an.norm() * fd.norm() + 1e-12)
    assert cos.item() > 0.9, cos.item()


def test_rasterize_soft_silhouette_optimization(dr, ctx):
    print("[torch] soft optimization", flush=True)
    pos0, tri = _soft_tri()
    with torch.no_grad():
        target = _soft_mask(dr, ctx, _soft_tri(0.12, -0.08)[0], tri, [32, 32])
    offset = torch.zeros(1, 2, requires_grad=True)
    opt = torch.optim.Adam([offset], lr=2e-2)

    def loss_fn():
        p = torch.cat([pos0[:, :2] + offset, pos0[:, 2:]], dim=1)
        return ((_soft_mask(dr, ctx, p, tri, [32, 32]) - target) ** 2).sum()

    l0 = loss_fn().item()
    for _ in range(120):
        opt.zero_grad()
        loss_fn().backward()
        opt.step()
    assert loss_fn().item() < l0 * 0.1
    assert offset[0, 0].item() == pytest.approx(0.12, abs=0.03)
    assert offset[0, 1].item() == pytest.approx(-0.08, abs=0.03)


def test_rasterize_soft_matches_oracle(dr, ctx, oracle):
    """Two peels: SoftClip -> RasterizeSoft, then the peel against the first
    layer's shifted depth; backward = ColSum(GatherDistGrad) per peel,
    summed last peel first, mapped to GL clip space and summed over the
    batch for a shared [V, 4] pos."""
    print("[torch] soft parity", flush=True)
    clip_gl, faces = _sphere(seed=4)
    nv, nf = len(clip_gl), len(faces)
    h, w, r = 40, 40, 3.0
    rng = np.random.default_rng(17)
    tri = torch.from_numpy(faces).cuda()
    pos = torch.from_numpy(clip_gl).cuda().requires_grad_(True)
    rs = dr.rasterize_soft(ctx, pos, tri, [h, w], radius_px=r, peels=2)
    gy = rng.standard_normal((1, 2, h, w, 4)).astype(np.float32)
    rs.backward(torch.from_numpy(gy).cuda())
    ff = faces.astype(np.float32)
    vft = oracle.vertex_faces_tex(ff, nv)
    clip = _gl_to_vk(clip_gl)
    sc = oracle.soft_clip(clip, ff, w, h, r)
    fid = np.repeat(np.arange(nf, dtype=np.float32), 3)
    seq = np.arange(3 * nf, dtype=np.float32).reshape(nf, 3)
    rs0 = oracle.rasterize_soft(sc, fid, seq, clip, ff, w, h, r)
    dist, z, cov = rs0[..., 0], rs0[..., 2], rs0[..., 3]
    ge = (dist >= 0).astype(np.float32)
    near = np.clip(z, 0, 1) * np.float32(0.5)
    far = np.clip(dist * np.float32(-1.0 / r), 0, 1) * np.float32(0.5) + np.float32(0.5)
    prev = cov * (ge * near + (np.float32(1.0) - ge) * far)
    rs1 = oracle.rasterize_soft(sc, fid, seq, clip, ff, w, h, r, prev=prev)
    _exact(_np(rs), np.stack([rs0, rs1])[None], "rasterize_soft")
    g1 = oracle.col_sum(oracle.gather_dist_grad(gy[0, 1], rs1, clip, ff, vft, True))
    g0 = oracle.col_sum(oracle.gather_dist_grad(gy[0, 0], rs0, clip, ff, vft, True))
    want = _grad_vk_to_gl((g1 + g0)[None]).sum(0)
    _exact(_np(pos.grad), want, "rasterize_soft grad")
    assert np.abs(want).max() > 0


# ------------------------------ two streams --------------------------------


def _stream_case(dr, ctx, pos, tri, res):
    """rasterize + antialias (colour and position gradients) + rasterize_soft
    of one scene, all on torch's current stream."""
    rast, _ = dr.rasterize(ctx, pos, tri, resolution=res)
    col = torch.ones(1, res[0], res[1], 1, device=pos.device)
    pos_g = pos.clone().requires_grad_(True)
    out = dr.antialias(col, rast, pos_g, tri, n_samples=0)
    out.backward(torch.ones_like(out))
    soft = dr.rasterize_soft(ctx, pos, tri, res, radius_px=3.0)
    return [rast, out.detach(), pos_g.grad, soft]


def test_ops_on_two_streams_match_one_stream(dr, ctx):
    """The per-op entry points share the context's workspace slots (records,
    bins, face ids); calls issued from two torch streams, back to back with
    no host synchronisation, must give the single-stream results (each slot
    orders its next user after its last one, on whichever stream)."""
    print("[torch] two streams", flush=True)
    big = _sphere(level=3, seed=5)
    small = _sphere(level=1, seed=6)
    cases = [(torch.from_numpy(c).cuda(), torch.from_numpy(f).cuda(), r)
             for (c, f), r in ((big, [96, 112]), (small, [40, 36]), (big, [64, 64]))]
    want = [[_np(t) for t in _stream_case(dr, ctx, *c)] for c in cases]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    got = []
    for rep in range(2):
        for i, c in enumerate(cases):
            s = streams[(i + rep) % 2]
            with torch.cuda.stream(s):
                got.append((i, _stream_case(dr, ctx, *c)))
    for s in streams:
        torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for i, outs in got:
        for k, (a, b) in enumerate(zip(outs, want[i])):
            _exact(a.detach().cpu().numpy(), b, f"case {i} output {k}")
