"""The allocation-free RasterizeSoft entry point
(dressi_rasterize_soft_noalloc) against the workspace one
(dressi_rasterize_soft), both called through the C ABI: bit-identical
results on two calls in a row, the second with a smaller input (so stale
scratch contents from the first call must not leak into it), and a clear
error for a problem beyond the fixed scratch size."""
import ctypes as C
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


def _scene(level, s, seed):
    import opendressi_amd as od
    rng = np.random.default_rng(seed)
    pos, faces = od.icosphere(level)
    pos = pos * (1 + 0.1 * rng.standard_normal((len(pos), 1))).astype(np.float32)
    yaw, pitch = rng.uniform(0, 2 * math.pi), rng.uniform(-1.0, 1.0)
    eye = [3.0 * math.cos(pitch) * math.sin(yaw), 3.0 * math.sin(pitch),
           3.0 * math.cos(pitch) * math.cos(yaw)]
    mvp = od.mat4_mul(od.perspective_vk(math.radians(45.0), 1.0, 0.1, 10.0), od.look_at(eye))
    clip = np.concatenate([pos, np.ones((len(pos), 1), np.float32)], 1) @ \
        mvp.reshape(4, 4).astype(np.float32)
    return np.ascontiguousarray(clip, np.float32), faces


def _inputs(ctx, clip, faces, s, r):
    import torch

    from opendressi_amd import ops
    nf = len(faces)
    d_clip = torch.from_numpy(clip).cuda()
    d_faces = torch.from_numpy(faces).cuda()
    soft = ops.soft_clip(ctx, d_clip, d_faces, s, s, r)
    fid = torch.arange(nf, dtype=torch.float32).repeat_interleave(3).cuda()
    fsoft = torch.arange(3 * nf, dtype=torch.float32).reshape(nf, 3).cuda()
    return soft, fid, fsoft, d_clip, d_faces


def _call(ctx, name, args, s, r):
    import torch

    from opendressi_amd._lib import check, lib
    soft, fid, fsoft, clip, faces = args
    out = torch.full((s, s, 4), float("nan"), dtype=torch.float32, device="cuda")
    p = lambda t: C.c_void_p(t.data_ptr())  # noqa: E731
    ctx.use_torch_stream()
    check(getattr(lib, name)(ctx.handle, p(soft), p(fid), p(fsoft), p(clip), clip.shape[0],
                             p(faces), faces.shape[0], s, s, float(r), None, p(out)))
    torch.cuda.synchronize()
    ctx.synchronize()
    return out.cpu().numpy()


def test_noalloc_matches_workspace_entry_point(ctx):
    r = 3.0
    # second call smaller (fewer faces, smaller screen) than the first
    for level, s, seed in ((4, 320, 11), (2, 96, 12)):
        print(f"[noalloc] level={level} screen={s} seed={seed}", flush=True)
        clip, faces = _scene(level, s, seed)
        args = _inputs(ctx, clip, faces, s, r)
        got = _call(ctx, "dressi_rasterize_soft_noalloc", args, s, r)
        want = _call(ctx, "dressi_rasterize_soft", args, s, r)
        assert (want[..., 3] > 0).sum() > 100  # the scene is on screen
        assert np.array_equal(got, want), f"level {level} screen {s}: results differ"


def test_noalloc_rejects_oversized_problem(ctx):
    from opendressi_amd._lib import DressiError
    clip, faces = _scene(1, 32, 13)
    args = _inputs(ctx, clip, faces, 32, 3.0)
    # a 4096 x 4096 screen needs 65536 tiles x 4100 B of bins: above 32 MiB;
    # the size check runs before any launch
    with pytest.raises(DressiError, match="scratch"):
        _call_no_out(ctx, args, 4096)


def _call_no_out(ctx, args, s):
    import torch

    from opendressi_amd._lib import check, lib
    soft, fid, fsoft, clip, faces = args
    out = torch.empty((s, s, 4), dtype=torch.float32, device="cuda")  # full size all the same
    p = lambda t: C.c_void_p(t.data_ptr())  # noqa: E731
    check(lib.dressi_rasterize_soft_noalloc(ctx.handle, p(soft), p(fid), p(fsoft), p(clip),
                                            clip.shape[0], p(faces), faces.shape[0], s, s, 3.0,
                                            None, p(out)))


def test_noalloc_orders_calls_on_two_streams(ctx):
    """Two calls on two streams (two contexts) with no host synchronisation
    between them: the second waits for the first's use of the shared
    scratch, so both match the workspace entry point."""
    import torch

    import opendressi_amd as od
    from opendressi_amd._lib import check, lib
    r = 3.0
    ctx2 = od.Context(0)  # its own stream
    try:
        cases = [(4, 320, 21), (3, 192, 22)]
        args = []
        for level, s, seed in cases:
            clip, faces = _scene(level, s, seed)
            args.append(_inputs(ctx, clip, faces, s, r))
        torch.cuda.synchronize()
        outs = []
        p = lambda t: C.c_void_p(t.data_ptr())  # noqa: E731
        ctx.use_torch_stream()
        for c, (level, s, _), a in zip((ctx, ctx2), cases, args):
            print(f"[noalloc 2 streams] level={level} screen={s}", flush=True)
            soft, fid, fsoft, clip, faces = a
            out = torch.full((s, s, 4), float("nan"), dtype=torch.float32, device="cuda")
            check(lib.dressi_rasterize_soft_noalloc(
                c.handle, p(soft), p(fid), p(fsoft), p(clip), clip.shape[0], p(faces),
                faces.shape[0], s, s, r, None, p(out)))
            outs.append(out)
        ctx2.synchronize()
        ctx.synchronize()
        torch.cuda.synchronize()
        for (level, s, _), a, out in zip(cases, args, outs):
            want = _call(ctx, "dressi_rasterize_soft", a, s, r)
            assert np.array_equal(out.cpu().numpy(), want), f"level {level} screen {s}"
    finally:
        ctx2.close()
