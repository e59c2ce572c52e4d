"""Pins the oracle's GatherDistGrad (oracle/dressi_oracle.c
or_gather_dist_grad, src/core/f_ops.cpp:1248-1358) before it is trusted as
the checker of the HIP path:

* bit-exact against the reference's own CPU evaluator through the committed
  fixture tests/golden/ds_unit.npz (RasterizeSoft's backward w.r.t. the hard
  clips on three cameras: the wide partials and their ColSum);
* against what the mathematics fixes: with every pixel's face held fixed, the
  gradient is the derivative of sum_p gy_p dist_p(clip) -- central finite
  differences in float64 of the signed distance to the projected triangle
  (tests/test_softras.cpp:180-216 checks the same way); the {V,1} form equals
  ColSum of the wide form up to summation order.
"""
import numpy as np


def _exact(a, b, what=""):
    assert a.shape == b.shape, (what, a.shape, b.shape)
    if not np.array_equal(a, b):
        d = np.abs(a.astype(np.float64) - b)
        raise AssertionError(f"{what}: not bit-exact, max diff {d.max():.3g}, "
                             f"{int((d > 0).sum())} differ")


def test_gather_dist_grad_matches_reference_fixture(oracle, golden):
    g = golden("ds_unit.npz")
    for i in range(3):
        wide = oracle.gather_dist_grad(g[f"in_gy{i}"], g[f"in_rs{i}"], g[f"in_clip{i}"],
                                       g["in_faces"], g["in_vf"], wide=True)
        _exact(wide, g[f"out_wide{i}"], f"wide {i}")
        _exact(oracle.col_sum(wide), g[f"out_g{i}"], f"colsum {i}")
        flat = oracle.gather_dist_grad(g[f"in_gy{i}"], g[f"in_rs{i}"], g[f"in_clip{i}"],
                                       g["in_faces"], g["in_vf"], wide=False)
        np.testing.assert_allclose(flat, g[f"out_g{i}"], rtol=1e-5, atol=1e-4)


def _dist64(p, s):
    """SignedDistToTri in float64 (cpu_raster.cpp:114-151)."""
    best, npos, nneg = None, 0, 0
    for k in range(3):
        a, b = s[k], s[(k + 1) % 3]
        e = b - a
        l2 = e @ e
        t = min(max(((p - a) @ e) / l2, 0.0), 1.0) if l2 > 1e-12 else 0.0
        d2 = float(((p - (a + t * e)) ** 2).sum())
        best = d2 if best is None or d2 < best else best
        cr = e[0] * (p[1] - a[1]) - e[1] * (p[0] - a[0])
        npos += cr >= 0
        nneg += cr <= 0
    return (1.0 if (npos == 3 or nneg == 3) else -1.0) * np.sqrt(best)


def test_gather_dist_grad_matches_finite_differences(oracle, golden):
    g = golden("ds_unit.npz")
    s = int(g["in_cfg"][0])
    clip, rs, gy, faces = g["in_clip0"], g["in_rs0"], g["in_gy0"], g["in_faces"]
    flat = oracle.gather_dist_grad(gy, rs, clip, faces, g["in_vf"], wide=False)
    cov = rs[..., 3] > 0.5
    ys, xs = np.nonzero(cov & (gy[..., 0] != 0))
    fidx = (rs[ys, xs, 1] + 0.5).astype(np.int64)

    def total(c):
        c = c.astype(np.float64)
        acc = 0.0
        for y, x, f in zip(ys, xs, fidx):
            sc = np.array([[(c[v, 0] / c[v, 3] * 0.5 + 0.5) * s,
                            (c[v, 1] / c[v, 3] * 0.5 + 0.5) * s] for v in faces[f].astype(int)])
            acc += gy[y, x, 0] * _dist64(np.array([x + 0.5, y + 0.5]), sc)
        return acc

    rng = np.random.default_rng(0)
    verts = rng.choice(np.unique(faces[fidx].astype(int)), 6, replace=False)
    h = 1e-4
    for v in verts:
        for comp in (0, 1, 3):
            cp, cm = clip.copy(), clip.copy()
            cp[v, comp] += h
            cm[v, comp] -= h
            fd = (total(cp) - total(cm)) / (2 * h)
            assert abs(fd - flat[v, comp]) <= 2e-2 * max(1.0, abs(fd)), (v, comp, fd, flat[v, comp])
        assert flat[v, 2] == 0.0
