"""The F:: op catalogue through DressiAD's generic executor on the GPU.

tests/graph_ops.cpp builds one small graph per op family (textures, the
equirect lookup, the IBL convolutions, pooling, the BRDF LUT, matrices,
math and vector ops, reductions, in-graph fetches, the regularisers), runs
one execStep with RSP packing (fused elementwise stages) and with Naive
packing (one kernel per function), and returns every output and the
gradient of every requires-grad leaf under an upstream image g (the loss is
sum(y * g)).

Checks: RSP and Naive give the same floats; the texture, pooling and
convolution ops and their backwards equal the oracle's per-op functions bit
for bit (they are the per-op entry points the C ABI tests pin); the equirect
lookup, its VJP and PrefilterEnv within 1e-5 of their scale and the LUT
within 1e-6 (the per-op bars of tests/test_gpu_pbr.py); matrices,
reductions, fetches and the regularisers equal a float32 restatement of the
reference's CPU kernels (same operation order) bit for bit; the
transcendental ops within 2e-6 relative of numpy's float32 results and their
gradients within 1e-4 of a float64 PyTorch autograd reference.
"""
import os
import struct
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "_bin", "graph_ops")
F32 = np.float32


def _write(path, imgs):
    with open(path, "wb") as f:
        f.write(struct.pack("<I", len(imgs)))
        for name, a in imgs.items():
            a = np.ascontiguousarray(a, F32)
            if a.ndim == 1:
                a = a.reshape(1, -1, 1)
            elif a.ndim == 2:
                a = a.reshape(1, a.shape[0], a.shape[1])
            h, w, c = a.shape
            f.write(struct.pack("<I", len(name)) + name.encode())
            f.write(struct.pack("<III", w, h, c))
            f.write(a.tobytes())


def _read(path):
    out = {}
    with open(path, "rb") as f:
        (n,) = struct.unpack("<I", f.read(4))
        for _ in range(n):
            (ln,) = struct.unpack("<I", f.read(4))
            name = f.read(ln).decode()
            w, h, c = struct.unpack("<III", f.read(12))
            out[name] = np.frombuffer(f.read(w * h * c * 4), F32).reshape(h, w, c)
    return out


def _run(tmp_path, case, imgs):
    """{output: array} from the RSP run, after checking the Naive run
    matches it bit for bit."""
    if not os.path.exists(EXE):
        pytest.fail("tests/_bin/graph_ops is not built (run __graft_entry__.build())")
    inp = tmp_path / f"{case}_in.bin"
    _write(inp, imgs)
    res = {}
    for packing in ("rsp", "naive"):
        out = tmp_path / f"{case}_{packing}.bin"
        r = subprocess.run([EXE, case, packing, str(inp), str(out)], capture_output=True,
                           text=True, timeout=120)
        print(r.stdout.strip(), r.stderr.strip(), flush=True)
        assert r.returncode == 0, r.stderr
        res[packing] = _read(out)
    assert res["rsp"].keys() == res["naive"].keys()
    for k in res["rsp"]:
        assert np.array_equal(res["rsp"][k], res["naive"][k]), f"{case}/{k}: RSP != Naive"
    return res["rsp"]


def _exact(a, b, what):
    a = np.asarray(a, F32).reshape(np.shape(b))
    if not np.array_equal(a, b):
        d = np.abs(a.astype(np.float64) - b)
        raise AssertionError(f"{what}: {int((d > 0).sum())} differ, max {d.max():.3g}")


def _close(a, b, tol, what):
    a = np.asarray(a, np.float64).reshape(np.shape(b))
    d = np.abs(a - b).max()
    m = float(np.abs(b).max())
    assert d <= tol * max(m, 1e-30), f"{what}: max diff {d:.3g} vs max {m:.3g} (tol {tol})"


def test_texture_ops(tmp_path, oracle):
    rng = np.random.default_rng(11)
    th, tw, sh, sw = 37, 53, 61, 47
    tex = rng.random((th, tw, 4)).astype(F32)
    tex2 = rng.random((th, tw, 3)).astype(F32)
    uv = rng.random((sh, sw, 2)).astype(F32)
    iv = np.zeros((th, tw, 4), F32)
    iv[..., 0] = rng.random((th, tw)) * 51 - 2
    iv[..., 1] = rng.random((th, tw)) * 65 - 2
    iv[..., 2] = (rng.random((th, tw)) < 0.5)
    g = rng.standard_normal((sh, sw, 4)).astype(F32)
    g2 = rng.standard_normal((sh, sw, 3)).astype(F32)
    r = _run(tmp_path, "texture", dict(tex=tex, tex2=tex2, uv=uv, inv_uv=iv, g=g, g2=g2))
    _exact(r["bilinear"], oracle.texture_bilinear(tex, uv), "TextureBilinear")
    _exact(r["dtex"], oracle.gather_inv_uv_bilinear(g, iv, uv), "GatherByInverseUVBilinear")
    _exact(r["nearest"], oracle.texture_nearest(tex2, uv), "Texture")
    _exact(r["dtex2"], oracle.gather_inv_uv(g2, iv, uv), "GatherByInverseUV")


def test_equirect_sample(tmp_path, oracle):
    rng = np.random.default_rng(12)
    m = (1.0 + rng.random((32, 64, 3))).astype(F32)
    d = rng.standard_normal((24, 40, 3)).astype(F32)
    g = rng.standard_normal((24, 40, 3)).astype(F32)
    r = _run(tmp_path, "equirect", dict(map=m, dir=d, g=g))
    _close(r["y"], oracle.equirect_sample(m, d), 1e-5, "EquirectSample")
    _close(r["dmap"], oracle.equirect_sample(np.zeros_like(m), d, g), 1e-5, "EquirectSampleBwd")


def test_ibl_convolutions_pool_lut(tmp_path, oracle):
    rng = np.random.default_rng(13)
    env = (0.5 + rng.random((32, 64, 3))).astype(F32)
    ow, oh, rough, n_env, lw, lh, n_lut = 32, 16, 0.5, 64, 32, 32, 128
    g_irr = rng.standard_normal((oh, ow, 3)).astype(F32)
    g_pref = rng.standard_normal((oh, ow, 3)).astype(F32)
    g_pool = rng.standard_normal((16, 32, 3)).astype(F32)
    params = np.array([ow, oh, rough, n_env, lw, lh, n_lut], F32)
    r = _run(tmp_path, "conv", dict(env=env, env1=env, env2=env, env3=env, g_irr=g_irr,
                                    g_pref=g_pref, g_pool=g_pool, params=params))
    _exact(r["irr"], oracle.irradiance_conv(env, ow, oh), "IrradianceConv")
    _exact(r["denv1"], oracle.irradiance_conv(env, ow, oh, g_irr), "IrradianceConvBwd")
    _exact(r["pref"], oracle.prefilter_conv(env, ow, oh, rough), "PrefilterConv")
    _exact(r["denv2"], oracle.prefilter_conv(env, ow, oh, rough, g_pref), "PrefilterConvBwd")
    _exact(r["pool"], oracle.avg_pool2x2(env), "AvgPool2x2")
    _exact(r["denv3"], oracle.avg_pool2x2(env, g_pool), "AvgPool2x2 backward")
    _close(r["prefenv"], oracle.prefilter_env(env, ow, oh, rough, n_env), 1e-5, "PrefilterEnv")
    _close(r["lut"], oracle.brdf_lut(lw, lh, n_lut), 1e-6, "BrdfIntegrationLut")


# ---- float32 restatements of the reference's CPU kernels (column-major) -------

def _mm(a, b):
    """MAT4 x MAT4 per pixel: out[c*4+r] = sum_k a[k*4+r] * b[c*4+k], k in order."""
    out = np.zeros_like(a)
    for c in range(4):
        for rr in range(4):
            acc = np.zeros(a.shape[:-1], F32)
            for k in range(4):
                acc = (acc + a[..., k * 4 + rr] * b[..., c * 4 + k]).astype(F32)
            out[..., c * 4 + rr] = acc
    return out


def _mv(a, v):
    out = np.zeros(v.shape, F32)
    for rr in range(4):
        acc = np.zeros(v.shape[:-1], F32)
        for c in range(4):
            acc = (acc + a[..., c * 4 + rr] * v[..., c]).astype(F32)
        out[..., rr] = acc
    return out


def _tr(a):
    out = np.zeros_like(a)
    for c in range(4):
        for rr in range(4):
            out[..., c * 4 + rr] = a[..., rr * 4 + c]
    return out


def _outer(u, w):
    out = np.zeros(u.shape[:-1] + (16,), F32)
    for c in range(4):
        for rr in range(4):
            out[..., c * 4 + rr] = u[..., rr] * w[..., c]
    return out


def test_matrix_ops(tmp_path):
    rng = np.random.default_rng(14)
    n = 37
    a, b, a2, a3 = (rng.standard_normal((1, n, 16)).astype(F32) for _ in range(4))
    v, v2 = (rng.standard_normal((1, n, 4)).astype(F32) for _ in range(2))
    g_ab, g_at, g_a3x2, g_vv = (rng.standard_normal((1, n, 16)).astype(F32) for _ in range(4))
    g_av = rng.standard_normal((1, n, 4)).astype(F32)
    r = _run(tmp_path, "matrix", dict(a=a, b=b, v=v, a2=a2, a3=a3, v2=v2, g_ab=g_ab, g_av=g_av,
                                      g_at=g_at, g_a3x2=g_a3x2, g_vv=g_vv))
    _exact(r["ab"], _mm(a, b), "MatMul")
    _exact(r["av"], _mv(a2, v), "MatMul vector")
    _exact(r["at"], _tr(a3), "Transpose")
    _exact(r["a3x2"], a3 * F32(2), "matrix * 2")
    _exact(r["vv"], _outer(v2, v2), "OuterProduct")
    _exact(r["da"], _mm(g_ab, _tr(b)), "MatMul backward (left)")
    _exact(r["db"], _mm(_tr(a), g_ab), "MatMul backward (right)")
    _exact(r["da2"], _outer(g_av, v), "MatMul vector backward (matrix)")
    _exact(r["dv"], _mv(_tr(a2), g_av), "MatMul vector backward (vector)")
    _exact(r["da3"], _tr(g_at) + g_a3x2 * F32(2), "two matrix contributions")
    _exact(r["dv2"], _mv(g_vv, v2) + _mv(_tr(g_vv), v2), "OuterProduct backward")


def _reduce_tree(x):
    """Sum(x): Reduce2x2Sum until {1,1}, each output summing its 2x2 block
    in row order from 0 (x {h, w, c})."""
    while x.shape[0] > 1 or x.shape[1] > 1:
        h, w = x.shape[:2]
        y = np.zeros(((h + 1) // 2, (w + 1) // 2, x.shape[2]), F32)
        for oy in range(y.shape[0]):
            for ox in range(y.shape[1]):
                acc = np.zeros(x.shape[2], F32)
                for dy in range(2):
                    for dx in range(2):
                        sy, sx = 2 * oy + dy, 2 * ox + dx
                        if sy < h and sx < w:
                            acc = (acc + x[sy, sx]).astype(F32)
                y[oy, ox] = acc
        x = y
    return x[0, 0]


def _sum_all(x):
    """SumAll: above 256 pixels 64 strided double partials, each rounded to
    float, then their double sum rounded once."""
    flat = x.reshape(-1, x.shape[-1]).astype(np.float64)
    parts = []
    for t in range(64):
        s = 0.0
        for i in range(t, flat.shape[0], 64):
            for c in range(flat.shape[1]):
                s += flat[i, c]
        parts.append(np.float64(F32(s)))
    return F32(sum(parts))


def test_math_vector_and_reduction_ops(tmp_path):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(15)
    n = 300  # > 256: SumAll takes its 64-partial path
    x = rng.uniform(-0.9, 0.9, (1, n, 1)).astype(F32)
    y = rng.uniform(0.2, 1.5, (1, n, 1)).astype(F32)
    z = rng.uniform(-3, 3, (1, n, 1)).astype(F32)
    p = rng.standard_normal((1, n, 3)).astype(F32)
    q = rng.standard_normal((1, n, 3)).astype(F32)
    g = rng.standard_normal((1, n, 1)).astype(F32)
    g3 = rng.standard_normal((1, n, 3)).astype(F32)
    r = _run(tmp_path, "math", dict(x=x, y=y, z=z, p=p, q=q, g=g, g3=g3))
    with np.errstate(all="ignore"):
        ref = {
            "sin": np.sin(x), "cos": np.cos(x), "tan": np.tan(x), "asin": np.arcsin(x),
            "acos": np.arccos(x), "atan": np.arctan(x), "atan2": np.arctan2(x, y),
            "exp": np.exp(x), "exp2": np.exp2(x), "log": np.log(y), "log2": np.log2(y),
            "sqrt": np.sqrt(y), "rsqrt": F32(1) / np.sqrt(y), "pow": np.power(y, x),
            "sigmoid": F32(1) / (F32(1) + np.exp(-z)),
        }
    for k, want in ref.items():
        np.testing.assert_allclose(r[k], want, rtol=2e-6, atol=1e-7, err_msg=k)
    exact = {
        "abs": np.abs(z), "sign": np.sign(z), "floor": np.floor(z), "fract": z - np.floor(z),
        "mod": (z - y * np.floor(z / y)).astype(F32), "max": np.maximum(x, y),
        "min": np.minimum(x, y), "clamp": np.clip(z, F32(-0.5), F32(0.5)),
        "mix": (x + (y - x) * F32(0.25)).astype(F32), "step": (y >= x).astype(F32),
        "less": (x < y).astype(F32), "gequal": (x >= y).astype(F32),
    }
    for k, want in exact.items():
        _exact(r[k], want, k)
    s = np.clip((x - F32(0.2)) / (F32(0.8) - F32(0.2)), 0, 1).astype(F32)
    _exact(r["smooth"], (s * s * (F32(3) - F32(2) * s)).astype(F32), "SmoothStep")
    # vector ops: sequential component sums
    dot = ((p[..., 0] * q[..., 0] + p[..., 1] * q[..., 1]).astype(F32) + p[..., 2] * q[..., 2])
    _exact(r["dot"], dot[..., None], "Dot")
    cross = np.stack([p[..., 1] * q[..., 2] - p[..., 2] * q[..., 1],
                      p[..., 2] * q[..., 0] - p[..., 0] * q[..., 2],
                      p[..., 0] * q[..., 1] - p[..., 1] * q[..., 0]], -1)
    _exact(r["cross"], cross, "Cross")
    ss = ((p[..., 0] * p[..., 0] + p[..., 1] * p[..., 1]).astype(F32) + p[..., 2] * p[..., 2])
    _exact(r["length"], np.sqrt(ss)[..., None], "Length")
    _exact(r["compsum"], ((p[..., 0] + p[..., 1]).astype(F32) + p[..., 2])[..., None], "CompSum")
    np.testing.assert_allclose(r["normalize"], p / np.linalg.norm(p, axis=-1, keepdims=True),
                               rtol=2e-6, atol=1e-7)
    # reductions
    _exact(r["sum"].reshape(-1), _reduce_tree(x.reshape(1, n, 1)), "Sum")
    sp = _reduce_tree(p.reshape(1, n, 3))
    mean = F32((sp[0] + sp[1]).astype(F32) + sp[2]) * (F32(1) / F32(n * 3))
    _exact(r["mean"].reshape(-1), np.array([mean], F32), "Mean")
    _exact(r["sumall"].reshape(-1), np.array([_sum_all(p)], F32), "SumAll")
    # gradients against float64 autograd
    t = {k: torch.tensor(v.astype(np.float64), requires_grad=k in "xypq")
         for k, v in dict(x=x, y=y, p=p, q=q).items()}
    tg, tg3 = torch.tensor(g.astype(np.float64)), torch.tensor(g3.astype(np.float64))
    X, Y, P, Q = t["x"], t["y"], t["p"], t["q"]
    nq = Q / Q.norm(dim=-1, keepdim=True)
    terms = [torch.sin(X), torch.cos(X), torch.tan(X), torch.asin(X), torch.acos(X),
             torch.atan(X), torch.atan2(X, Y), torch.exp(X), torch.exp2(X), torch.log(Y),
             torch.log2(Y), torch.sqrt(Y), torch.rsqrt(Y), torch.pow(Y, X), torch.maximum(X, Y),
             torch.minimum(X, Y), X + (Y - X) * 0.25, (P * Q).sum(-1, keepdim=True),
             P.norm(dim=-1, keepdim=True), (P - Q).norm(dim=-1, keepdim=True),
             P.sum(-1, keepdim=True)]
    loss = sum((u * tg).sum() for u in terms)
    loss = loss + (torch.cross(P, Q, dim=-1) * tg3).sum() \
        + ((P / P.norm(dim=-1, keepdim=True)) * tg3).sum() \
        + ((P - 2 * (nq * P).sum(-1, keepdim=True) * nq) * tg3).sum()
    loss.backward()
    for k in "xypq":
        _close(r["d" + k], t[k].grad.numpy(), 1e-4, f"d{k}")


def test_fetch_ops(tmp_path):
    rng = np.random.default_rng(16)
    tex = rng.random((8, 5, 4)).astype(F32)       # {w 5, h 8} VEC4
    atlas = rng.random((12, 6, 1)).astype(F32)    # three 6 x 4 tiles
    row = np.array([[[1.6]]], F32)                # rounds to 2
    r = _run(tmp_path, "fetch", dict(tex=tex, atlas=atlas, row=row,
                                     params=np.array([3, 4], F32)))
    _exact(r["pixel"].reshape(-1), tex[2, 3], "PixelFetch")
    _exact(r["tile"], atlas[8:12], "TileFetch")


def test_regulariser_ops(tmp_path, oracle):
    """VertexNeighborMean and the normal-consistency chain on an icosphere
    (f_ops.cpp:1983-2181), against their float32 restatement."""
    pos, faces = oracle.icosphere(1)
    rng = np.random.default_rng(17)
    pos = (pos * (1 + 0.1 * rng.standard_normal((len(pos), 1)))).astype(F32)
    nv, nf = len(pos), len(faces)
    fi = faces.astype(np.int64)
    nb = [sorted({int(fi[f, (k + j) % 3]) for f in range(nf) for k in range(3)
                  if fi[f, k] == v for j in (1, 2)}) for v in range(nv)]
    deg = max(len(x) for x in nb)
    nbrs = -np.ones((deg, nv), F32)
    for v, lst in enumerate(nb):
        nbrs[:len(lst), v] = lst
    vf = oracle.vertex_faces_tex(faces, nv)
    edges = {}
    for f in range(nf):
        for k in range(3):
            e = tuple(sorted((int(fi[f, k]), int(fi[f, (k + 1) % 3]))))
            edges.setdefault(e, []).append(f)
    fadj = -np.ones((nf, 3), F32)
    used = np.zeros(nf, int)
    for e in sorted(edges):
        fs = edges[e]
        for i in range(len(fs)):
            for j in range(i + 1, len(fs)):
                for a, b in ((fs[i], fs[j]), (fs[j], fs[i])):
                    if used[a] < 3:
                        fadj[a, used[a]] = b
                        used[a] += 1
    r = _run(tmp_path, "regular", dict(pos=pos.reshape(1, nv, 3), nbrs=nbrs[..., None],
                                       faces=faces.reshape(1, nf, 3), fadj=fadj.reshape(1, nf, 3),
                                       vf=vf[..., None]))
    mean = np.zeros((nv, 3), F32)
    for v, lst in enumerate(nb):
        acc = np.zeros(3, F32)
        for u in lst:
            acc = (acc + pos[u]).astype(F32)
        mean[v] = acc / F32(len(lst))
    _exact(r["mean"], mean.reshape(1, nv, 3), "VertexNeighborMean")

    def cross(a, b):
        return np.array([a[1] * b[2] - a[2] * b[1], a[2] * b[0] - a[0] * b[2],
                         a[0] * b[1] - a[1] * b[0]], F32)

    def face_cross(f):
        p0, p1, p2 = pos[fi[f, 0]], pos[fi[f, 1]], pos[fi[f, 2]]
        return cross((p1 - p0).astype(F32), (p2 - p0).astype(F32))

    def length(c):
        return F32(np.sqrt(F32(F32(c[0] * c[0] + c[1] * c[1]) + c[2] * c[2])))

    term = np.zeros((nf, 3), F32)
    for f in range(nf):
        ca = face_cross(f)
        la = length(ca)
        gsum = np.zeros(3, F32)
        if not la < F32(1e-12):
            na = (ca / la).astype(F32)
            for j in range(3):
                gv = fadj[f, j]
                if gv < -0.5:
                    continue
                cb = face_cross(int(gv))
                lb = length(cb)
                if lb < F32(1e-12):
                    continue
                nbv = (cb / lb).astype(F32)
                d = F32(F32(na[0] * nbv[0] + na[1] * nbv[1]) + na[2] * nbv[2])
                gsum = (gsum + (-(nbv - d * na) / la).astype(F32)).astype(F32)
        term[f] = gsum
    _exact(r["term"], term.reshape(1, nf, 3), "NormalConsistencyFaceTerm")
    grad = np.zeros((nv, 3), F32)
    for v in range(nv):
        acc = np.zeros(3, F32)
        for d in range(vf.shape[0]):
            f = vf[d, v]
            if f < -0.5:
                continue
            f = int(f)
            p0, p1, p2 = pos[fi[f, 0]], pos[fi[f, 1]], pos[fi[f, 2]]
            e1, e2 = (p1 - p0).astype(F32), (p2 - p0).astype(F32)
            g1, g2 = cross(e2, term[f]), cross(term[f], e1)
            for c in range(3):
                if fi[f, 1] == v:
                    acc[c] = F32(acc[c] + g1[c])
                if fi[f, 2] == v:
                    acc[c] = F32(acc[c] + g2[c])
                if fi[f, 0] == v:
                    acc[c] = F32(acc[c] - F32(g1[c] + g2[c]))
        grad[v] = acc
    _exact(r["grad"], grad.reshape(1, nv, 3), "NormalConsistencyVertexGrad")


@pytest.mark.gpu
def test_loss_reset_replaces_the_optimizer_updates(tmp_path):
    """setLossVar after a step re-runs the optimizer for the new graph; the
    update pairs it registered for the old graph are dropped: the same
    DressiAD then matches a fresh one built on the new loss (state and
    function count)."""
    rng = np.random.default_rng(12)
    imgs = {"x": rng.standard_normal((3, 5, 3)).astype(F32),
            "tgt": rng.standard_normal((3, 5, 3)).astype(F32)}
    for packing in ("rsp", "naive"):
        inp = tmp_path / "rebuild_in.bin"
        out = tmp_path / f"rebuild_{packing}.bin"
        _write(inp, imgs)
        r = subprocess.run([EXE, "rebuild", packing, str(inp), str(out)], capture_output=True,
                           text=True, timeout=120)
        print(r.stdout.strip(), r.stderr.strip(), flush=True)
        assert r.returncode == 0, r.stderr
        o = _read(out)
        assert np.array_equal(o["xa"], o["xb"]) and np.array_equal(o["ma"], o["mb"])
        assert not np.array_equal(o["xa"], imgs["x"])
        fa, fb = (int(t.split("=")[1]) for t in r.stdout.split()[2:4])
        assert fa == fb, r.stdout
