"""ctypes front-end of the CPU oracle (liboracle.so) and of the reference's own
CPU build (oracle/_ref/libdressi_ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() (as the
checker) and bench.py's cpu_baseline leg. The product package never imports
this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libdressi_ref.so")
REF_ROOT = "/root/reference"

_F = C.POINTER(C.c_float)
_U32 = C.c_uint32


def build(ref: bool = False) -> None:
    """Compile liboracle.so (and, when asked and the reference checkout is
    present, the reference harness)."""
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)
    if ref and os.path.isdir(REF_ROOT):
        subprocess.run(["make", "-s", "-C", HERE, "ref", f"REF={REF_ROOT}"], check=True)


def _fp(a):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_F)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class _Lib:
    prefix = ""

    def __init__(self, path: str):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.lib = C.CDLL(path)

    def fn(self, name):
        return getattr(self.lib, self.prefix + name)

    # ---- ops shared by both libraries (same argument lists) ---------------
    def soft_clip(self, clip, faces, w, h, radius):
        clip, faces = _f32(clip), _f32(faces)
        nv, nf = clip.shape[0], faces.shape[0]
        out = np.zeros((3 * nf, 4), np.float32)
        self._call("soft_clip", _fp(clip), _U32(nv), _fp(faces), _U32(nf), _U32(w), _U32(h),
                   C.c_float(radius), _fp(out))
        return out

    def rasterize(self, clip, attr, faces, w, h):
        clip, attr, faces = _f32(clip), _f32(attr), _f32(faces)
        if attr.ndim == 1:
            attr = attr[:, None]
        nc = attr.shape[1]
        out = np.zeros((h, w, nc), np.float32)
        self._call("rasterize", _fp(clip), _U32(clip.shape[0]), _fp(attr), _U32(nc), _fp(faces),
                   _U32(faces.shape[0]), _U32(w), _U32(h), _fp(out))
        return out

    def rasterize_face_id(self, clip, faces, w, h):
        clip, faces = _f32(clip), _f32(faces)
        out = np.zeros((h, w), np.float32)
        self._call("rasterize_face_id", _fp(clip), _U32(clip.shape[0]), _fp(faces),
                   _U32(faces.shape[0]), _U32(w), _U32(h), _fp(out))
        return out

    def face_fetch(self, attr, idx):
        attr, idx = _f32(attr), _f32(idx)
        nc = attr.shape[1]
        h, w = idx.shape
        out = np.zeros((h, w, nc), np.float32)
        self._call("face_fetch", _fp(attr), _U32(nc), _U32(attr.shape[0]), _fp(idx), _U32(w),
                   _U32(h), _fp(out))
        return out

    def face_fetch_bwd(self, gy, idx, prj0, prj1, prj2, seed, radius, n_samples):
        gy, idx = _f32(gy), _f32(idx)
        prj0, prj1, prj2 = _f32(prj0), _f32(prj1), _f32(prj2)
        h, w = idx.shape
        nc = gy.shape[-1]
        nf = prj0.shape[0]
        out = np.zeros((nf, nc), np.float32)
        self._call("face_fetch_bwd", _fp(gy), _U32(nc), _fp(idx), _U32(w), _U32(h), _fp(prj0),
                   _fp(prj1), _fp(prj2), _U32(nf), C.c_float(seed), C.c_float(radius),
                   _U32(n_samples), _fp(out))
        return out

    def lookup_faces_bwd(self, gy, faces, vtx_faces, corner):
        gy, faces, vtx_faces = _f32(gy), _f32(faces), _f32(vtx_faces)
        nc = gy.shape[1]
        deg, nv = vtx_faces.shape
        out = np.zeros((nv, nc), np.float32)
        self._call("lookup_faces_bwd", _fp(gy), _U32(nc), _fp(faces), _U32(faces.shape[0]),
                   _fp(vtx_faces), _U32(nv), _U32(deg), _U32(corner), _fp(out))
        return out

    def hsr_fit(self, pos0, faces, tgt_pos, tgt_faces, mvps, screen, radius=3.0, samples=8,
                lr=1e-3, iters=1, want_images=True):
        pos0, faces = _f32(pos0), _f32(faces)
        tgt_pos, tgt_faces, mvps = _f32(tgt_pos), _f32(tgt_faces), _f32(mvps)
        nv, nf = pos0.shape[0], faces.shape[0]
        n = mvps.shape[0]
        s = screen
        r = dict(pos=np.zeros((nv, 3), np.float32), m=np.zeros((nv, 3), np.float32),
                 v=np.zeros((nv, 3), np.float32), t=np.zeros(1, np.float32),
                 loss=np.zeros(max(iters, 1), np.float32), grad0=np.zeros((nv, 3), np.float32))
        if want_images:
            r.update(pred0=np.zeros((n, s, s), np.float32), target=np.zeros((n, s, s), np.float32),
                     rs0=np.zeros((n, s, s, 4), np.float32), lossimg0=np.zeros((s, s), np.float32))
        g = r.get
        self._call("hsr_fit", _fp(pos0), _U32(nv), _fp(faces), _U32(nf), _fp(tgt_pos),
                   _U32(tgt_pos.shape[0]), _fp(tgt_faces), _U32(tgt_faces.shape[0]), _fp(mvps),
                   _U32(n), _U32(s), C.c_float(radius), _U32(samples), C.c_float(lr),
                   _U32(iters), _fp(r["pos"]), _fp(r["m"]), _fp(r["v"]), _fp(r["t"]),
                   _fp(r["loss"]), _fp(r["grad0"]), _fp(g("pred0")), _fp(g("target")),
                   _fp(g("rs0")), _fp(g("lossimg0")))
        return r


    def aa_fit(self, pos0, faces, tgt_pos, tgt_faces, mvps, screen, samples=8, lr=1e-3,
               iters=1, want_images=True):
        """The AA silhouette fit (technique aa): dict pos, m, v, t, loss, grad0
        and, with want_images, pred0 / target / tri0 {N,S,S}, lossimg0 {S,S}."""
        pos0, faces = _f32(pos0), _f32(faces)
        tgt_pos, tgt_faces, mvps = _f32(tgt_pos), _f32(tgt_faces), _f32(mvps)
        nv, nf = pos0.shape[0], faces.shape[0]
        n = mvps.shape[0]
        s = screen
        r = dict(pos=np.zeros((nv, 3), np.float32), m=np.zeros((nv, 3), np.float32),
                 v=np.zeros((nv, 3), np.float32), t=np.zeros(1, np.float32),
                 loss=np.zeros(max(iters, 1), np.float32), grad0=np.zeros((nv, 3), np.float32))
        if want_images:
            r.update(pred0=np.zeros((n, s, s), np.float32), target=np.zeros((n, s, s), np.float32),
                     tri0=np.zeros((n, s, s), np.float32), lossimg0=np.zeros((s, s), np.float32))
        g = r.get
        self._call("aa_fit", _fp(pos0), _U32(nv), _fp(faces), _U32(nf), _fp(tgt_pos),
                   _U32(tgt_pos.shape[0]), _fp(tgt_faces), _U32(tgt_faces.shape[0]), _fp(mvps),
                   _U32(n), _U32(s), _U32(samples), C.c_float(lr), _U32(iters), _fp(r["pos"]),
                   _fp(r["m"]), _fp(r["v"]), _fp(r["t"]), _fp(r["loss"]), _fp(r["grad0"]),
                   _fp(g("pred0")), _fp(g("target")), _fp(g("tri0")), _fp(g("lossimg0")))
        return r


    # ---- texture path ----------------------------------------------------
    def uv_sphere(self, stacks, slices):
        nv, nf = _U32(), _U32()
        self._call("uv_sphere", _U32(stacks), _U32(slices), C.byref(nv), C.byref(nf), None,
                   None, None)
        pos = np.zeros((nv.value, 3), np.float32)
        uv = np.zeros((nv.value, 2), np.float32)
        faces = np.zeros((nf.value, 3), np.float32)
        self._call("uv_sphere", _U32(stacks), _U32(slices), C.byref(nv), C.byref(nf), _fp(pos),
                   _fp(uv), _fp(faces))
        return pos, uv, faces

    def gather_inv_uv_bilinear(self, gy, inv_uv, uv):
        """gy {sh, sw, nc}, inv_uv {th, tw, 4}, uv {sh, sw, 2} -> {th, tw, nc}."""
        gy, inv_uv, uv = _f32(gy), _f32(inv_uv), _f32(uv)
        sh, sw, nc = gy.shape
        th, tw = inv_uv.shape[:2]
        out = np.zeros((th, tw, nc), np.float32)
        self._call("gather_inv_uv_bilinear" if self.prefix == "or_" else "gather_bilinear",
                   _fp(gy), _U32(nc), _U32(sw), _U32(sh), _fp(inv_uv), _U32(tw), _U32(th),
                   _fp(uv), _fp(out))
        return out

    def tex_fit(self, pos, uv, faces, mvps, screen, gt_tex, tex0, lr=1e-2, iters=1,
                want_images=True):
        """The C3 texture fit; mvps {n_sets, n_views, 16}; textures {th, tw, 4}."""
        pos, uv, faces, mvps = _f32(pos), _f32(uv), _f32(faces), _f32(mvps)
        gt_tex, tex0 = _f32(gt_tex), _f32(tex0)
        n_sets, n = mvps.shape[0], mvps.shape[1]
        th, tw = gt_tex.shape[:2]
        s = screen
        z = lambda *sh: np.zeros(sh, np.float32)
        r = dict(tex=z(th, tw, 4), m=z(th, tw, 4), v=z(th, tw, 4), t=z(1),
                 loss=z(max(iters, 1)), grad0=z(th, tw, 4))
        if want_images:
            r.update(pred0=z(n, s, s, 4), target0=z(n, s, s, 4), lossimg0=z(s, s, 4),
                     uv0=z(n, s, s, 2), invuv0=z(n, th, tw, 4))
        g = r.get
        self._call("tex_fit", _fp(pos), _U32(pos.shape[0]), _fp(uv), _fp(faces),
                   _U32(faces.shape[0]), _fp(mvps), _U32(n_sets), _U32(n), _U32(s), _U32(tw),
                   _U32(th), _fp(gt_tex), _fp(tex0), C.c_float(lr), _U32(iters), _fp(r["tex"]),
                   _fp(r["m"]), _fp(r["v"]), _fp(r["t"]), _fp(r["loss"]), _fp(r["grad0"]),
                   _fp(g("pred0")), _fp(g("target0")), _fp(g("lossimg0")), _fp(g("uv0")),
                   _fp(g("invuv0")))
        return r

    # ---- PBR / IBL ops ----------------------------------------------------
    def equirect_sample(self, map_, dirs, gy=None):
        """map {mh, mw, n}, dirs {dh, dw, 3}; with gy {dh, dw, n} the map VJP."""
        map_, dirs = _f32(map_), _f32(dirs)
        mh, mw, n = map_.shape
        dh, dw = dirs.shape[:2]
        if gy is None:
            out = np.zeros((dh, dw, n), np.float32)
        else:
            gy = _f32(gy)
            out = np.zeros((mh, mw, n), np.float32)
        self._call("equirect_sample", _fp(map_), _U32(mw), _U32(mh), _U32(n), _fp(dirs),
                   _U32(dw), _U32(dh), _fp(gy), _fp(out))
        return out

    def avg_pool2x2(self, x, gy=None):
        x = _f32(x)
        h, w, n = x.shape
        out = np.zeros(((h + 1) // 2, (w + 1) // 2, n) if gy is None else (h, w, n), np.float32)
        self._call("avg_pool2x2", _fp(x), _U32(w), _U32(h), _U32(n),
                   _fp(None if gy is None else _f32(gy)), _fp(out))
        return out

    def irradiance_conv(self, env, ow, oh, gy=None):
        env = _f32(env)
        sh, sw, n = env.shape
        out = np.zeros((oh, ow, n) if gy is None else (sh, sw, n), np.float32)
        self._call("irradiance_conv", _fp(env), _U32(sw), _U32(sh), _U32(n), _U32(ow), _U32(oh),
                   _fp(None if gy is None else _f32(gy)), _fp(out))
        return out

    def prefilter_conv(self, env, ow, oh, roughness, gy=None):
        env = _f32(env)
        sh, sw, n = env.shape
        out = np.zeros((oh, ow, n) if gy is None else (sh, sw, n), np.float32)
        self._call("prefilter_conv", _fp(env), _U32(sw), _U32(sh), _U32(n), _U32(ow), _U32(oh),
                   C.c_float(roughness), _fp(None if gy is None else _f32(gy)), _fp(out))
        return out

    def prefilter_env(self, env, ow, oh, roughness, n_samples):
        env = _f32(env)
        sh, sw, n = env.shape
        out = np.zeros((oh, ow, n), np.float32)
        self._call("prefilter_env", _fp(env), _U32(sw), _U32(sh), _U32(n), _U32(ow), _U32(oh),
                   C.c_float(roughness), _U32(n_samples), _fp(out))
        return out

    def brdf_lut(self, w, h, n_samples):
        out = np.zeros((h, w, 2), np.float32)
        self._call("brdf_lut", _U32(w), _U32(h), _U32(n_samples), _fp(out))
        return out

    def pbr_fit(self, scene, iters=1, want_images=True):
        """The C5 PBR/IBL fit on a scene dict (pos, normal, uv, faces, mvps
        {N,16}, frames {N,12}, light {6}, screen, levels, lr, gt_albedo,
        gt_mr {th,tw,3}, gt_env {eh,ew,3}, albedo0, mr0, env0)."""
        a = {k: (_f32(v) if isinstance(v, np.ndarray) else v) for k, v in scene.items()}
        n = a["mvps"].shape[0]
        th, tw = a["gt_albedo"].shape[:2]
        eh, ew = a["gt_env"].shape[:2]
        s = a["screen"]
        z = lambda *sh: np.zeros(sh, np.float32)
        r = dict(albedo=z(th, tw, 3), mr=z(th, tw, 3), env=z(eh, ew, 3), loss=z(max(iters, 1)),
                 g_albedo0=z(th, tw, 3), g_mr0=z(th, tw, 3), g_env0=z(eh, ew, 3))
        if want_images:
            r.update(pred0=z(n, s, s, 3), target0=z(n, s, s, 3), mask0=z(n, s, s))
        g = r.get
        self._call("pbr_fit", _fp(a["pos"]), _fp(a["normal"]), _U32(a["pos"].shape[0]),
                   _fp(a["uv"]), _fp(a["faces"]), _U32(a["faces"].shape[0]), _fp(a["mvps"]),
                   _fp(a["frames"]), _fp(a["light"]), _U32(n), _U32(s), _U32(tw), _U32(th),
                   _U32(ew), _U32(eh), _U32(a["levels"]), _fp(a["gt_albedo"]), _fp(a["gt_mr"]),
                   _fp(a["gt_env"]), _fp(a["albedo0"]), _fp(a["mr0"]), _fp(a["env0"]),
                   C.c_float(a["lr"]), _U32(iters), _fp(r["albedo"]), _fp(r["mr"]), _fp(r["env"]),
                   _fp(r["loss"]), _fp(r["g_albedo0"]), _fp(r["g_mr0"]), _fp(r["g_env0"]),
                   _fp(g("pred0")), _fp(g("target0")), _fp(g("mask0")))
        return r


class Oracle(_Lib):
    """The C restatement (oracle/dressi_oracle.c)."""

    prefix = "or_"

    def __init__(self, path: str = ORACLE_SO):
        super().__init__(path)
        self.fn("hash_to_unit").restype = C.c_float
        self.fn("wang_hash").restype = C.c_uint32
        self.fn("vertex_faces_tex").restype = C.c_uint32

    # functions of the restatement that return a status (the rest are void)
    _STATUS = frozenset(("equirect_sample", "avg_pool2x2", "irradiance_conv", "prefilter_conv",
                         "prefilter_env", "brdf_lut", "pbr_fit"))

    def _call(self, name, *args):
        rc = self.fn(name)(*args)
        if name in self._STATUS and rc != 0:
            raise RuntimeError(f"or_{name} failed ({rc})")

    def rasterize_soft(self, soft_clip, face_id, faces_soft, hard_clip, faces_tex, w, h, radius,
                       prev=None, vtx_faces=None):
        sc, fi, fs = _f32(soft_clip), _f32(face_id), _f32(faces_soft)
        hc, ft = _f32(hard_clip), _f32(faces_tex)
        out = np.zeros((h, w, 4), np.float32)
        self.fn("rasterize_soft")(_fp(sc), _fp(fi), _fp(fs), _fp(hc), _U32(hc.shape[0]), _fp(ft),
                                  _U32(ft.shape[0]), _U32(w), _U32(h), C.c_float(radius),
                                  _fp(None if prev is None else _f32(prev)), _fp(out))
        return out

    def lookup_faces(self, attr, faces, corner):
        attr, faces = _f32(attr), _f32(faces)
        out = np.zeros((faces.shape[0], attr.shape[1]), np.float32)
        self.fn("lookup_faces")(_fp(attr), _U32(attr.shape[1]), _fp(faces), _U32(faces.shape[0]),
                                _U32(corner), _fp(out))
        return out

    def vertex_faces_tex(self, faces, n_verts):
        faces = _f32(faces)
        deg = self.fn("vertex_faces_tex")(_fp(faces), _U32(faces.shape[0]), _U32(n_verts), None,
                                          _U32(0))
        out = np.zeros((deg, n_verts), np.float32)
        self.fn("vertex_faces_tex")(_fp(faces), _U32(faces.shape[0]), _U32(n_verts), _fp(out),
                                    _U32(out.size))
        return out

    def icosphere(self, level):
        nv, nf = _U32(), _U32()
        self.fn("icosphere")(_U32(level), C.byref(nv), C.byref(nf), None, None)
        pos = np.zeros((nv.value, 3), np.float32)
        faces = np.zeros((nf.value, 3), np.float32)
        self.fn("icosphere")(_U32(level), C.byref(nv), C.byref(nf), _fp(pos), _fp(faces))
        return pos, faces

    def look_at(self, eye, center=(0, 0, 0), up=(0, 1, 0)):
        e, c, u = _f32(eye), _f32(center), _f32(up)
        m = np.zeros(16, np.float32)
        self.fn("look_at")(_fp(e), _fp(c), _fp(u), _fp(m))
        return m

    def perspective_vk(self, fovy, aspect, zn, zf):
        m = np.zeros(16, np.float32)
        self.fn("perspective_vk")(C.c_float(fovy), C.c_float(aspect), C.c_float(zn),
                                  C.c_float(zf), _fp(m))
        return m

    def mat4_mul(self, a, b):
        r = np.zeros(16, np.float32)
        self.fn("mat4_mul")(_fp(_f32(a)), _fp(_f32(b)), _fp(r))
        return r

    def randn(self, seed, n):
        out = np.zeros(n, np.float32)
        self.fn("randn")(C.c_uint64(seed), _U32(n), _fp(out))
        return out

    def transform_to_clip(self, pos, mvp):
        pos = _f32(pos)
        out = np.zeros((pos.shape[0], 4), np.float32)
        self.fn("transform_to_clip")(_fp(pos), _U32(pos.shape[0]), _fp(_f32(mvp)), _fp(out))
        return out

    def hash_to_unit(self, f, s, seed, salt):
        return self.fn("hash_to_unit")(_U32(f), _U32(s), _U32(seed), _U32(salt))

    def wang_hash(self, x):
        return self.fn("wang_hash")(_U32(x))

    def antialias(self, img, tri, clip, faces):
        img, tri, clip, faces = _f32(img), _f32(tri), _f32(clip), _f32(faces)
        h, w = tri.shape
        nc = 1 if img.ndim == 2 else img.shape[2]
        out = np.zeros(img.shape, np.float32)
        self.fn("antialias")(_fp(img), _U32(nc), _fp(tri), _fp(clip), _U32(clip.shape[0]),
                             _fp(faces), _U32(faces.shape[0]), _U32(w), _U32(h), _fp(out))
        return out

    def antialias_bwd_img(self, gy, tri, clip, faces):
        gy, tri, clip, faces = _f32(gy), _f32(tri), _f32(clip), _f32(faces)
        h, w = tri.shape
        nc = 1 if gy.ndim == 2 else gy.shape[2]
        out = np.zeros(gy.shape, np.float32)
        self.fn("antialias_bwd_img")(_fp(gy), _U32(nc), _fp(tri), _fp(clip),
                                     _U32(clip.shape[0]), _fp(faces), _U32(faces.shape[0]),
                                     _U32(w), _U32(h), _fp(out))
        return out

    def antialias_bwd_vtx(self, gy, img, tri, clip, faces, vtx_faces, seed, n_samples,
                          wide=True):
        """n_samples > 0 and wide: the {deg, V, 4} partials; else {V, 4}."""
        gy, img, tri, clip = _f32(gy), _f32(img), _f32(tri), _f32(clip)
        faces, vtx_faces = _f32(faces), _f32(vtx_faces)
        h, w = tri.shape
        nc = 1 if gy.ndim == 2 else gy.shape[2]
        deg, nv = vtx_faces.shape
        is_wide = bool(wide and n_samples > 0)
        out = np.zeros((deg if is_wide else 1, nv, 4), np.float32)
        self.fn("antialias_bwd_vtx")(_fp(gy), _fp(img), _U32(nc), _fp(tri), _fp(clip),
                                     _U32(nv), _fp(faces), _U32(faces.shape[0]), _fp(vtx_faces),
                                     _U32(deg), C.c_float(seed), _U32(n_samples),
                                     C.c_int(1 if is_wide else 0), _U32(w), _U32(h), _fp(out))
        return out if is_wide else out[0]

    def col_sum(self, x):
        x = _f32(x)
        h, w, nc = x.shape
        out = np.zeros((w, nc), np.float32)
        self.fn("col_sum")(_fp(x), _U32(nc), _U32(w), _U32(h), _fp(out))
        return out

    def gather_dist_grad(self, gy, rs, clip, faces, vtx_faces, wide=True):
        """gy, rs {h, w, 4}; -> wide {deg, V, 4} or {V, 4}."""
        gy, rs, clip, faces, vf = (_f32(a) for a in (gy, rs, clip, faces, vtx_faces))
        h, w = rs.shape[:2]
        deg, nv = vf.shape
        out = np.zeros((deg if wide else 1, nv, 4), np.float32)
        self.fn("gather_dist_grad")(_fp(gy), _fp(rs), _fp(clip), _U32(nv), _fp(faces),
                                    _U32(faces.shape[0]), _fp(vf), _U32(deg),
                                    C.c_int(1 if wide else 0), _U32(w), _U32(h), _fp(out))
        return out if wide else out[0]

    def texture_bilinear(self, tex, uv):
        """tex {th, tw, nc}, uv {..., 2} -> {..., nc}."""
        tex, uv = _f32(tex), _f32(uv)
        th, tw, nc = tex.shape
        n_px = uv.size // 2
        out = np.zeros(uv.shape[:-1] + (nc,), np.float32)
        self.fn("texture_bilinear")(_fp(tex), _U32(tw), _U32(th), _U32(nc), _fp(uv),
                                    C.c_size_t(n_px), _fp(out))
        return out

    def texture_nearest(self, tex, uv):
        """tex {th, tw, nc}, uv {..., 2} -> {..., nc} (nearest, clamp to edge)."""
        tex, uv = _f32(tex), _f32(uv)
        th, tw, nc = tex.shape
        n_px = uv.size // 2
        out = np.zeros(uv.shape[:-1] + (nc,), np.float32)
        self.fn("texture_nearest")(_fp(tex), _U32(tw), _U32(th), _U32(nc), _fp(uv),
                                   C.c_size_t(n_px), _fp(out))
        return out

    def gather_inv_uv(self, gy, inv_uv, uv):
        """GatherByInverseUV: gy {sh, sw, nc}, inv_uv {th, tw, 4}, uv {sh, sw, 2}
        -> {th, tw, nc}."""
        gy, inv_uv, uv = _f32(gy), _f32(inv_uv), _f32(uv)
        sh, sw, nc = gy.shape
        th, tw = inv_uv.shape[:2]
        out = np.zeros((th, tw, nc), np.float32)
        self.fn("gather_inv_uv")(_fp(gy), _U32(nc), _U32(sw), _U32(sh), _fp(inv_uv), _U32(tw),
                                 _U32(th), _fp(uv), _fp(out))
        return out

    def uv_as_clip(self, uv):
        uv = _f32(uv)
        out = np.zeros((uv.shape[0], 4), np.float32)
        self.fn("uv_as_clip")(_fp(uv), _U32(uv.shape[0]), _fp(out))
        return out

    def screen_attr(self, clip, w, h):
        clip = _f32(clip)
        out = np.zeros((clip.shape[0], 4), np.float32)
        self.fn("screen_attr")(_fp(clip), _U32(clip.shape[0]), _U32(w), _U32(h), _fp(out))
        return out

    def hsr_forward(self, rs, tri0, tri1, tri2, target, radius):
        rs, target = _f32(rs), _f32(target)
        h, w = target.shape
        pred = np.zeros((h, w), np.float32)
        vl = np.zeros((h, w), np.float32)
        self.fn("hsr_forward")(_fp(rs), _fp(_f32(tri0)), _fp(_f32(tri1)), _fp(_f32(tri2)),
                               _U32(tri0.shape[0]), _fp(target), _U32(w), _U32(h),
                               C.c_float(radius), _fp(pred), _fp(vl))
        return pred, vl

    def hsr_backward(self, rs, tri0, tri1, tri2, target, radius):
        rs, target = _f32(rs), _f32(target)
        h, w = target.shape
        gys = [np.zeros((h, w, 4), np.float32) for _ in range(3)]
        self.fn("hsr_backward")(_fp(rs), _fp(_f32(tri0)), _fp(_f32(tri1)), _fp(_f32(tri2)),
                                _U32(tri0.shape[0]), _fp(target), _U32(w), _U32(h),
                                C.c_float(radius), *[_fp(g) for g in gys])
        return gys


class Reference(_Lib):
    """The reference's own CPU evaluator (oracle/_ref, built from the reference
    sources by oracle/Makefile)."""

    prefix = "refh_"

    def __init__(self, path: str = REF_SO):
        super().__init__(path)
        self.fn("last_error").restype = C.c_char_p

    def _call(self, name, *args):
        rc = self.fn(name)(*args)
        if rc != 0:
            raise RuntimeError(self.fn("last_error")().decode())

    def rasterize_soft(self, soft_clip, face_id, faces_soft, hard_clip, faces_tex, w, h, radius,
                       prev=None, vtx_faces=None):
        sc, fi, fs = _f32(soft_clip), _f32(face_id), _f32(faces_soft)
        hc, ft = _f32(hard_clip), _f32(faces_tex)
        if vtx_faces is None:
            vtx_faces = np.full((1, hc.shape[0]), -1, np.float32)
        vf = _f32(vtx_faces)
        out = np.zeros((h, w, 4), np.float32)
        self._call("rasterize_soft", _fp(sc), _fp(fi), _fp(fs), _fp(hc), _U32(hc.shape[0]),
                   _fp(ft), _fp(vf), _U32(vf.shape[0]), _U32(ft.shape[0]), _U32(w), _U32(h),
                   C.c_float(radius), _fp(None if prev is None else _f32(prev)), _fp(out))
        return out

    def vertex_faces_tex(self, faces, n_verts):
        faces = _f32(faces)
        deg = _U32()
        self._call("vertex_faces_tex", _fp(faces), _U32(faces.shape[0]), _U32(n_verts),
                   C.byref(deg), None, _U32(0))
        out = np.zeros((deg.value, n_verts), np.float32)
        self._call("vertex_faces_tex", _fp(faces), _U32(faces.shape[0]), _U32(n_verts),
                   C.byref(deg), _fp(out), _U32(out.size))
        return out

    def icosphere(self, level):
        nv, nf = _U32(), _U32()
        self._call("icosphere", _U32(level), C.byref(nv), C.byref(nf), None, None)
        pos = np.zeros((nv.value, 3), np.float32)
        faces = np.zeros((nf.value, 3), np.float32)
        self._call("icosphere", _U32(level), C.byref(nv), C.byref(nf), _fp(pos), _fp(faces))
        return pos, faces


def _ref_antialias(self, img, tri, clip, faces, vtx_faces):
    img, tri, clip, faces, vtx_faces = (_f32(a) for a in (img, tri, clip, faces, vtx_faces))
    h, w = tri.shape
    nc = 1 if img.ndim == 2 else img.shape[2]
    deg, nv = vtx_faces.shape
    out = np.zeros(img.shape, np.float32)
    self._call("antialias", _fp(img), _U32(nc), _fp(tri), _fp(clip), _U32(nv), _fp(faces),
               _U32(faces.shape[0]), _fp(vtx_faces), _U32(deg), _U32(w), _U32(h), _fp(out))
    return out


def _ref_antialias_bwd(self, gy, img, tri, clip, faces, vtx_faces, seed, n_samples):
    """(g_img {like gy}, wide {deg, V, 4} or None, g_vtx {V, 4})."""
    gy, img, tri, clip, faces, vtx_faces = (_f32(a) for a in (gy, img, tri, clip, faces,
                                                              vtx_faces))
    h, w = tri.shape
    nc = 1 if gy.ndim == 2 else gy.shape[2]
    deg, nv = vtx_faces.shape
    g_img = np.zeros(gy.shape, np.float32)
    wide = np.zeros((deg, nv, 4), np.float32) if n_samples > 0 else None
    g_vtx = np.zeros((nv, 4), np.float32)
    self._call("antialias_bwd", _fp(gy), _fp(img), _U32(nc), _fp(tri), _fp(clip), _U32(nv),
               _fp(faces), _U32(faces.shape[0]), _fp(vtx_faces), _U32(deg), C.c_float(seed),
               _U32(n_samples), _U32(w), _U32(h), _fp(g_img), _fp(wide), _fp(g_vtx))
    return g_img, wide, g_vtx


def _ref_rasterize_soft_bwd(self, soft_clip, face_id, faces_soft, hard_clip, faces_tex,
                            vtx_faces, w, h, radius, gy):
    """(wide {deg, V, 4}, g_clip {V, 4}) of RasterizeSoft's backward."""
    sc, fi, fs, hc, ft, vf = (_f32(a) for a in (soft_clip, face_id, faces_soft, hard_clip,
                                                 faces_tex, vtx_faces))
    gy = _f32(gy)
    deg, nv = vf.shape
    wide = np.zeros((deg, nv, 4), np.float32)
    g = np.zeros((nv, 4), np.float32)
    self._call("rasterize_soft_bwd", _fp(sc), _fp(fi), _fp(fs), _fp(hc), _U32(nv), _fp(ft),
               _fp(vf), _U32(deg), _U32(ft.shape[0]), _U32(w), _U32(h), C.c_float(radius),
               _fp(gy), _fp(wide), _fp(g))
    return wide, g


def _ref_texture_bilinear(self, tex, uv):
    """tex {th, tw, nc}, uv {uh, uw, 2} -> {uh, uw, nc}."""
    tex, uv = _f32(tex), _f32(uv)
    th, tw, nc = tex.shape
    uh, uw = uv.shape[:2]
    out = np.zeros((uh, uw, nc), np.float32)
    self._call("texture_bilinear", _fp(tex), _U32(tw), _U32(th), _U32(nc), _fp(uv), _U32(uw),
               _U32(uh), _fp(out))
    return out


def face_id_buffer(rs):
    """The fused plan's face-id buffer for RasterizeSoft output `rs` (dist,
    fid, hard z, coverage): face + 1 where covered, 0 elsewhere, bit 31 set
    where the winning fragment is a rim fragment (signed distance < 0)."""
    rs = np.asarray(rs, np.float32)
    ids = np.where(rs[..., 3] > 0, rs[..., 1] + 1, 0).astype(np.uint32)
    rim = (rs[..., 3] > 0) & (rs[..., 0] < 0)
    return ids | np.where(rim, np.uint32(0x80000000), np.uint32(0))


def have_reference() -> bool:
    return os.path.exists(REF_SO)


Reference.antialias = _ref_antialias
Reference.antialias_bwd = _ref_antialias_bwd
Reference.texture_bilinear = _ref_texture_bilinear
Reference.rasterize_soft_bwd = _ref_rasterize_soft_bwd
