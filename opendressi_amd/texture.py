"""Host-side mirror of the texture-optimisation iteration (the graph of
examples/texture_optimization/run.cpp:112-145 with TextureBilinear, an RGBA
texture, the RGB L2 image loss and in-graph Adam) over the fused plan of
include/dressi_hip.h (dressi_tex_*), plus its synthetic workload.

Workload c3 (fp32): UV sphere GenerateUvSphere(stacks 128, slices 64) =
8385 v / 16256 f with its equirectangular uv; 1024^2 screen, 8 views per
iteration, each a random orbit camera (yaw U[0, 2pi), pitch U[-60, 60] deg,
distance 3, PerspectiveVk(45 deg, 1, 0.1, 10) * LookAt(eye, 0, +y)); a
1024^2 RGBA texture initialised to 0.5; target texture = per channel a sum
of 16 sinusoids with integer frequencies in u, v (1..8), random phases and
amplitudes, mapped into [0, 1] (alpha = 1); Adam lr 1e-2, b1 .9, b2 .999,
eps 1e-8; 100 iterations, camera set t (one set per iteration).
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import check, lib
from .runtime import Context, look_at, mat4_mul, perspective_vk, uniform, uv_sphere

_FP = C.POINTER(C.c_float)


def _fp(a):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_FP)


@dataclass(frozen=True)
class TexWorkload:
    name: str
    stacks: int
    slices: int
    screen: int
    tex: int
    views: int
    sets: int          # camera sets (one per iteration)
    lr: float
    iters: int
    seed: int


TEX_WORKLOADS = {
    "c3": TexWorkload("c3", 128, 64, 1024, 1024, 8, 100, 1e-2, 100, 3),
}


def orbit_cameras(n_sets: int, n_views: int, seed: int, dist: float = 3.0,
                  max_pitch_deg: float = 60.0, fov_deg: float = 45.0) -> np.ndarray:
    """{n_sets, n_views, 16} column-major MVPs of random orbit cameras."""
    u = uniform(seed, 2 * n_sets * n_views).reshape(n_sets, n_views, 2)
    proj = perspective_vk(fov_deg * 3.14159265 / 180.0, 1.0, 0.1, 10.0)
    out = np.zeros((n_sets, n_views, 16), np.float32)
    for s in range(n_sets):
        for v in range(n_views):
            yaw = 2.0 * math.pi * u[s, v, 0]
            pitch = math.radians(max_pitch_deg) * (2.0 * u[s, v, 1] - 1.0)
            eye = [dist * math.cos(pitch) * math.sin(yaw), dist * math.sin(pitch),
                   dist * math.cos(pitch) * math.cos(yaw)]
            out[s, v] = mat4_mul(proj, look_at(eye))
    return out


def sinusoid_texture(size: int, seed: int, n_waves: int = 16) -> np.ndarray:
    """{size, size, 4} float32 in [0, 1]: per RGB channel
    0.5 + 0.5 * sum_k a_k sin(2 pi (fx_k u + fy_k v) + phi_k) / sum_k a_k at
    texel centres, integer frequencies 1..8 (periodic across the u seam);
    alpha 1."""
    r = uniform(seed, 3 * n_waves * 4).reshape(3, n_waves, 4)
    c = (np.arange(size, dtype=np.float64) + 0.5) / size
    uu, vv = np.meshgrid(c, c)
    out = np.ones((size, size, 4), np.float32)
    for ch in range(3):
        fx = np.floor(r[ch, :, 0] * 8) + 1
        fy = np.floor(r[ch, :, 1] * 8) + 1
        ph = 2.0 * math.pi * r[ch, :, 2]
        amp = 0.2 + 0.8 * r[ch, :, 3]
        acc = np.zeros_like(uu)
        for k in range(n_waves):
            acc += amp[k] * np.sin(2.0 * math.pi * (fx[k] * uu + fy[k] * vv) + ph[k])
        out[..., ch] = (0.5 + 0.5 * acc / amp.sum()).astype(np.float32)
    return out


def make_tex_scene(w: TexWorkload):
    """(pos, uv, faces, mvps {sets, views, 16}, gt_tex, tex0) of a workload."""
    pos, uv, faces = uv_sphere(w.stacks, w.slices)
    mvps = orbit_cameras(w.sets, w.views, w.seed)
    gt = sinusoid_texture(w.tex, w.seed + 1)
    tex0 = np.full((w.tex, w.tex, 4), 0.5, np.float32)
    return pos, uv, faces, mvps, gt, tex0


class TextureFit:
    """One fused texture-fit plan (the DressiAD GpuPlan of the texture graph)
    on one device."""

    def __init__(self, ctx: Context, pos, uv, faces, mvps, screen: int, gt_tex, tex0,
                 lr: float = 1e-2, keep_images: bool = False, keep_grad: bool = False):
        self.ctx = ctx
        pos = np.ascontiguousarray(pos, np.float32)
        uv = np.ascontiguousarray(uv, np.float32)
        faces = np.ascontiguousarray(faces, np.float32)
        mvps = np.ascontiguousarray(mvps, np.float32)
        gt_tex = np.ascontiguousarray(gt_tex, np.float32)
        self.n_sets, self.n_views = mvps.shape[0], mvps.shape[1]
        self.n_verts, self.n_faces = len(pos), len(faces)
        self.screen = screen
        self.tex_h, self.tex_w = gt_tex.shape[:2]
        d = _lib.TexDesc(self.n_verts, self.n_faces, self.n_views, screen, screen, self.tex_w,
                         self.tex_h, self.n_sets, lr, 0.9, 0.999, 1e-8,
                         (_lib.TEX_KEEP_IMAGES if keep_images else 0)
                         | (_lib.TEX_KEEP_GRAD if keep_grad else 0))
        h = C.c_void_p()
        check(lib.dressi_tex_create(ctx.handle, C.byref(d), C.byref(h)))
        self.handle = h
        check(lib.dressi_tex_set_mesh(h, _fp(pos), _fp(uv), _fp(faces)))
        check(lib.dressi_tex_set_cameras(h, _fp(mvps)))
        check(lib.dressi_tex_set_target(h, _fp(gt_tex)))
        self.set_state(tex0)

    @classmethod
    def from_workload(cls, ctx: Context, name: str, **kw) -> "TextureFit":
        w = TEX_WORKLOADS[name]
        pos, uv, faces, mvps, gt, tex0 = make_tex_scene(w)
        return cls(ctx, pos, uv, faces, mvps, w.screen, gt, tex0, lr=w.lr, **kw)

    def close(self) -> None:
        if self.handle:
            check(lib.dressi_tex_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_state(self, tex, m=None, v=None, t: float = 0.0) -> None:
        f = lambda a: None if a is None else _fp(np.ascontiguousarray(a, np.float32))
        check(lib.dressi_tex_set_state(self.handle, f(tex), f(m), f(v), float(t)))

    def state(self):
        z = lambda: np.zeros((self.tex_h, self.tex_w, 4), np.float32)
        tex, m, v = z(), z(), z()
        t = np.zeros(1, np.float32)
        check(lib.dressi_tex_get_state(self.handle, _fp(tex), _fp(m), _fp(v), _fp(t)))
        return tex, m, v, float(t[0])

    def step(self, n: int = 1, graph: bool = True) -> None:
        fn = lib.dressi_tex_step if graph else lib.dressi_tex_step_eager
        check(fn(self.handle, n))

    def synchronize(self) -> None:
        self.ctx.synchronize()

    def read(self, which: int) -> np.ndarray:
        s, n, th, tw = self.screen, self.n_views, self.tex_h, self.tex_w
        shapes = {_lib.TEX_LOSS: ((s, s, 4), np.float32),
                  _lib.TEX_PRED: ((n, s, s, 4), np.float32),
                  _lib.TEX_TARGET: ((n, s, s, 4), np.float32),
                  _lib.TEX_FACE_ID: ((n, s, s), np.uint32),
                  _lib.TEX_GRAD: ((th, tw, 4), np.float32),
                  _lib.TEX_TEX: ((th, tw, 4), np.float32),
                  _lib.TEX_UV: ((n, s, s, 2), np.float32)}
        shape, dt = shapes[which]
        out = np.zeros(shape, dt)
        check(lib.dressi_tex_read(self.handle, which, out.ctypes.data_as(C.c_void_p), out.nbytes))
        return out

    def loss(self) -> float:
        return float(self.read(_lib.TEX_LOSS).astype(np.float64).sum())

    def profile(self, iters: int = 10) -> dict[str, float]:
        cap = 16
        names = C.create_string_buffer(64 * cap)
        usec = np.zeros(cap, np.float32)
        n = C.c_uint32()
        check(lib.dressi_tex_profile(self.handle, iters, names, 64, _fp(usec), cap, C.byref(n)))
        return {names.raw[64 * i:64 * (i + 1)].split(b"\0")[0].decode(): float(usec[i])
                for i in range(n.value)}


__all__ = ["TexWorkload", "TEX_WORKLOADS", "orbit_cameras", "sinusoid_texture",
           "make_tex_scene", "TextureFit"]
