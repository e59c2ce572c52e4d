"""Host-side mirror of the split-sum PBR / IBL material + environment fit
(examples/common/pbr_graph.cpp shading, src/core/ibl.cpp maps, in-graph Adam
as in examples/pbr_material_optimization/run.cpp and
examples/pbr_envmap_optimization/run.cpp) over the fused plan of
include/dressi_hip.h (dressi_pbr_*), plus its synthetic workload.

Workload c5 (fp32): icosphere subdivision 5 (10242 v / 20480 f), unit radius,
normals = positions, uv = the equirect projection of the vertex direction
(u = atan2(z, x) / 2pi + 0.5, v = acos(y) / pi, as the IBL maps); 1024^2
screen, 6 views on the material example's camera ring (eye = (2.2 sin a
0.92, 0.85, 2.2 cos a 0.92), a = 2 pi i / 6, PerspectiveVk(45 deg, 1, 0.1,
10)), point light (2, 2, 2) with colour (20, 20, 20); 512^2 albedo (RGB) and
metallic-roughness (G = roughness, B = metallic) textures, ground truth
U[0.05, 0.95] per texel and channel (R of mr = 0); environment 512 x 256
RGB: 0.3 exp(0.6 z) with z a bilinearly upsampled 32 x 16 field of standard
normals, plus 3 Gaussian lobes (random unit directions, widths U[0.08, 0.25]
rad, per-channel amplitudes U[4, 16]); irradiance map 32 x 16 (env pooled to
64 x 32), 6 prefiltered levels from 128 x 64 (env pooled to 128 x 64),
roughness i / 5, BRDF LUT 256^2 x 512 samples. Optimisation starts from 0.5
materials and a constant 0.3 environment; L1 loss on the Reinhard-mapped
image, Adam lr 1e-2 (b1 .9, b2 .999, eps 1e-8) on albedo, mr and env; 100
iterations.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import check, lib
from .runtime import Context, icosphere, look_at, mat4_mul, perspective_vk, randn, uniform

_FP = C.POINTER(C.c_float)


def _fp(a):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_FP)


@dataclass(frozen=True)
class PbrWorkload:
    name: str
    level: int         # icosphere subdivision
    screen: int
    views: int
    tex: int           # albedo / mr texture side
    env_w: int
    env_h: int
    levels: int        # prefiltered levels
    lr: float
    iters: int
    seed: int


PBR_WORKLOADS = {
    "c5": PbrWorkload("c5", 5, 1024, 6, 512, 512, 256, 6, 1e-2, 100, 5),
}


def equirect_uv(pos: np.ndarray) -> np.ndarray:
    """{V,2} float32 equirect uv of the (unit) vertex directions."""
    p = pos.astype(np.float64)
    d = p / np.linalg.norm(p, axis=1, keepdims=True)
    u = np.arctan2(d[:, 2], d[:, 0]) / (2.0 * math.pi) + 0.5
    v = np.arccos(np.clip(d[:, 1], -1.0, 1.0)) / math.pi
    return np.stack([u, v], 1).astype(np.float32)


def ring_cameras(n_views: int, screen: int) -> tuple[np.ndarray, np.ndarray]:
    """MVPs {N,16} and frames {N,12} (cam_pos, cam_fwd, cam_right * tan(fov/2),
    cam_up * tan(fov/2)) of examples/pbr_material_optimization/run.cpp:
    189-236 (aspect 1)."""
    fov = np.float32(45.0 * 3.14159265 / 180.0)
    tan_half = np.float32(math.tan(float(fov) * 0.5))
    proj = perspective_vk(float(fov), 1.0, 0.1, 10.0)
    mvps = np.zeros((n_views, 16), np.float32)
    frames = np.zeros((n_views, 12), np.float32)
    for i in range(n_views):
        ang = np.float32(2.0 * 3.14159265 * i / n_views)
        eye = np.array([2.2 * math.sin(ang) * 0.92, 0.85, 2.2 * math.cos(ang) * 0.92], np.float32)
        vm = look_at(eye)
        mvps[i] = mat4_mul(proj, vm)
        frames[i, 0:3] = eye
        frames[i, 3:6] = [-vm[2], -vm[6], -vm[10]]
        frames[i, 6:9] = np.array([vm[0], vm[4], vm[8]], np.float32) * tan_half
        frames[i, 9:12] = np.array([vm[1], vm[5], vm[9]], np.float32) * tan_half
    return mvps, frames


def synthetic_env(w: int, h: int, seed: int) -> np.ndarray:
    """{h, w, 3} float32 HDR equirect map: seeded log-normal radiance (a
    smooth 32 x 16 normal field, bilinearly upsampled) + 3 Gaussian lobes."""
    cw, ch = 32, 16
    z = randn(seed, cw * ch).astype(np.float64).reshape(ch, cw)
    xs = (np.arange(w) + 0.5) / w * cw - 0.5
    ys = (np.arange(h) + 0.5) / h * ch - 0.5
    x0 = np.floor(xs).astype(int)
    y0 = np.floor(ys).astype(int)
    fx, fy = xs - x0, ys - y0
    xa, xb = x0 % cw, (x0 + 1) % cw
    ya, yb = np.clip(y0, 0, ch - 1), np.clip(y0 + 1, 0, ch - 1)
    zz = ((z[ya][:, xa] * (1 - fx) + z[ya][:, xb] * fx) * (1 - fy)[:, None]
          + (z[yb][:, xa] * (1 - fx) + z[yb][:, xb] * fx) * fy[:, None])
    env = 0.3 * np.exp(0.6 * zz)[..., None] * np.ones(3)
    u = (np.arange(w) + 0.5) / w
    v = (np.arange(h) + 0.5) / h
    phi = (u - 0.5) * 2.0 * math.pi
    th = v * math.pi
    d = np.stack([np.sin(th)[:, None] * np.cos(phi)[None, :],
                  np.cos(th)[:, None] * np.ones(w)[None, :],
                  np.sin(th)[:, None] * np.sin(phi)[None, :]], -1)
    r = uniform(seed + 1, 3 * 8).reshape(3, 8)
    mu = randn(seed + 2, 9).astype(np.float64).reshape(3, 3)
    for k in range(3):
        m = mu[k] / np.linalg.norm(mu[k])
        ang = np.arccos(np.clip(d @ m, -1.0, 1.0))
        sig = 0.08 + 0.17 * r[k, 0]
        amp = 4.0 + 12.0 * r[k, 1:4]
        env += np.exp(-ang ** 2 / (2.0 * sig * sig))[..., None] * amp
    return env.astype(np.float32)


def make_pbr_scene(level: int, screen: int, n_views: int, tex: int, env_w: int, env_h: int,
                   levels: int = 6, lr: float = 1e-2, seed: int = 5) -> dict:
    """The scene dict of a C5-style fit (see the module docstring)."""
    pos, faces = icosphere(level)
    mvps, frames = ring_cameras(n_views, screen)
    u = uniform(seed + 10, tex * tex * 5).reshape(tex, tex, 5)
    gt_albedo = (0.05 + 0.9 * u[..., 0:3]).astype(np.float32)
    gt_mr = np.zeros((tex, tex, 3), np.float32)
    gt_mr[..., 1:3] = 0.05 + 0.9 * u[..., 3:5]
    return dict(pos=pos, normal=pos.copy(), uv=equirect_uv(pos), faces=faces, mvps=mvps,
                frames=frames, light=np.array([2, 2, 2, 20, 20, 20], np.float32), screen=screen,
                levels=levels, lr=lr, gt_albedo=gt_albedo, gt_mr=gt_mr,
                gt_env=synthetic_env(env_w, env_h, seed),
                albedo0=np.full((tex, tex, 3), 0.5, np.float32),
                mr0=np.full((tex, tex, 3), 0.5, np.float32),
                env0=np.full((env_h, env_w, 3), 0.3, np.float32))


def workload_scene(wl: PbrWorkload) -> dict:
    return make_pbr_scene(wl.level, wl.screen, wl.views, wl.tex, wl.env_w, wl.env_h, wl.levels,
                          wl.lr, wl.seed)


class PbrFit:
    """One fused PBR / IBL fit plan (the DressiAD GpuPlan of the material +
    environment graph) on one device. `scene` is make_pbr_scene's dict."""

    def __init__(self, ctx: Context, scene: dict, keep_pred: bool = False,
                 keep_grad: bool = False):
        self.ctx = ctx
        a = {k: (np.ascontiguousarray(v, np.float32) if isinstance(v, np.ndarray) else v)
             for k, v in scene.items()}
        self.n_views = a["mvps"].shape[0]
        self.screen = int(a["screen"])
        self.tex_h, self.tex_w = a["gt_albedo"].shape[:2]
        self.env_h, self.env_w = a["gt_env"].shape[:2]
        self.levels = int(a["levels"])
        self.n_verts, self.n_faces = len(a["pos"]), len(a["faces"])
        d = _lib.PbrDesc(len(a["pos"]), len(a["faces"]), self.n_views, self.screen, self.screen,
                         self.tex_w, self.tex_h, self.env_w, self.env_h, self.levels,
                         float(a["lr"]), 0.9, 0.999, 1e-8,
                         (_lib.PBR_KEEP_PRED if keep_pred else 0)
                         | (_lib.PBR_KEEP_GRAD if keep_grad else 0))
        h = C.c_void_p()
        check(lib.dressi_pbr_create(ctx.handle, C.byref(d), C.byref(h)))
        self.handle = h
        check(lib.dressi_pbr_set_scene(h, _fp(a["pos"]), _fp(a["normal"]), _fp(a["uv"]),
                                       _fp(a["faces"]), _fp(a["mvps"]), _fp(a["frames"]),
                                       _fp(a["light"])))
        check(lib.dressi_pbr_set_target(h, _fp(a["gt_albedo"]), _fp(a["gt_mr"]),
                                        _fp(a["gt_env"])))
        self.set_state(a["albedo0"], a["mr0"], a["env0"])

    @classmethod
    def from_workload(cls, ctx: Context, name: str, **kw) -> "PbrFit":
        return cls(ctx, workload_scene(PBR_WORKLOADS[name]), **kw)

    def close(self) -> None:
        if self.handle:
            check(lib.dressi_pbr_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_state(self, albedo, mr, env, t: float = 0.0) -> None:
        f = lambda x: _fp(np.ascontiguousarray(x, np.float32))
        check(lib.dressi_pbr_set_state(self.handle, f(albedo), f(mr), f(env), float(t)))

    def state(self):
        alb = np.zeros((self.tex_h, self.tex_w, 3), np.float32)
        mr = np.zeros_like(alb)
        env = np.zeros((self.env_h, self.env_w, 3), np.float32)
        t = np.zeros(1, np.float32)
        check(lib.dressi_pbr_get_state(self.handle, _fp(alb), _fp(mr), _fp(env), _fp(t)))
        return alb, mr, env, float(t[0])

    def step(self, n: int = 1, graph: bool = True) -> None:
        fn = lib.dressi_pbr_step if graph else lib.dressi_pbr_step_eager
        check(fn(self.handle, n))

    def synchronize(self) -> None:
        self.ctx.synchronize()

    def read(self, which: int) -> np.ndarray:
        s, n = self.screen, self.n_views
        t, e = (self.tex_h, self.tex_w), (self.env_h, self.env_w)
        n_pref = 0
        w, h = min(128, self._psrc()[0]), min(64, self._psrc()[1])
        for _ in range(self.levels):
            n_pref += w * h
            w, h = max(w // 2, 1), max(h // 2, 1)
        shapes = {_lib.PBR_LOSS: (1,), _lib.PBR_PRED: (n, s, s, 4),
                  _lib.PBR_TARGET: (n, s, s, 4), _lib.PBR_G_ALBEDO: t + (4,),
                  _lib.PBR_G_MR: t + (4,), _lib.PBR_G_ENV: e + (4,), _lib.PBR_IRR: (16, 32, 4),
                  _lib.PBR_PREF: (n_pref, 4), _lib.PBR_GBUF0: (n, s, s, 4)}
        out = np.zeros(shapes[which], np.float32)
        check(lib.dressi_pbr_read(self.handle, which, out.ctypes.data_as(C.c_void_p),
                                  out.nbytes))
        return out

    @property
    def pooled_texels(self) -> int:
        """Texels of the pooled env levels (the irradiance and prefilter sources)."""
        w, h, n = self.env_w, self.env_h, 0
        while w > 64 or h > 32:
            w, h = (w + 1) // 2, (h + 1) // 2
            n += w * h
        return n

    @property
    def map_texels(self) -> int:
        """Texels of the irradiance map and every prefiltered level."""
        w, h = min(128, self._psrc()[0]), min(64, self._psrc()[1])
        n = 32 * 16
        for _ in range(self.levels):
            n += w * h
            w, h = max(w // 2, 1), max(h // 2, 1)
        return n

    @property
    def gather_maps(self) -> list[tuple[int, int, int]]:
        """(w, h, bands) of every map the shading samples (irradiance, each
        prefilter level, env): EquirectSampleBwd splits the dir rows into
        `bands` bands, doubling from 1 while w h bands < 65536 and bands <
        the dir image's height (f_ops.cpp:2823-2919)."""
        maps = [(32, 16)]
        w, h = min(128, self._psrc()[0]), min(64, self._psrc()[1])
        for _ in range(self.levels):
            maps.append((w, h))
            w, h = max(w // 2, 1), max(h // 2, 1)
        maps.append((self.env_w, self.env_h))
        out = []
        for w, h in maps:
            k = 1
            while w * h * k < 65536 and k < self.screen:
                k *= 2
            out.append((w, h, k))
        return out

    @property
    def prefilter_source(self) -> tuple[int, int]:
        """(w, h) of the pooled env level the prefilter convolution reads."""
        return self._psrc()

    @property
    def irradiance_source(self) -> tuple[int, int]:
        """(w, h) of the pooled env level the irradiance convolution reads."""
        w, h = self.env_w, self.env_h
        while w > 64 or h > 32:
            w, h = (w + 1) // 2, (h + 1) // 2
        return w, h

    def _psrc(self):
        w, h = self.env_w, self.env_h
        while w > 128 or h > 64:
            w, h = (w + 1) // 2, (h + 1) // 2
        return w, h

    def loss(self) -> float:
        return float(self.read(_lib.PBR_LOSS)[0])

    def profile(self, iters: int = 10) -> dict[str, float]:
        cap = 16
        names = C.create_string_buffer(64 * cap)
        usec = np.zeros(cap, np.float32)
        n = C.c_uint32()
        check(lib.dressi_pbr_profile(self.handle, iters, names, 64, _fp(usec), cap, C.byref(n)))
        return {names.raw[64 * i:64 * (i + 1)].split(b"\0")[0].decode(): float(usec[i])
                for i in range(n.value)}


__all__ = ["PbrWorkload", "PBR_WORKLOADS", "equirect_uv", "ring_cameras", "synthetic_env",
           "make_pbr_scene", "workload_scene", "PbrFit"]
