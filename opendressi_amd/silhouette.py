"""Host-side mirror of the reference's silhouette fit
(examples/silhouette_optimization/run.cpp, technique hardsoftras with
peels = 1, or aa; no regularizers) over the fused plan of
include/dressi_hip.h, plus the synthetic workloads it is benchmarked on.

Workloads (all fp32, r = 3 px, 8 backward samples per face, Adam b1 .9,
b2 .999, eps 1e-8; target = StopGradient(Rasterize(target mesh)) per view,
AntiAlias'd for technique aa):

  c1      icosphere L3 (642 v / 1280 f), 256^2, 1 view (front, distance 3),
          target radius 1 + N(0, .05), lr 1e-3, 50 iterations
  c2      icosphere L4 (2562 v / 5120 f), 512^2, 4 orbit views (yaw
          0/90/180/270, pitch 15 deg, distance 3), noise N(0, .05), lr 1e-3,
          200 iterations
  c4      icosphere L6 (40962 v / 81920 f), 2048^2, the same 4 orbit views,
          noise N(0, .02) + 0.1 * P2(y) bump, lr 5e-4, 100 iterations,
          technique aa (target = AntiAlias of the target mask)
  c4_hsr  the same scene with HardSoftRas

Cameras: PerspectiveVk(45 deg, 1, 0.1, 10) * LookAt(eye, 0, +y).
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import check, lib
from .runtime import Context, icosphere, look_at, mat4_mul, perspective_vk, randn

_FP = C.POINTER(C.c_float)


def _fp(a):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_FP)


@dataclass(frozen=True)
class Workload:
    name: str
    level: int
    screen: int
    views: int          # 1 = front camera, else an orbit of `views` cameras
    noise: float
    bump: float
    lr: float
    iters: int
    seed: int
    technique: str = "hsr"  # "hsr" (HardSoftRas) or "aa" (screen-space AA)


WORKLOADS = {
    "c1": Workload("c1", 3, 256, 1, 0.05, 0.0, 1e-3, 50, 1),
    "c2": Workload("c2", 4, 512, 4, 0.05, 0.0, 1e-3, 200, 2),
    "c4": Workload("c4", 6, 2048, 4, 0.02, 0.1, 5e-4, 100, 4, "aa"),
    "c4_hsr": Workload("c4_hsr", 6, 2048, 4, 0.02, 0.1, 5e-4, 100, 4),
}


def camera_mvps(views: int, dist: float = 3.0, pitch_deg: float = 15.0,
                fov_deg: float = 45.0) -> np.ndarray:
    proj = perspective_vk(fov_deg * 3.14159265 / 180.0, 1.0, 0.1, 10.0)
    if views == 1:
        return mat4_mul(proj, look_at([0.0, 0.0, dist]))[None].copy()
    out = []
    for v in range(views):
        yaw = math.radians(360.0 * v / views)
        pitch = math.radians(pitch_deg)
        eye = [dist * math.cos(pitch) * math.sin(yaw), dist * math.sin(pitch),
               dist * math.cos(pitch) * math.cos(yaw)]
        out.append(mat4_mul(proj, look_at(eye)))
    return np.stack(out).astype(np.float32)


def make_scene(w: Workload):
    """(pos0, faces, target_pos, mvps) of a workload."""
    pos, faces = icosphere(w.level)
    r = 1.0 + w.noise * randn(w.seed, len(pos))
    if w.bump:
        r = r + np.float32(w.bump) * (1.5 * pos[:, 1] * pos[:, 1] - 0.5)
    tgt = (pos * r[:, None]).astype(np.float32)
    return pos, faces, tgt, camera_mvps(w.views)


class SilhouetteFit:
    """One fused HardSoftRas silhouette-fit plan (the DressiAD GpuPlan of the
    example graph) living on one device."""

    def __init__(self, ctx: Context, pos0: np.ndarray, faces: np.ndarray, mvps: np.ndarray,
                 screen: int, targets: np.ndarray | None = None,
                 target_mesh: tuple[np.ndarray, np.ndarray] | None = None,
                 radius_px: float = 3.0, samples: int = 8, lr: float = 1e-3,
                 keep_pred: bool = False, keep_grad: bool = False, technique: str = "hsr"):
        self.ctx = ctx
        pos0 = np.ascontiguousarray(pos0, np.float32)
        faces = np.ascontiguousarray(faces, np.float32)
        mvps = np.ascontiguousarray(mvps, np.float32).reshape(-1, 16)
        self.n_verts, self.n_faces, self.n_views = len(pos0), len(faces), len(mvps)
        self.screen = screen
        if technique not in ("hsr", "aa"):
            raise ValueError(f"technique must be 'hsr' or 'aa', got {technique!r}")
        self.technique = technique
        d = _lib.HsrDesc(self.n_verts, self.n_faces, self.n_views, screen, screen,
                         radius_px, samples, lr, 0.9, 0.999, 1e-8,
                         (_lib.HSR_KEEP_PRED if keep_pred else 0)
                         | (_lib.HSR_KEEP_GRAD if keep_grad else 0)
                         | (_lib.HSR_TECHNIQUE_AA if technique == "aa" else 0))
        h = C.c_void_p()
        check(lib.dressi_hsr_create(ctx.handle, C.byref(d), C.byref(h)))
        self.handle = h
        check(lib.dressi_hsr_set_mesh(h, _fp(faces), _fp(mvps)))
        if targets is not None:
            check(lib.dressi_hsr_set_targets(h, _fp(np.ascontiguousarray(targets, np.float32))))
        elif target_mesh is not None:
            tp = np.ascontiguousarray(target_mesh[0], np.float32)
            tf = np.ascontiguousarray(target_mesh[1], np.float32)
            check(lib.dressi_hsr_render_targets(h, _fp(tp), len(tp), _fp(tf), len(tf)))
        else:
            raise ValueError("targets or target_mesh required")
        self.set_state(pos0)

    @classmethod
    def from_workload(cls, ctx: Context, name: str, **kw) -> "SilhouetteFit":
        w = WORKLOADS[name]
        pos, faces, tgt, mvps = make_scene(w)
        kw.setdefault("technique", w.technique)
        return cls(ctx, pos, faces, mvps, w.screen, target_mesh=(tgt, faces), lr=w.lr, **kw)

    def close(self) -> None:
        if self.handle:
            check(lib.dressi_hsr_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_state(self, pos, m=None, v=None, t: float = 0.0) -> None:
        f = lambda a: None if a is None else _fp(np.ascontiguousarray(a, np.float32))
        check(lib.dressi_hsr_set_state(self.handle, f(pos), f(m), f(v), float(t)))

    def state(self):
        pos = np.zeros((self.n_verts, 3), np.float32)
        m = np.zeros_like(pos)
        v = np.zeros_like(pos)
        t = np.zeros(1, np.float32)
        check(lib.dressi_hsr_get_state(self.handle, _fp(pos), _fp(m), _fp(v), _fp(t)))
        return pos, m, v, float(t[0])

    def step(self, n: int = 1, graph: bool = True) -> None:
        """Enqueue n iterations (execStep x n) without synchronizing."""
        fn = lib.dressi_hsr_step if graph else lib.dressi_hsr_step_eager
        check(fn(self.handle, n))

    def synchronize(self) -> None:
        self.ctx.synchronize()

    @property
    def bin_capacity(self) -> int:
        """Entries per soft bin (grows after an iteration overflowed one)."""
        n = C.c_uint32()
        check(lib.dressi_hsr_bin_capacity(self.handle, C.byref(n)))
        return n.value

    def buffer(self, which: int) -> tuple[int, int]:
        p = C.c_void_p()
        b = C.c_size_t()
        check(lib.dressi_hsr_buffer(self.handle, which, C.byref(p), C.byref(b)))
        return p.value, b.value

    def read(self, which: int) -> np.ndarray:
        s, n, v = self.screen, self.n_views, self.n_verts
        shapes = {_lib.BUF_LOSS: ((s, s), np.float32), _lib.BUF_PRED: ((n, s, s), np.float32),
                  _lib.BUF_TARGET: ((n, s, s), np.float32),
                  _lib.BUF_FACE_ID: ((n, s, s), np.uint32), _lib.BUF_GRAD: ((v, 3), np.float32),
                  _lib.BUF_POS: ((v, 3), np.float32)}
        shape, dt = shapes[which]
        out = np.zeros(shape, dt)
        check(lib.dressi_hsr_read(self.handle, which, out.ctypes.data_as(C.c_void_p), out.nbytes))
        return out

    def loss(self) -> float:
        """Sum of the loss image (the example's loss_value, run.cpp:548-556)."""
        return float(self.read(_lib.BUF_LOSS).astype(np.float64).sum())

    def profile(self, iters: int = 10) -> dict[str, float]:
        cap = 16
        names = C.create_string_buffer(64 * cap)
        usec = np.zeros(cap, np.float32)
        n = C.c_uint32()
        check(lib.dressi_hsr_profile(self.handle, iters, names, 64, _fp(usec), cap, C.byref(n)))
        return {names.raw[64 * i:64 * (i + 1)].split(b"\0")[0].decode(): float(usec[i])
                for i in range(n.value)}


__all__ = ["Workload", "WORKLOADS", "camera_mvps", "make_scene", "SilhouetteFit"]
