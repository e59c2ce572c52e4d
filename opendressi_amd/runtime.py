"""Device context and host-side scene builders over the C ABI.

`Context` mirrors the reference's shared Vulkan context
(DressiAD::createContext, include/dressi/dressi_ad.h:53-55): one HIP device +
one stream; every op and plan created from it is stream-ordered on it.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import DressiError, check, lib

_FP = C.POINTER(C.c_float)


def _fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_FP)


class Context:
    def __init__(self, device: int = 0):
        h = C.c_void_p()
        check(lib.dressi_ctx_create(device, C.byref(h)))
        self.handle = h
        self.device = device

    def close(self) -> None:
        if self.handle:
            check(lib.dressi_ctx_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_stream(self, stream_ptr: int | None) -> None:
        """Order the context's work on `stream_ptr` (0: the null stream, which
        is torch's default stream); None restores the context's own."""
        if stream_ptr is None:
            check(lib.dressi_ctx_reset_stream(self.handle))
        else:
            check(lib.dressi_ctx_set_stream(self.handle, C.c_void_p(stream_ptr)))

    def use_torch_stream(self) -> None:
        """Order this context's work on torch's current HIP stream."""
        import torch
        self.set_stream(torch.cuda.current_stream(self.device).cuda_stream)

    def synchronize(self) -> None:
        check(lib.dressi_ctx_synchronize(self.handle))

    @property
    def device_name(self) -> str:
        buf = C.create_string_buffer(256)
        check(lib.dressi_ctx_device_name(self.handle, buf, 256))
        return buf.value.decode()


# ---- host-side scene builders (examples/common/geometry_utils.cpp,
# ---- examples/common/asset_utils.cpp, src/core/mesh_utils.cpp) -------------

def icosphere(level: int) -> tuple[np.ndarray, np.ndarray]:
    """GenerateIcosphere: unit-radius pos {V,3}, faces {F,3} (float ids)."""
    nv, nf = C.c_uint32(), C.c_uint32()
    check(lib.dressi_icosphere(level, C.byref(nv), C.byref(nf), None, None))
    pos = np.zeros((nv.value, 3), np.float32)
    faces = np.zeros((nf.value, 3), np.float32)
    check(lib.dressi_icosphere(level, C.byref(nv), C.byref(nf), _fp(pos), _fp(faces)))
    return pos, faces


def vertex_faces_tex(faces: np.ndarray, n_verts: int) -> np.ndarray:
    """VertexFacesTex: {max_deg, V} incident-face ids, -1 padding."""
    faces = np.ascontiguousarray(faces, np.float32)
    deg = C.c_uint32()
    check(lib.dressi_vertex_faces_tex(_fp(faces), len(faces), n_verts, C.byref(deg), None, 0))
    out = np.zeros((deg.value, n_verts), np.float32)
    check(lib.dressi_vertex_faces_tex(_fp(faces), len(faces), n_verts, C.byref(deg), _fp(out),
                                      out.size))
    return out


def look_at(eye, center=(0.0, 0.0, 0.0), up=(0.0, 1.0, 0.0)) -> np.ndarray:
    m = np.zeros(16, np.float32)
    lib.dressi_look_at(_fp(np.asarray(eye, np.float32)), _fp(np.asarray(center, np.float32)),
                       _fp(np.asarray(up, np.float32)), _fp(m))
    return m


def perspective_vk(fovy_rad: float, aspect: float, z_near: float, z_far: float) -> np.ndarray:
    m = np.zeros(16, np.float32)
    lib.dressi_perspective_vk(fovy_rad, aspect, z_near, z_far, _fp(m))
    return m


def mat4_mul(a, b) -> np.ndarray:
    r = np.zeros(16, np.float32)
    lib.dressi_mat4_mul(_fp(np.ascontiguousarray(a, np.float32)),
                        _fp(np.ascontiguousarray(b, np.float32)), _fp(r))
    return r


def uniform(seed: int, n: int) -> np.ndarray:
    """Seeded uniforms in (0, 1), float64: the SplitMix64 sequence of `seed`
    (outputs 1 .. n), top 53 bits + 0.5 ulp."""
    mask = np.uint64(0xFFFFFFFFFFFFFFFF)
    with np.errstate(over="ignore"):
        k = np.arange(1, n + 1, dtype=np.uint64)
        z = (np.uint64(seed) + k * np.uint64(0x9E3779B97F4A7C15)) & mask
        z = ((z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)) & mask
        z = ((z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)) & mask
        z = z ^ (z >> np.uint64(31))
    return ((z >> np.uint64(11)).astype(np.float64) + 0.5) * 2.0 ** -53


def randn(seed: int, n: int) -> np.ndarray:
    """Seeded standard normals: SplitMix64 uniforms in (0,1), Box-Muller
    (cosine branch) in double, rounded once to float32."""
    u = uniform(seed, 2 * n)
    u1, u2 = u[0::2], u[1::2]
    return (np.sqrt(-2.0 * np.log(u1)) * np.cos(6.283185307179586 * u2)).astype(np.float32)


def uv_sphere(stacks: int, slices: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """GenerateUvSphere: pos {V,3}, uv {V,2}, faces {F,3} (float ids)."""
    nv, nf = C.c_uint32(), C.c_uint32()
    check(lib.dressi_uv_sphere(stacks, slices, C.byref(nv), C.byref(nf), None, None, None))
    pos = np.zeros((nv.value, 3), np.float32)
    uv = np.zeros((nv.value, 2), np.float32)
    faces = np.zeros((nf.value, 3), np.float32)
    check(lib.dressi_uv_sphere(stacks, slices, C.byref(nv), C.byref(nf), _fp(pos), _fp(uv),
                               _fp(faces)))
    return pos, uv, faces


__all__ = ["Context", "DressiError", "icosphere", "vertex_faces_tex", "look_at",
           "perspective_vk", "mat4_mul", "randn", "uniform", "uv_sphere"]
