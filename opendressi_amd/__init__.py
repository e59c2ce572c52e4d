"""opendressi_amd -- MI355X-native Dressi-AD hot path: the silhouette fit
(HardSoftRas, screen-space AA), the texture fit and the PBR / IBL fit.

Hand-written gfx950 HIP kernels behind the C ABI of include/dressi_hip.h
(libdressi_hip.so, built in-tree by opendressi_amd.build). The first use of
any export loads the library and fails loudly when it is missing; importing
the package itself (e.g. to run the build) does not.
"""
import importlib

_EXPORTS = {
    "DressiError": "._lib", "EXPORTED": "._lib", "LIB_PATH": "._lib",
    "Context": ".runtime", "icosphere": ".runtime", "look_at": ".runtime",
    "mat4_mul": ".runtime", "perspective_vk": ".runtime", "randn": ".runtime",
    "vertex_faces_tex": ".runtime",
    "WORKLOADS": ".silhouette", "SilhouetteFit": ".silhouette", "Workload": ".silhouette",
    "camera_mvps": ".silhouette", "make_scene": ".silhouette",
    "uniform": ".runtime", "uv_sphere": ".runtime",
    "TEX_WORKLOADS": ".texture", "TexWorkload": ".texture", "TextureFit": ".texture",
    "make_tex_scene": ".texture", "orbit_cameras": ".texture", "sinusoid_texture": ".texture",
    "PBR_WORKLOADS": ".pbr", "PbrWorkload": ".pbr", "PbrFit": ".pbr",
    "make_pbr_scene": ".pbr", "ring_cameras": ".pbr", "synthetic_env": ".pbr",
}

__all__ = sorted(_EXPORTS)


def __getattr__(name):
    mod = _EXPORTS.get(name)
    if mod is None:
        raise AttributeError(f"module 'opendressi_amd' has no attribute {name!r}")
    return getattr(importlib.import_module(mod, __name__), name)
