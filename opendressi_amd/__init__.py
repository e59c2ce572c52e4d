"""opendressi_amd -- MI355X-native Dressi-AD HardSoftRas silhouette hot path.

Hand-written gfx950 HIP kernels behind the C ABI of include/dressi_hip.h
(libdressi_hip.so, built in-tree by opendressi_amd.build). Importing the
package loads the library and fails loudly when it is missing.
"""
from ._lib import DressiError, EXPORTED, LIB_PATH
from .runtime import (Context, icosphere, look_at, mat4_mul, perspective_vk, randn,
                      vertex_faces_tex)
from .silhouette import WORKLOADS, SilhouetteFit, Workload, camera_mvps, make_scene

__all__ = ["DressiError", "EXPORTED", "LIB_PATH", "Context", "icosphere", "look_at", "mat4_mul",
           "perspective_vk", "randn", "vertex_faces_tex", "WORKLOADS", "SilhouetteFit",
           "Workload", "camera_mvps", "make_scene"]
