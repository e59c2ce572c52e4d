"""ctypes binding of the C ABI in include/dressi_hip.h (libdressi_hip.so).

The library must be built in-tree (opendressi_amd.build / __graft_entry__.build);
importing this module without it raises immediately -- there is no fallback.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdressi_hip.so")

_P = C.c_void_p
_F = C.c_float
_U = C.c_uint32
_I = C.c_int
_S = C.c_size_t
_FP = C.POINTER(C.c_float)
_UP = C.POINTER(C.c_uint32)


class DressiError(RuntimeError):
    """Raised for every non-zero status of the C ABI (the reference raises
    DressiError "msg (file:line)", include/dressi/types.h:110-123)."""


class HsrDesc(C.Structure):
    _fields_ = [("n_verts", _U), ("n_faces", _U), ("n_views", _U), ("width", _U),
                ("height", _U), ("radius_px", _F), ("n_samples", _U), ("lr", _F),
                ("beta1", _F), ("beta2", _F), ("eps", _F), ("flags", _U)]


class TexDesc(C.Structure):
    _fields_ = [("n_verts", _U), ("n_faces", _U), ("n_views", _U), ("width", _U),
                ("height", _U), ("tex_w", _U), ("tex_h", _U), ("n_sets", _U), ("lr", _F),
                ("beta1", _F), ("beta2", _F), ("eps", _F), ("flags", _U)]


class PbrDesc(C.Structure):
    _fields_ = [("n_verts", _U), ("n_faces", _U), ("n_views", _U), ("width", _U),
                ("height", _U), ("tex_w", _U), ("tex_h", _U), ("env_w", _U), ("env_h", _U),
                ("levels", _U), ("lr", _F), ("beta1", _F), ("beta2", _F), ("eps", _F),
                ("flags", _U)]


PBR_KEEP_PRED = 1
PBR_KEEP_GRAD = 2
(PBR_LOSS, PBR_PRED, PBR_TARGET, PBR_G_ALBEDO, PBR_G_MR, PBR_G_ENV, PBR_IRR,
 PBR_PREF, PBR_GBUF0) = range(9)

TEX_KEEP_IMAGES = 1
TEX_KEEP_GRAD = 2
TEX_EXTERNAL_CLIP = 4
(TEX_LOSS, TEX_PRED, TEX_TARGET, TEX_FACE_ID, TEX_GRAD, TEX_TEX, TEX_UV) = range(7)

HSR_KEEP_PRED = 1
HSR_KEEP_GRAD = 2
HSR_TECHNIQUE_AA = 4
BUF_LOSS, BUF_PRED, BUF_TARGET, BUF_FACE_ID, BUF_GRAD, BUF_POS = range(6)
FACE_ID_RIM = 0x80000000  # bit of a face-id entry: winner outside its hard triangle

# name -> (restype, argtypes)
_SIGS = {
    "dressi_last_error": (C.c_char_p, []),
    "dressi_version": (C.c_char_p, []),
    "dressi_ctx_create": (_I, [_I, C.POINTER(_P)]),
    "dressi_ctx_destroy": (_I, [_P]),
    "dressi_ctx_set_stream": (_I, [_P, _P]),
    "dressi_ctx_reset_stream": (_I, [_P]),
    "dressi_ctx_stream": (_P, [_P]),
    "dressi_ctx_workspace_generation": (C.c_uint64, [_P]),
    "dressi_ctx_synchronize": (_I, [_P]),
    "dressi_ctx_device_name": (_I, [_P, C.c_char_p, _S]),
    "dressi_malloc": (_I, [_P, C.POINTER(_P), _S]),
    "dressi_free": (_I, [_P, _P]),
    "dressi_memcpy_h2d": (_I, [_P, _P, _P, _S]),
    "dressi_memcpy_d2h": (_I, [_P, _P, _P, _S]),
    "dressi_memset": (_I, [_P, _P, _I, _S]),
    "dressi_soft_clip": (_I, [_P, _P, _U, _P, _U, _U, _U, _F, _P]),
    "dressi_rasterize_soft": (_I, [_P, _P, _P, _P, _P, _U, _P, _U, _U, _U, _F, _P, _P]),
    "dressi_rasterize_soft_noalloc": (_I, [_P, _P, _P, _P, _P, _U, _P, _U, _U, _U, _F, _P, _P]),
    "dressi_rasterize": (_I, [_P, _P, _U, _P, _U, _P, _U, _U, _U, _P]),
    "dressi_rasterize_face_id": (_I, [_P, _P, _U, _P, _U, _U, _U, _P]),
    "dressi_rasterize_batch": (_I, [_P, _P, _U, _U, _P, _U, _I, _P, _U, _U, _U, _P, _P]),
    "dressi_lookup_faces": (_I, [_P, _P, _U, _U, _P, _U, _U, _P]),
    "dressi_lookup_faces_bwd": (_I, [_P, _P, _U, _P, _U, _P, _U, _U, _U, _P]),
    "dressi_face_fetch": (_I, [_P, _P, _U, _U, _P, _U, _U, _P]),
    "dressi_face_fetch_bwd": (_I, [_P, _P, _U, _P, _U, _U, _P, _P, _P, _U, _P, _F, _U, _P]),
    "dressi_lookup_faces_batch": (_I, [_P, _P, _U, _U, _I, _P, _U, _U, _U, _P]),
    "dressi_lookup_faces_bwd_batch": (_I, [_P, _P, _U, _P, _U, _P, _U, _U, _U, _U, _P]),
    "dressi_face_fetch_batch": (_I, [_P, _P, _U, _U, _I, _P, _U, _U, _U, _P]),
    "dressi_face_fetch_bwd_batch": (_I, [_P, _P, _U, _P, _U, _U, _P, _P, _P, _I, _U, _P, _F, _U,
                                         _U, _P]),
    "dressi_antialias": (_I, [_P, _P, _U, _P, _P, _U, _P, _U, _U, _U, _P]),
    "dressi_antialias_bwd_img": (_I, [_P, _P, _U, _P, _P, _U, _P, _U, _U, _U, _P]),
    "dressi_antialias_bwd_vtx": (_I, [_P, _P, _P, _U, _P, _P, _U, _P, _U, _P, _U, _P, _U, _I,
                                      _U, _U, _P]),
    "dressi_col_sum": (_I, [_P, _P, _U, _U, _U, _P]),
    "dressi_antialias_batch": (_I, [_P, _P, _U, _P, _P, _U, _I, _P, _U, _U, _U, _U, _P]),
    "dressi_antialias_bwd_img_batch": (_I, [_P, _P, _U, _P, _P, _U, _I, _P, _U, _U, _U, _U, _P]),
    "dressi_antialias_bwd_vtx_batch": (_I, [_P, _P, _P, _U, _P, _P, _U, _I, _P, _U, _P, _U, _P, _U,
                                            _I, _U, _U, _U, _P]),
    "dressi_col_sum_batch": (_I, [_P, _P, _U, _U, _U, _U, _P]),
    "dressi_gather_dist_grad": (_I, [_P, _P, _P, _P, _U, _P, _U, _P, _U, _F, _I, _U, _U, _P]),
    "dressi_equirect_sample": (_I, [_P, _P, _U, _U, _U, _P, _U, _U, _P]),
    "dressi_equirect_sample_bwd": (_I, [_P, _P, _U, _P, _U, _U, _U, _U, _P]),
    "dressi_avg_pool2x2": (_I, [_P, _P, _U, _U, _U, _P]),
    "dressi_avg_pool2x2_bwd": (_I, [_P, _P, _U, _U, _U, _P]),
    "dressi_irradiance_conv": (_I, [_P, _P, _U, _U, _U, _U, _U, _P]),
    "dressi_irradiance_conv_bwd": (_I, [_P, _P, _U, _U, _U, _U, _U, _P]),
    "dressi_prefilter_conv_norm": (_I, [_P, _U, _U, _U, _U, _F, _P]),
    "dressi_prefilter_conv": (_I, [_P, _P, _U, _U, _U, _U, _U, _F, _P, _P]),
    "dressi_prefilter_conv_bwd": (_I, [_P, _P, _U, _U, _U, _U, _U, _F, _P, _P]),
    "dressi_prefilter_env": (_I, [_P, _P, _U, _U, _U, _U, _U, _F, _U, _P]),
    "dressi_brdf_lut": (_I, [_P, _U, _U, _U, _P]),
    "dressi_texture_bilinear": (_I, [_P, _P, _U, _U, _U, _P, _U, _U, _P]),
    "dressi_texture_bilinear_bwd": (_I, [_P, _P, _U, _U, _U, _P, _U, _U, _P, _P]),
    "dressi_texture_nearest": (_I, [_P, _P, _U, _U, _U, _P, _U, _U, _P]),
    "dressi_texture_nearest_bwd": (_I, [_P, _P, _U, _U, _U, _P, _U, _U, _P, _P]),
    "dressi_screen_attr": (_I, [_P, _P, _U, _U, _U, _P]),
    "dressi_uv_sphere": (_I, [_U, _U, _UP, _UP, _FP, _FP, _FP]),
    "dressi_uv_as_clip": (None, [_FP, _U, _FP]),
    "dressi_icosphere": (_I, [_U, _UP, _UP, _FP, _FP]),
    "dressi_vertex_faces_tex": (_I, [_FP, _U, _U, _UP, _FP, _S]),
    "dressi_look_at": (None, [_FP, _FP, _FP, _FP]),
    "dressi_perspective_vk": (None, [_F, _F, _F, _F, _FP]),
    "dressi_mat4_mul": (None, [_FP, _FP, _FP]),
    "dressi_expf": (_F, [_F]),
    "dressi_hsr_create": (_I, [_P, C.POINTER(HsrDesc), C.POINTER(_P)]),
    "dressi_hsr_destroy": (_I, [_P]),
    "dressi_hsr_set_mesh": (_I, [_P, _FP, _FP]),
    "dressi_hsr_set_targets": (_I, [_P, _FP]),
    "dressi_hsr_render_targets": (_I, [_P, _FP, _U, _FP, _U]),
    "dressi_hsr_set_state": (_I, [_P, _FP, _FP, _FP, _F]),
    "dressi_hsr_get_state": (_I, [_P, _FP, _FP, _FP, _FP]),
    "dressi_hsr_step": (_I, [_P, _U]),
    "dressi_hsr_step_eager": (_I, [_P, _U]),
    "dressi_hsr_buffer": (_I, [_P, _I, C.POINTER(_P), C.POINTER(_S)]),
    "dressi_hsr_read": (_I, [_P, _I, _P, _S]),
    "dressi_hsr_profile": (_I, [_P, _U, C.c_char_p, _S, _FP, _U, _UP]),
    "dressi_hsr_bin_capacity": (_I, [_P, _UP]),
    "dressi_pbr_create": (_I, [_P, C.POINTER(PbrDesc), C.POINTER(_P)]),
    "dressi_pbr_destroy": (_I, [_P]),
    "dressi_pbr_set_scene": (_I, [_P, _FP, _FP, _FP, _FP, _FP, _FP, _FP]),
    "dressi_pbr_set_scene_clips": (_I, [_P, _FP, _FP, _FP, _FP, _FP, _FP, _FP]),
    "dressi_pbr_set_adam": (_I, [_P, _FP, _FP, _FP, _FP, _FP, _FP]),
    "dressi_pbr_get_adam": (_I, [_P, _FP, _FP, _FP, _FP, _FP, _FP]),
    "dressi_pbr_set_target": (_I, [_P, _FP, _FP, _FP]),
    "dressi_pbr_set_state": (_I, [_P, _FP, _FP, _FP, _F]),
    "dressi_pbr_get_state": (_I, [_P, _FP, _FP, _FP, _FP]),
    "dressi_pbr_step": (_I, [_P, _U]),
    "dressi_pbr_step_eager": (_I, [_P, _U]),
    "dressi_pbr_buffer": (_I, [_P, _I, C.POINTER(_P), C.POINTER(_S)]),
    "dressi_pbr_read": (_I, [_P, _I, _P, _S]),
    "dressi_pbr_profile": (_I, [_P, _U, C.c_char_p, _S, _FP, _U, _UP]),
    "dressi_tex_create": (_I, [_P, C.POINTER(TexDesc), C.POINTER(_P)]),
    "dressi_tex_destroy": (_I, [_P]),
    "dressi_tex_set_mesh": (_I, [_P, _FP, _FP, _FP]),
    "dressi_tex_set_cameras": (_I, [_P, _FP]),
    "dressi_tex_set_clips": (_I, [_P, _FP, _FP]),
    "dressi_tex_set_target": (_I, [_P, _FP]),
    "dressi_tex_set_state": (_I, [_P, _FP, _FP, _FP, _F]),
    "dressi_tex_get_state": (_I, [_P, _FP, _FP, _FP, _FP]),
    "dressi_tex_step": (_I, [_P, _U]),
    "dressi_tex_step_eager": (_I, [_P, _U]),
    "dressi_tex_buffer": (_I, [_P, _I, C.POINTER(_P), C.POINTER(_S)]),
    "dressi_tex_read": (_I, [_P, _I, _P, _S]),
    "dressi_tex_profile": (_I, [_P, _U, C.c_char_p, _S, _FP, _U, _UP]),
}

EXPORTED = tuple(_SIGS)


def load(path: str = LIB_PATH) -> C.CDLL:
    if not os.path.exists(path):
        raise ImportError(
            f"{path} is missing: build the HIP library first "
            "(python -m opendressi_amd.build or __graft_entry__.build()); "
            "there is no CPU fallback")
    # PyTorch-ROCm bundles its own libamdhip64.so.7. Loading torch first makes
    # the library's libamdhip64.so.7 dependency resolve to that same runtime;
    # loading the library first would map a second HIP + HSA runtime into the
    # process and torch's device initialisation then fails.
    import torch  # noqa: F401
    lib = C.CDLL(path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = load()


def check(rc: int) -> None:
    if rc != 0:
        msg = lib.dressi_last_error()
        raise DressiError(f"dressi status {rc}: {msg.decode() if msg else ''}")
