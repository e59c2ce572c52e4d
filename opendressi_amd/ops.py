"""Per-op entry points on PyTorch-ROCm device tensors (zero copy).

Each function mirrors one reference op (src/core/f_ops.cpp) with the
reference's logical layouts: {N,1} arrays as (N, C) float32 tensors, faces as
float ids, screen images as (H, W[, C]). Inputs must be contiguous float32
tensors on the context's device; the work is ordered on torch's current
stream. PyTorch is only the memory/stream provider here.
"""
from __future__ import annotations

import ctypes as C

import torch

from ._lib import check, lib
from .runtime import Context


def _ptr(t: torch.Tensor | None, name: str) -> C.c_void_p:
    if t is None:
        return C.c_void_p(0)
    if t.dtype != torch.float32 or not t.is_contiguous() or t.device.type != "cuda":
        raise ValueError(f"{name}: expected a contiguous float32 device tensor, got "
                         f"{t.dtype} {tuple(t.shape)} on {t.device}")
    return C.c_void_p(t.data_ptr())


def _prep(ctx: Context) -> None:
    ctx.use_torch_stream()


def soft_clip(ctx: Context, clip: torch.Tensor, faces: torch.Tensor, width: int, height: int,
              radius_px: float) -> torch.Tensor:
    """F::SoftClip (src/core/f_ops.cpp:1890-1981) -> (3F, 4)."""
    _prep(ctx)
    out = torch.empty((faces.shape[0] * 3, 4), dtype=torch.float32, device=clip.device)
    check(lib.dressi_soft_clip(ctx.handle, _ptr(clip, "clip"), clip.shape[0],
                               _ptr(faces, "faces"), faces.shape[0], width, height,
                               float(radius_px), _ptr(out, "out")))
    return out


def rasterize_soft(ctx: Context, soft_clip: torch.Tensor, face_id: torch.Tensor,
                   faces_soft: torch.Tensor, hard_clip: torch.Tensor, faces_tex: torch.Tensor,
                   width: int, height: int, radius_px: float,
                   prev_shifted_depth: torch.Tensor | None = None) -> torch.Tensor:
    """F::RasterizeSoft (src/core/f_ops.cpp:1362-1465) -> (H, W, 4) =
    (signed_dist_px, face_id, hard_z, coverage)."""
    _prep(ctx)
    out = torch.empty((height, width, 4), dtype=torch.float32, device=soft_clip.device)
    check(lib.dressi_rasterize_soft(
        ctx.handle, _ptr(soft_clip, "soft_clip"), _ptr(face_id, "face_id"),
        _ptr(faces_soft, "faces_soft"), _ptr(hard_clip, "hard_clip"), hard_clip.shape[0],
        _ptr(faces_tex, "faces_tex"), faces_tex.shape[0], width, height, float(radius_px),
        _ptr(prev_shifted_depth, "prev_shifted_depth"), _ptr(out, "out")))
    return out


def rasterize(ctx: Context, clip: torch.Tensor, attr: torch.Tensor, faces: torch.Tensor,
              width: int, height: int) -> torch.Tensor:
    """F::Rasterize (src/core/f_ops.cpp:1182-1207) -> (H, W, C)."""
    _prep(ctx)
    attr2 = attr if attr.dim() == 2 else attr.reshape(-1, 1)
    nc = attr2.shape[1]
    out = torch.empty((height, width, nc), dtype=torch.float32, device=clip.device)
    check(lib.dressi_rasterize(ctx.handle, _ptr(clip, "clip"), clip.shape[0], _ptr(attr2, "attr"),
                               nc, _ptr(faces, "faces"), faces.shape[0], width, height,
                               _ptr(out, "out")))
    return out


def rasterize_face_id(ctx: Context, clip: torch.Tensor, faces: torch.Tensor, width: int,
                      height: int) -> torch.Tensor:
    """F::RasterizeFaceId (src/core/f_ops.cpp:2183-2209) -> (H, W)."""
    _prep(ctx)
    out = torch.empty((height, width), dtype=torch.float32, device=clip.device)
    check(lib.dressi_rasterize_face_id(ctx.handle, _ptr(clip, "clip"), clip.shape[0],
                                       _ptr(faces, "faces"), faces.shape[0], width, height,
                                       _ptr(out, "out")))
    return out


def rasterize_batch(ctx: Context, clip: torch.Tensor, attr: torch.Tensor, faces: torch.Tensor,
                    width: int, height: int, with_face_id: bool = False):
    """dressi_rasterize_batch: clip (N, V, 4), attr (V, C) shared or (N, V, C)
    per item -> (N, H, W, C) and, with `with_face_id`, the (N, H, W) face
    ids from the same pass (each item as rasterize / rasterize_face_id)."""
    _prep(ctx)
    n, nv = clip.shape[0], clip.shape[1]
    per_item = attr.dim() == 3
    nc = attr.shape[-1]
    out = torch.empty((n, height, width, nc), dtype=torch.float32, device=clip.device)
    ids = (torch.empty((n, height, width), dtype=torch.float32, device=clip.device)
           if with_face_id else None)
    check(lib.dressi_rasterize_batch(ctx.handle, _ptr(clip, "clip"), nv, n, _ptr(attr, "attr"),
                                     nc, 1 if per_item else 0, _ptr(faces, "faces"),
                                     faces.shape[0], width, height, _ptr(out, "out"),
                                     _ptr(ids, "face_id")))
    return (out, ids) if with_face_id else out


def lookup_faces(ctx: Context, attr: torch.Tensor, faces: torch.Tensor, corner: int) -> torch.Tensor:
    """F::LookupFaces (src/core/f_ops.cpp:1568-1619) -> (F, C)."""
    _prep(ctx)
    out = torch.empty((faces.shape[0], attr.shape[1]), dtype=torch.float32, device=attr.device)
    check(lib.dressi_lookup_faces(ctx.handle, _ptr(attr, "attr"), attr.shape[1], attr.shape[0],
                                  _ptr(faces, "faces"), faces.shape[0], corner, _ptr(out, "out")))
    return out


def lookup_faces_bwd(ctx: Context, gy: torch.Tensor, faces: torch.Tensor,
                     vtx_faces: torch.Tensor, corner: int) -> torch.Tensor:
    """LookupFacesBwd (src/core/f_ops.cpp:1521-1565) -> (V, C)."""
    _prep(ctx)
    deg, nv = vtx_faces.shape
    out = torch.empty((nv, gy.shape[1]), dtype=torch.float32, device=gy.device)
    check(lib.dressi_lookup_faces_bwd(ctx.handle, _ptr(gy, "gy"), gy.shape[1], _ptr(faces, "faces"),
                                      faces.shape[0], _ptr(vtx_faces, "vtx_faces"), nv, deg,
                                      corner, _ptr(out, "out")))
    return out


def face_fetch(ctx: Context, attr: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """F::FaceFetch forward (src/core/f_ops.cpp:1736-1799) -> (H, W, C)."""
    _prep(ctx)
    h, w = idx.shape
    out = torch.empty((h, w, attr.shape[1]), dtype=torch.float32, device=attr.device)
    check(lib.dressi_face_fetch(ctx.handle, _ptr(attr, "attr"), attr.shape[1], attr.shape[0],
                                _ptr(idx, "idx"), w, h, _ptr(out, "out")))
    return out


def face_fetch_bwd(ctx: Context, gy: torch.Tensor, idx: torch.Tensor, prj0: torch.Tensor,
                   prj1: torch.Tensor, prj2: torch.Tensor, seed: torch.Tensor, radius_px: float,
                   n_samples: int) -> torch.Tensor:
    """FaceFetchBwd (src/core/f_ops.cpp:1631-1733) -> (F, C); `seed` is a
    1-element device tensor (the in-graph iteration counter)."""
    _prep(ctx)
    h, w = idx.shape
    nc = gy.shape[-1]
    out = torch.empty((prj0.shape[0], nc), dtype=torch.float32, device=gy.device)
    check(lib.dressi_face_fetch_bwd(ctx.handle, _ptr(gy, "gy"), nc, _ptr(idx, "idx"), w, h,
                                    _ptr(prj0, "prj0"), _ptr(prj1, "prj1"), _ptr(prj2, "prj2"),
                                    prj0.shape[0], _ptr(seed, "seed"), float(radius_px), n_samples,
                                    _ptr(out, "out")))
    return out


def _nc(img: torch.Tensor) -> int:
    return 1 if img.dim() == 2 else img.shape[2]


def antialias(ctx: Context, img: torch.Tensor, tri: torch.Tensor, clip: torch.Tensor,
              faces: torch.Tensor) -> torch.Tensor:
    """F::AntiAlias forward (src/core/f_ops.cpp:2480-2579): img (H, W[, C]),
    tri (H, W) float face + 1, clip (V, 4), faces (F, 3) float ids."""
    _prep(ctx)
    h, w = tri.shape
    out = torch.empty_like(img)
    check(lib.dressi_antialias(ctx.handle, _ptr(img, "img"), _nc(img), _ptr(tri, "tri"),
                               _ptr(clip, "clip"), clip.shape[0], _ptr(faces, "faces"),
                               faces.shape[0], w, h, _ptr(out, "out")))
    return out


def antialias_bwd_img(ctx: Context, gy: torch.Tensor, tri: torch.Tensor, clip: torch.Tensor,
                      faces: torch.Tensor) -> torch.Tensor:
    """AntiAliasBwdImg (src/core/f_ops.cpp:2220-2278) -> like gy."""
    _prep(ctx)
    h, w = tri.shape
    out = torch.empty_like(gy)
    check(lib.dressi_antialias_bwd_img(ctx.handle, _ptr(gy, "gy"), _nc(gy), _ptr(tri, "tri"),
                                       _ptr(clip, "clip"), clip.shape[0], _ptr(faces, "faces"),
                                       faces.shape[0], w, h, _ptr(out, "out")))
    return out


def antialias_bwd_vtx(ctx: Context, gy: torch.Tensor, img: torch.Tensor, tri: torch.Tensor,
                      clip: torch.Tensor, faces: torch.Tensor, vtx_faces: torch.Tensor,
                      seed: torch.Tensor | None, n_samples: int, wide: bool = True) -> torch.Tensor:
    """AntiAliasBwdVtx (src/core/f_ops.cpp:2284-2476): n_samples > 0 and wide
    -> (deg, V, 4) partials; otherwise (V, 4). `seed` is a 1-element device
    tensor (the in-graph counter), unused when n_samples == 0."""
    _prep(ctx)
    h, w = tri.shape
    deg, nv = vtx_faces.shape
    is_wide = bool(wide and n_samples > 0)
    out = torch.empty((deg if is_wide else 1, nv, 4), dtype=torch.float32, device=gy.device)
    check(lib.dressi_antialias_bwd_vtx(
        ctx.handle, _ptr(gy, "gy"), _ptr(img, "img"), _nc(gy), _ptr(tri, "tri"),
        _ptr(clip, "clip"), nv, _ptr(faces, "faces"), faces.shape[0],
        _ptr(vtx_faces, "vtx_faces"), deg, _ptr(seed, "seed"), n_samples, 1 if is_wide else 0,
        w, h, _ptr(out, "out")))
    return out if is_wide else out[0]


def col_sum(ctx: Context, x: torch.Tensor) -> torch.Tensor:
    """F::ColSum (src/core/f_ops.cpp:1218-1246): (H, W, C) -> (W, C)."""
    _prep(ctx)
    h, w, nc = x.shape
    out = torch.empty((w, nc), dtype=torch.float32, device=x.device)
    check(lib.dressi_col_sum(ctx.handle, _ptr(x, "x"), nc, w, h, _ptr(out, "out")))
    return out


def _batch_clip(clip: torch.Tensor, n: int) -> tuple[int, int]:
    """(n_verts, clip_per_item) of a (V, 4) shared or (N, V, 4) clip."""
    if clip.dim() == 3:
        if clip.shape[0] != n:
            raise ValueError(f"clip: {clip.shape[0]} items for a batch of {n}")
        return clip.shape[1], 1
    return clip.shape[0], 0


def antialias_batch(ctx: Context, img: torch.Tensor, tri: torch.Tensor, clip: torch.Tensor,
                    faces: torch.Tensor) -> torch.Tensor:
    """dressi_antialias_batch: img (N, H, W, C), tri (N, H, W), clip (V, 4)
    shared or (N, V, 4) -> (N, H, W, C); each item as antialias()."""
    _prep(ctx)
    n, h, w, nc = img.shape
    nv, per_item = _batch_clip(clip, n)
    out = torch.empty_like(img)
    check(lib.dressi_antialias_batch(ctx.handle, _ptr(img, "img"), nc, _ptr(tri, "tri"),
                                     _ptr(clip, "clip"), nv, per_item, _ptr(faces, "faces"),
                                     faces.shape[0], w, h, n, _ptr(out, "out")))
    return out


def antialias_bwd_img_batch(ctx: Context, gy: torch.Tensor, tri: torch.Tensor,
                            clip: torch.Tensor, faces: torch.Tensor) -> torch.Tensor:
    """dressi_antialias_bwd_img_batch: gy (N, H, W, C) -> like gy."""
    _prep(ctx)
    n, h, w, nc = gy.shape
    nv, per_item = _batch_clip(clip, n)
    out = torch.empty_like(gy)
    check(lib.dressi_antialias_bwd_img_batch(ctx.handle, _ptr(gy, "gy"), nc, _ptr(tri, "tri"),
                                             _ptr(clip, "clip"), nv, per_item,
                                             _ptr(faces, "faces"), faces.shape[0], w, h, n,
                                             _ptr(out, "out")))
    return out


def antialias_bwd_vtx_batch(ctx: Context, gy: torch.Tensor, img: torch.Tensor,
                            tri: torch.Tensor, clip: torch.Tensor, faces: torch.Tensor,
                            vtx_faces: torch.Tensor, seeds: torch.Tensor | None, n_samples: int,
                            wide: bool = True) -> torch.Tensor:
    """dressi_antialias_bwd_vtx_batch: gy, img (N, H, W, C), seeds (N,) ->
    (N, deg, V, 4) partials when n_samples > 0 and wide, else (N, V, 4)."""
    _prep(ctx)
    n, h, w, nc = gy.shape
    nv, per_item = _batch_clip(clip, n)
    deg = vtx_faces.shape[0]
    is_wide = bool(wide and n_samples > 0)
    out = torch.empty((n, deg if is_wide else 1, vtx_faces.shape[1], 4), dtype=torch.float32,
                      device=gy.device)
    check(lib.dressi_antialias_bwd_vtx_batch(
        ctx.handle, _ptr(gy, "gy"), _ptr(img, "img"), nc, _ptr(tri, "tri"), _ptr(clip, "clip"),
        nv, per_item, _ptr(faces, "faces"), faces.shape[0], _ptr(vtx_faces, "vtx_faces"), deg,
        _ptr(seeds, "seeds"), n_samples, 1 if is_wide else 0, w, h, n, _ptr(out, "out")))
    return out if is_wide else out[:, 0]


def lookup_faces_batch(ctx: Context, attr: torch.Tensor, faces: torch.Tensor, corner: int,
                       n_items: int) -> torch.Tensor:
    """dressi_lookup_faces_batch: attr (V, C) shared or (N, V, C) per item ->
    (N, F, C); each item as lookup_faces()."""
    _prep(ctx)
    per_item = attr.dim() == 3
    nv, nc = attr.shape[-2], attr.shape[-1]
    out = torch.empty((n_items, faces.shape[0], nc), dtype=torch.float32, device=attr.device)
    check(lib.dressi_lookup_faces_batch(ctx.handle, _ptr(attr, "attr"), nc, nv,
                                        1 if per_item else 0, _ptr(faces, "faces"),
                                        faces.shape[0], corner, n_items, _ptr(out, "out")))
    return out


def lookup_faces_bwd_batch(ctx: Context, gy: torch.Tensor, faces: torch.Tensor,
                           vtx_faces: torch.Tensor, corner: int) -> torch.Tensor:
    """dressi_lookup_faces_bwd_batch: gy (N, F, C) -> (N, V, C)."""
    _prep(ctx)
    n, nf, nc = gy.shape
    deg, nv = vtx_faces.shape
    out = torch.empty((n, nv, nc), dtype=torch.float32, device=gy.device)
    check(lib.dressi_lookup_faces_bwd_batch(ctx.handle, _ptr(gy, "gy"), nc, _ptr(faces, "faces"),
                                            faces.shape[0], _ptr(vtx_faces, "vtx_faces"), nv,
                                            deg, corner, n, _ptr(out, "out")))
    return out


def face_fetch_batch(ctx: Context, attr: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """dressi_face_fetch_batch: attr (F, C) shared or (N, F, C) per item, idx
    (N, H, W) -> (N, H, W, C)."""
    _prep(ctx)
    n, h, w = idx.shape
    per_item = attr.dim() == 3
    nf, nc = attr.shape[-2], attr.shape[-1]
    out = torch.empty((n, h, w, nc), dtype=torch.float32, device=attr.device)
    check(lib.dressi_face_fetch_batch(ctx.handle, _ptr(attr, "attr"), nc, nf,
                                      1 if per_item else 0, _ptr(idx, "idx"), w, h, n,
                                      _ptr(out, "out")))
    return out


def face_fetch_bwd_batch(ctx: Context, gy: torch.Tensor, idx: torch.Tensor, prj0: torch.Tensor,
                         prj1: torch.Tensor, prj2: torch.Tensor, seeds: torch.Tensor,
                         radius_px: float, n_samples: int) -> torch.Tensor:
    """dressi_face_fetch_bwd_batch: gy (N, H, W, C), idx (N, H, W), prj* (F, 4)
    shared or (N, F, 4), seeds (N,) -> (N, F, C)."""
    _prep(ctx)
    n, h, w, nc = gy.shape
    per_item = prj0.dim() == 3
    nf = prj0.shape[-2]
    out = torch.empty((n, nf, nc), dtype=torch.float32, device=gy.device)
    check(lib.dressi_face_fetch_bwd_batch(
        ctx.handle, _ptr(gy, "gy"), nc, _ptr(idx, "idx"), w, h, _ptr(prj0, "prj0"),
        _ptr(prj1, "prj1"), _ptr(prj2, "prj2"), 1 if per_item else 0, nf, _ptr(seeds, "seeds"),
        float(radius_px), n_samples, n, _ptr(out, "out")))
    return out


def col_sum_batch(ctx: Context, x: torch.Tensor) -> torch.Tensor:
    """dressi_col_sum_batch: (N, H, W, C) -> (N, W, C)."""
    _prep(ctx)
    n, h, w, nc = x.shape
    out = torch.empty((n, w, nc), dtype=torch.float32, device=x.device)
    check(lib.dressi_col_sum_batch(ctx.handle, _ptr(x, "x"), nc, w, h, n, _ptr(out, "out")))
    return out


__all__ = ["soft_clip", "rasterize_soft", "rasterize", "rasterize_face_id", "lookup_faces",
           "lookup_faces_bwd", "face_fetch", "face_fetch_bwd", "antialias", "antialias_bwd_img",
           "antialias_bwd_vtx", "col_sum", "rasterize_batch", "antialias_batch",
           "antialias_bwd_img_batch", "antialias_bwd_vtx_batch", "col_sum_batch",
           "lookup_faces_batch", "lookup_faces_bwd_batch", "face_fetch_batch",
           "face_fetch_bwd_batch"]


def texture_bilinear(ctx: Context, tex: torch.Tensor, uv: torch.Tensor) -> torch.Tensor:
    """F::TextureBilinear forward (src/core/f_ops.cpp:2736-2780): tex (TH, TW,
    C), uv (H, W, 2) -> (H, W, C)."""
    _prep(ctx)
    th, tw, nc = tex.shape
    uh, uw = uv.shape[:2]
    out = torch.empty((uh, uw, nc), dtype=torch.float32, device=uv.device)
    check(lib.dressi_texture_bilinear(ctx.handle, _ptr(tex, "tex"), tw, th, nc, _ptr(uv, "uv"),
                                      uw, uh, _ptr(out, "out")))
    return out


def texture_bilinear_bwd(ctx: Context, gy: torch.Tensor, inv_uv: torch.Tensor,
                         uv: torch.Tensor) -> torch.Tensor:
    """GatherByInverseUVBilinear (src/core/f_ops.cpp:2650-2732): gy (H, W, C),
    inv_uv (TH, TW, 4), uv (H, W, 2) -> d/d tex (TH, TW, C)."""
    _prep(ctx)
    sh, sw, nc = gy.shape
    th, tw = inv_uv.shape[:2]
    out = torch.empty((th, tw, nc), dtype=torch.float32, device=gy.device)
    check(lib.dressi_texture_bilinear_bwd(ctx.handle, _ptr(gy, "gy"), nc, sw, sh,
                                          _ptr(inv_uv, "inv_uv"), tw, th, _ptr(uv, "uv"),
                                          _ptr(out, "out")))
    return out


def texture_nearest(ctx: Context, tex: torch.Tensor, uv: torch.Tensor) -> torch.Tensor:
    """F::Texture forward (src/core/f_ops.cpp:2605-2639; nearest, clamp to
    edge): tex (TH, TW, C), uv (H, W, 2) -> (H, W, C)."""
    _prep(ctx)
    th, tw, nc = tex.shape
    uh, uw = uv.shape[:2]
    out = torch.empty((uh, uw, nc), dtype=torch.float32, device=uv.device)
    check(lib.dressi_texture_nearest(ctx.handle, _ptr(tex, "tex"), tw, th, nc, _ptr(uv, "uv"),
                                     uw, uh, _ptr(out, "out")))
    return out


def texture_nearest_bwd(ctx: Context, gy: torch.Tensor, inv_uv: torch.Tensor,
                        uv: torch.Tensor) -> torch.Tensor:
    """GatherByInverseUV (src/core/f_ops.cpp:2586-2601): gy (H, W, C), inv_uv
    (TH, TW, 4), uv (H, W, 2) -> d/d tex (TH, TW, C)."""
    _prep(ctx)
    sh, sw, nc = gy.shape
    th, tw = inv_uv.shape[:2]
    out = torch.empty((th, tw, nc), dtype=torch.float32, device=gy.device)
    check(lib.dressi_texture_nearest_bwd(ctx.handle, _ptr(gy, "gy"), nc, sw, sh,
                                         _ptr(inv_uv, "inv_uv"), tw, th, _ptr(uv, "uv"),
                                         _ptr(out, "out")))
    return out


def screen_attr(ctx: Context, clip: torch.Tensor, width: int, height: int) -> torch.Tensor:
    """ScreenAttr (src/core/mesh_utils.cpp:191-203): clip (V, 4) -> (V, 4)."""
    _prep(ctx)
    out = torch.empty_like(clip)
    check(lib.dressi_screen_attr(ctx.handle, _ptr(clip, "clip"), clip.shape[0], width, height,
                                 _ptr(out, "out")))
    return out


def gather_dist_grad(ctx: Context, gy: torch.Tensor, rs: torch.Tensor, clip: torch.Tensor,
                     faces: torch.Tensor, vtx_faces: torch.Tensor, radius_px: float = 3.0,
                     wide: bool = True) -> torch.Tensor:
    """GatherDistGrad (src/core/f_ops.cpp:1248-1358): gy, rs (H, W, 4), clip
    (V, 4), faces (F, 3) float ids, vtx_faces (deg, V) -> (deg, V, 4) when
    wide, else (V, 4)."""
    _prep(ctx)
    h, w = rs.shape[:2]
    deg, nv = vtx_faces.shape
    out = torch.empty((deg if wide else 1, nv, 4), dtype=torch.float32, device=rs.device)
    check(lib.dressi_gather_dist_grad(ctx.handle, _ptr(gy, "gy"), _ptr(rs, "rs"),
                                      _ptr(clip, "clip"), nv, _ptr(faces, "faces"),
                                      faces.shape[0], _ptr(vtx_faces, "vtx_faces"), deg,
                                      radius_px, 1 if wide else 0, w, h, _ptr(out, "out")))
    return out if wide else out[0]


# ---- split-sum IBL ops (maps are (H, W, C) equirect images) ----------------

def _map_nc(m: torch.Tensor) -> int:
    return 1 if m.dim() == 2 else m.shape[2]


def equirect_sample(ctx: Context, map_: torch.Tensor, dirs: torch.Tensor) -> torch.Tensor:
    """F::EquirectSample (src/core/f_ops.cpp:2921-2964): map (mh, mw, C) at
    dirs (H, W, 3) -> (H, W, C)."""
    _prep(ctx)
    mh, mw, nc = map_.shape[0], map_.shape[1], _map_nc(map_)
    h, w = dirs.shape[0], dirs.shape[1]
    out = torch.empty((h, w, nc), dtype=torch.float32, device=map_.device)
    check(lib.dressi_equirect_sample(ctx.handle, _ptr(map_, "map"), mw, mh, nc,
                                     _ptr(dirs, "dirs"), w, h, _ptr(out, "out")))
    return out


def equirect_sample_bwd(ctx: Context, gy: torch.Tensor, dirs: torch.Tensor, mw: int,
                        mh: int) -> torch.Tensor:
    """EquirectSample's VJP w.r.t. the map (f_ops.cpp:2786-2919) -> (mh, mw, C)."""
    _prep(ctx)
    nc = _map_nc(gy)
    h, w = dirs.shape[0], dirs.shape[1]
    out = torch.empty((mh, mw, nc), dtype=torch.float32, device=gy.device)
    check(lib.dressi_equirect_sample_bwd(ctx.handle, _ptr(gy, "gy"), nc, _ptr(dirs, "dirs"), w,
                                         h, mw, mh, _ptr(out, "out")))
    return out


def avg_pool2x2(ctx: Context, x: torch.Tensor) -> torch.Tensor:
    """F::AvgPool2x2 (f_ops.cpp:3411-3415): (h, w, C) -> (ceil(h/2), ceil(w/2), C)."""
    _prep(ctx)
    h, w, nc = x.shape[0], x.shape[1], _map_nc(x)
    out = torch.empty(((h + 1) // 2, (w + 1) // 2, nc), dtype=torch.float32, device=x.device)
    check(lib.dressi_avg_pool2x2(ctx.handle, _ptr(x, "x"), w, h, nc, _ptr(out, "out")))
    return out


def avg_pool2x2_bwd(ctx: Context, gy: torch.Tensor, w: int, h: int) -> torch.Tensor:
    """AvgPool2x2's VJP (UpsampleNearest2x of gy * 0.25) -> (h, w, C)."""
    _prep(ctx)
    nc = _map_nc(gy)
    out = torch.empty((h, w, nc), dtype=torch.float32, device=gy.device)
    check(lib.dressi_avg_pool2x2_bwd(ctx.handle, _ptr(gy, "gy"), w, h, nc, _ptr(out, "out")))
    return out


def irradiance_conv(ctx: Context, env: torch.Tensor, ow: int, oh: int) -> torch.Tensor:
    """F::IrradianceConv (f_ops.cpp:3006-3087) -> (oh, ow, C)."""
    _prep(ctx)
    sh, sw, nc = env.shape[0], env.shape[1], _map_nc(env)
    out = torch.empty((oh, ow, nc), dtype=torch.float32, device=env.device)
    check(lib.dressi_irradiance_conv(ctx.handle, _ptr(env, "env"), sw, sh, nc, ow, oh,
                                     _ptr(out, "out")))
    return out


def irradiance_conv_bwd(ctx: Context, gy: torch.Tensor, sw: int, sh: int) -> torch.Tensor:
    """IrradianceConvBwd (f_ops.cpp:2970-3004): gy (oh, ow, C) -> (sh, sw, C)."""
    _prep(ctx)
    oh, ow, nc = gy.shape[0], gy.shape[1], _map_nc(gy)
    out = torch.empty((sh, sw, nc), dtype=torch.float32, device=gy.device)
    check(lib.dressi_irradiance_conv_bwd(ctx.handle, _ptr(gy, "gy"), ow, oh, nc, sw, sh,
                                         _ptr(out, "out")))
    return out


def prefilter_conv_norm(ctx: Context, ow: int, oh: int, sw: int, sh: int, roughness: float,
                        device=None) -> torch.Tensor:
    """PrefilterConvNorm (f_ops.cpp:3166-3205) -> (oh, ow)."""
    _prep(ctx)
    out = torch.empty((oh, ow), dtype=torch.float32, device=device or f"cuda:{ctx.device}")
    check(lib.dressi_prefilter_conv_norm(ctx.handle, ow, oh, sw, sh, float(roughness),
                                         _ptr(out, "norm")))
    return out


def prefilter_conv(ctx: Context, env: torch.Tensor, ow: int, oh: int, roughness: float,
                   norm: torch.Tensor | None = None) -> torch.Tensor:
    """F::PrefilterConv (f_ops.cpp:3264-3348) -> (oh, ow, C); `norm` from
    prefilter_conv_norm (computed when None)."""
    sh, sw, nc = env.shape[0], env.shape[1], _map_nc(env)
    if norm is None:
        norm = prefilter_conv_norm(ctx, ow, oh, sw, sh, roughness, env.device)
    _prep(ctx)
    out = torch.empty((oh, ow, nc), dtype=torch.float32, device=env.device)
    check(lib.dressi_prefilter_conv(ctx.handle, _ptr(env, "env"), sw, sh, nc, ow, oh,
                                    float(roughness), _ptr(norm, "norm"), _ptr(out, "out")))
    return out


def prefilter_conv_bwd(ctx: Context, gy: torch.Tensor, sw: int, sh: int, roughness: float,
                       norm: torch.Tensor | None = None) -> torch.Tensor:
    """PrefilterConvBwd (f_ops.cpp:3207-3262): gy (oh, ow, C) -> (sh, sw, C)."""
    oh, ow, nc = gy.shape[0], gy.shape[1], _map_nc(gy)
    if norm is None:
        norm = prefilter_conv_norm(ctx, ow, oh, sw, sh, roughness, gy.device)
    _prep(ctx)
    out = torch.empty((sh, sw, nc), dtype=torch.float32, device=gy.device)
    check(lib.dressi_prefilter_conv_bwd(ctx.handle, _ptr(gy, "gy"), ow, oh, nc, sw, sh,
                                        float(roughness), _ptr(norm, "norm"), _ptr(out, "out")))
    return out


def prefilter_env(ctx: Context, env: torch.Tensor, ow: int, oh: int, roughness: float,
                  n_samples: int = 256) -> torch.Tensor:
    """F::PrefilterEnv (f_ops.cpp:3089-3157) -> (oh, ow, C)."""
    _prep(ctx)
    sh, sw, nc = env.shape[0], env.shape[1], _map_nc(env)
    out = torch.empty((oh, ow, nc), dtype=torch.float32, device=env.device)
    check(lib.dressi_prefilter_env(ctx.handle, _ptr(env, "env"), sw, sh, nc, ow, oh,
                                   float(roughness), n_samples, _ptr(out, "out")))
    return out


def brdf_lut(ctx: Context, w: int = 256, h: int = 256, n_samples: int = 512,
             device=None) -> torch.Tensor:
    """F::BrdfIntegrationLut (f_ops.cpp:3350-3409) -> (h, w, 2)."""
    _prep(ctx)
    out = torch.empty((h, w, 2), dtype=torch.float32, device=device or f"cuda:{ctx.device}")
    check(lib.dressi_brdf_lut(ctx.handle, w, h, n_samples, _ptr(out, "out")))
    return out
