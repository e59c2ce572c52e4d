"""Tensor-shape and clip-space conventions of the surface on device
tensors (the reference surface's conventions: python/dressi/torch/
convert.py:74-125)."""
from __future__ import annotations

import torch


def to_dev(t: torch.Tensor, device: torch.device, name: str) -> torch.Tensor:
    """`t` as a contiguous float32 tensor on `device` (no copy when it
    already is one)."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    return t.detach().to(device=device, dtype=torch.float32).contiguous()


def clip_gl_to_vk(pos: torch.Tensor) -> torch.Tensor:
    """OpenGL clip z in [-w, w] -> the rasterizers' z in [0, w]:
    z_vk = 0.5 * (z_gl + w); x, y, w unchanged (convert.py:93-100)."""
    out = pos.clone()
    out[..., 2] = 0.5 * (pos[..., 2] + pos[..., 3])
    return out


def clip_grad_vk_to_gl(g_vk: torch.Tensor) -> torch.Tensor:
    """Transpose of clip_gl_to_vk: dz_vk/dz_gl = 0.5, dz_vk/dw = 0.5
    (convert.py:103-109)."""
    out = g_vk.clone()
    out[..., 2] = 0.5 * g_vk[..., 2]
    out[..., 3] = g_vk[..., 3] + 0.5 * g_vk[..., 2]
    return out


def resolution_hw(resolution) -> tuple[int, int]:
    """(H, W) from an nvdiffrast `resolution` argument, which must name
    exactly two positive sizes."""
    try:
        dims = [int(x) for x in resolution]
    except (TypeError, ValueError):
        dims = []
    if len(dims) != 2 or min(dims) < 1:
        raise ValueError(f"opendressi_amd.torch: resolution must be two positive sizes "
                         f"[H, W]; got {resolution!r}")
    return dims[0], dims[1]


def batched(t: torch.Tensor, item_rank: int, name: str, layout: str) -> torch.Tensor:
    """`t` with a leading batch axis. An item has `item_rank` dimensions
    (`layout` names them, e.g. "V, C"); a single item becomes a batch of
    one, a batch passes through unchanged."""
    if t.dim() == item_rank + 1:
        return t
    if t.dim() == item_rank:
        return t.unsqueeze(0)
    raise ValueError(f"opendressi_amd.torch: {name} has shape {tuple(t.shape)}; expected "
                     f"[{layout}] or [N, {layout}]")


def vertex_batch(t: torch.Tensor, name: str = "pos") -> torch.Tensor:
    """[N, V, C] from [V, C] or [N, V, C]."""
    return batched(t, 2, name, "V, C")


def image_batch(t: torch.Tensor, name: str) -> torch.Tensor:
    """[N, H, W, C] from [H, W, C] or [N, H, W, C]."""
    return batched(t, 3, name, "H, W, C")


def channels(c: int, what: str) -> int:
    if not 1 <= c <= 4:
        raise ValueError(f"opendressi_amd.torch: {what} must have 1..4 channels, got {c}")
    return c


def sum_contribs(contribs: list[torch.Tensor]) -> torch.Tensor:
    """Sum gradient contributions as the reference's backward builder does
    (src/core/build_backward.cpp:36-57): groups of at most four, each summed
    left to right, level by level. Contributions come in descending order of
    their producing node's creation."""
    while len(contribs) > 1:
        nxt = []
        for i in range(0, len(contribs), 4):
            chunk = contribs[i:i + 4]
            acc = chunk[0]
            for c in chunk[1:]:
                acc = acc + c
            nxt.append(acc)
        contribs = nxt
    return contribs[0]
