"""RasterizeHipContext: one HIP device + per-topology and per-signature caches
(the reference's RasterizeVulkanContext, python/dressi/torch/context.py:13-52).
"""
from __future__ import annotations

import threading

import numpy as np
import torch

from ..runtime import Context, vertex_faces_tex


def tri_int32(tri: torch.Tensor) -> torch.Tensor:
    """[F, 3] int32/int64 -> contiguous int32 on the host
    (python/dressi/torch/convert.py:85-90)."""
    if tri.dim() != 2 or tri.shape[1] != 3:
        raise ValueError(f"tri must be [F, 3] int, got {tuple(tri.shape)}")
    if tri.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"tri must be int32/int64, got {tri.dtype}")
    return tri.detach().cpu().to(torch.int32).contiguous()


class MeshData:
    """Static-topology arrays of one triangle list, on the device
    (python/dressi/torch/meshdata.py:11-43): faces as float ids, the unweld
    gather index, sequential faces of the unwelded corners, the per-corner
    face id, the {max_deg, V} vertex -> face adjacency."""

    def __init__(self, tri: torch.Tensor, device: torch.device):
        # the source tensor is pinned: the cache key holds its data_ptr
        self.src = tri
        t = tri_int32(tri)
        self.n_faces = int(t.shape[0])
        self.n_verts = int(t.max().item()) + 1 if self.n_faces else 0
        faces_np = t.numpy().astype(np.float32)
        self.faces_f = torch.from_numpy(faces_np).to(device)
        self.unweld = t.reshape(-1).long().to(device)
        self.faces_seq = torch.arange(self.n_faces * 3, dtype=torch.float32).reshape(-1, 3).to(device)
        self.corner_face_id = torch.arange(self.n_faces, dtype=torch.float32).repeat_interleave(3).to(device)
        vft = vertex_faces_tex(faces_np, self.n_verts)
        self.vft = torch.from_numpy(vft).to(device)
        self.max_deg = int(vft.shape[0])


def mesh_key(tri: torch.Tensor) -> tuple:
    return (tri.data_ptr(), tri._version, tuple(tri.shape), str(tri.device))


class RasterizeHipContext:
    """MI355X counterpart of nvdiffrast's RasterizeGLContext and of the
    reference's RasterizeVulkanContext: one HIP device (`device`: index or
    torch device, default the current one) shared by every op. Per-signature
    constant buffers are cached in `_engines` (keyed by shape, as the
    reference keys its compiled graphs) and per-topology data in `_meshes`;
    `clear_cache()` frees both."""

    def __init__(self, device=None, debug: bool = False):
        del debug
        if device is None:
            device = torch.cuda.current_device()
        self.device = torch.device("cuda", torch.device(device).index
                                   if not isinstance(device, int) else device)
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self._ctx = Context(self.device.index)
        self._engines: dict[tuple, object] = {}
        self._meshes: dict[tuple, MeshData] = {}
        self.lock = threading.RLock()

    def engine(self, key: tuple, builder):
        """The cached object for `key`, built with `builder()` on first use."""
        with self.lock:
            eng = self._engines.get(key)
            if eng is None:
                eng = builder()
                self._engines[key] = eng
            return eng

    def mesh(self, tri: torch.Tensor) -> MeshData:
        key = mesh_key(tri)
        with self.lock:
            md = self._meshes.get(key)
            if md is None:
                md = MeshData(tri, self.device)
                self._meshes[key] = md
            return md

    def clear_cache(self) -> None:
        with self.lock:
            self._engines.clear()
            self._meshes.clear()


# the reference's name, so code written against dressi.torch runs unchanged
RasterizeVulkanContext = RasterizeHipContext
