"""Side table of producer metadata for tensors the surface returns
(python/dressi/torch/provenance.py:1-51).

nvdiffrast's signatures drop what the backward kernels need: `interpolate(attr,
rast, tri)` has no `pos`, yet its exact backward reads the corner clip
positions, and `texture(tex, uv)` has no mesh, yet its gradient gather
rasterizes the mesh in UV space. `rasterize` records its inputs against the
returned `rast`, `interpolate` records against its output; an entry lives as
long as the tensor object it describes.
"""
from __future__ import annotations

import weakref
from dataclasses import dataclass, field
from typing import Any

_table: dict[int, tuple[weakref.ref, Any]] = {}


@dataclass
class RastInfo:
    clip_vk: Any  # [N, V, 4] device clip positions, z remapped to [0, w]
    tri: Any  # the caller's [F, 3] int tensor
    resolution: tuple[int, int]  # (H, W)
    extra: dict = field(default_factory=dict)


@dataclass
class InterpInfo:
    attr: Any  # the vertex attribute tensor given to interpolate
    rast_info: RastInfo


def attach(tensor, info) -> None:
    key = id(tensor)

    def _drop(_ref, _key=key):
        _table.pop(_key, None)

    _table[key] = (weakref.ref(tensor, _drop), info)


def lookup(tensor, kind: str):
    entry = _table.get(id(tensor))
    if entry is None or entry[0]() is not tensor:
        raise RuntimeError(
            f"opendressi_amd.torch: this tensor has no {kind} provenance -- it must be "
            "produced by opendressi_amd.torch (`rast` from rasterize(), `uv` from "
            "interpolate()) within the same process.")
    return entry[1]
