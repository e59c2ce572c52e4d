"""Origin stamps on the tensors this surface returns.

nvdiffrast's signatures leave out what the backward passes need:
`interpolate(attr, rast, tri)` is not given `pos`, yet its exact backward
reads the corner clip positions; `texture(tex, uv)` is not given the mesh,
yet its gradient gather rasterizes that mesh in UV space. `rasterize`
therefore stamps the `rast` it returns with a `RasterOrigin`, and
`interpolate` stamps its output with an `InterpOrigin` that points back at
the raster it read.

A stamp is an attribute of the returned Python tensor object itself. It
lives exactly as long as that object, and every other tensor object -- a
clone, a view, a detached copy, anything computed from it -- has none, so
only the tensors this module handed out are accepted downstream. That is
the reference surface's rule (python/dressi/torch/provenance.py:1-51),
carried here without a side table.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any

_STAMP = "_opendressi_origin"


@dataclass(frozen=True)
class RasterOrigin:
    """What rasterize() saw: the device clip positions after the z remap
    ([N, V, 4]), the caller's triangle tensor, (H, W) and the context."""
    clip_vk: Any
    tri: Any
    resolution: tuple
    ctx: Any


@dataclass(frozen=True)
class InterpOrigin:
    """What interpolate() saw: the vertex attribute tensor and the raster
    whose pixels it was interpolated at."""
    attr: Any
    raster: RasterOrigin


def stamp(tensor, origin) -> None:
    """Record `origin` on `tensor` (the object returned to the caller)."""
    object.__setattr__(tensor, _STAMP, origin)


def origin(tensor, kind: type, producer: str):
    """The `kind` stamp of `tensor`; RuntimeError when it carries none
    (the tensor was not returned by `producer` of this module)."""
    rec = getattr(tensor, _STAMP, None) if tensor is not None else None
    if not isinstance(rec, kind):
        raise RuntimeError(
            f"opendressi_amd.torch: expected the tensor returned by {producer}() of this "
            f"module (found no {kind.__name__} on it; copies, views and results computed "
            "from it do not carry one)")
    return rec
