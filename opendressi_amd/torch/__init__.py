"""nvdiffrast-compatible PyTorch surface of the reference's `dressi.torch`
(python/dressi/torch/__init__.py), on ROCm device tensors.

    import opendressi_amd.torch as dr

    ctx = dr.RasterizeHipContext()
    rast, _ = dr.rasterize(ctx, pos, tri, resolution=[H, W])
    col, _  = dr.interpolate(attr, rast, tri)
    col     = dr.texture(tex, uv)
    col     = dr.antialias(col, rast, pos, tri)
    rs      = dr.rasterize_soft(ctx, pos, tri, [H, W], radius_px=3.0)

Coordinate conventions follow nvdiffrast (OpenGL clip space, z in [-w, w]);
the remap to the [0, w] depth range of the reference's rasterizers happens
inside. Every op runs the library's HIP kernels on the context's device,
ordered on torch's current stream; tensors already on that device are used
in place (no host round trip), others are moved there and the results are
returned on the input's device. `RasterizeVulkanContext` is kept as an alias
so reference code runs unchanged.
"""

from .context import RasterizeHipContext, RasterizeVulkanContext
from .ops import antialias, interpolate, rasterize, rasterize_soft, texture

__all__ = [
    "RasterizeHipContext",
    "RasterizeVulkanContext",
    "rasterize",
    "interpolate",
    "texture",
    "antialias",
    "rasterize_soft",
]
