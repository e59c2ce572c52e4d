"""Host-side logic of opendressi_amd.torch (no GPU): clip-space conventions,
the gradient-sum order, provenance lifetime, argument checks."""
import gc
import weakref

import numpy as np
import pytest
import torch

from opendressi_amd.torch import convert, provenance


def test_clip_grad_is_the_transpose_of_the_remap():
    """<remap(x), g> == <x, remap^T(g)> for random x, g (the remap is
    linear), and z_vk = 0.5 (z + w) on a known vertex."""
    rng = np.random.default_rng(0)
    x = torch.from_numpy(rng.standard_normal((5, 7, 4))).double()
    g = torch.from_numpy(rng.standard_normal((5, 7, 4))).double()
    lhs = (convert.clip_gl_to_vk(x) * g).sum()
    rhs = (x * convert.clip_grad_vk_to_gl(g)).sum()
    assert abs(lhs.item() - rhs.item()) < 1e-12
    v = convert.clip_gl_to_vk(torch.tensor([[0.3, -0.2, -0.5, 2.0]]))
    assert torch.equal(v, torch.tensor([[0.3, -0.2, 0.75, 2.0]]))


def test_sum_contribs_groups_of_four_left_to_right():
    """Six contributions sum as (a+b+c+d) + (e+f): in float32, 1e8 + (3+3)
    rounds to 1e8 + 8, while a flat left fold would drop each 3 on its own."""
    vals = [torch.tensor([x], dtype=torch.float32) for x in (1e8, 0.0, 0.0, 0.0, 3.0, 3.0)]
    assert convert.sum_contribs(vals).item() == 100000008.0
    flat = vals[0]
    for v in vals[1:]:
        flat = flat + v
    assert flat.item() == 1e8
    one = torch.tensor([3.0])
    assert convert.sum_contribs([one]) is one
    nine = [torch.tensor([float(i)]) for i in range(9)]
    assert convert.sum_contribs(nine).item() == 36.0


def test_provenance_lives_with_the_tensor():
    t = torch.zeros(3)
    rec = provenance.RasterOrigin(clip_vk=None, tri=None, resolution=(1, 1), ctx=None)
    provenance.stamp(t, rec)
    assert provenance.origin(t, provenance.RasterOrigin, "rasterize") is rec
    for other in (t.clone(), t.detach(), t[:2], t + 0):
        with pytest.raises(RuntimeError):
            provenance.origin(other, provenance.RasterOrigin, "rasterize")
    with pytest.raises(RuntimeError):
        provenance.origin(t, provenance.InterpOrigin, "interpolate")
    ref = weakref.ref(rec)
    del t, rec
    gc.collect()
    assert ref() is None  # the stamp dies with its tensor


def test_argument_checks():
    assert convert.resolution_hw([4, 6]) == (4, 6)
    assert convert.resolution_hw((np.int64(2), 3)) == (2, 3)
    for bad in ([0, 6], [4], [4, 6, 1], None, ["a", 2]):
        with pytest.raises(ValueError):
            convert.resolution_hw(bad)
    assert convert.vertex_batch(torch.zeros(3, 4)).shape == (1, 3, 4)
    assert convert.vertex_batch(torch.zeros(2, 3, 4)).shape == (2, 3, 4)
    with pytest.raises(ValueError):
        convert.vertex_batch(torch.zeros(3))
    assert convert.image_batch(torch.zeros(2, 3, 1), "c").shape == (1, 2, 3, 1)
    with pytest.raises(ValueError):
        convert.channels(5, "attr")
    from opendressi_amd.torch.context import tri_int32
    with pytest.raises(TypeError):
        tri_int32(torch.zeros(2, 3))
    with pytest.raises(ValueError):
        tri_int32(torch.zeros(2, 4, dtype=torch.int32))
    assert tri_int32(torch.tensor([[0, 1, 2]])).dtype == torch.int32


def test_vertex_adjacency_of_the_mesh_cache():
    """The {max_deg, V} adjacency the surface caches per topology lists each
    vertex's incident faces in ascending order, -1 padded."""
    from opendressi_amd.runtime import vertex_faces_tex
    faces = np.array([[0, 1, 2], [1, 3, 2], [2, 3, 4]], np.float32)
    vft = vertex_faces_tex(faces, 5)
    assert vft.shape == (3, 5)
    assert vft[:, 2].tolist() == [0, 1, 2]
    assert vft[:, 0].tolist() == [0, -1, -1]
    assert vft[:, 3].tolist() == [1, 2, -1]
