/* dressi/mesh_utils.h -- host builders of the static-topology images the
 * raster / gather ops read (the reference's include/dressi/mesh_utils.h:
 * 16-53). Faces are {F,1} images of float vertex ids (3 channels). */
#ifndef DRESSI_MESH_UTILS_H
#define DRESSI_MESH_UTILS_H

#include <array>
#include <vector>

#include "dressi/types.h"

namespace dressi {

// neighbours of each vertex (ascending ids)
std::vector<std::vector<uint32_t>> BuildVertexAdjacency(const CpuImage& faces, uint32_t n_verts);
// each pair of faces sharing an edge, once
std::vector<std::array<uint32_t, 2>> BuildFaceAdjacency(const CpuImage& faces);
// {V, max_degree} incident face ids per vertex (ascending), -1 padding
CpuImage VertexFacesTex(const CpuImage& faces, uint32_t n_verts);
// {V, max_degree} neighbour vertex ids per vertex, -1 padding
CpuImage VertexNeighborsTex(const CpuImage& faces, uint32_t n_verts);
// {F,1} x 3: up to three edge-adjacent faces, in ascending order of the
// shared edge's (min, max) vertex ids, -1 padding
CpuImage FaceNeighborsTex(const CpuImage& faces);

// HardSoftRas soft geometry on the host: every face unwelded and enlarged
// about its screen centroid (the F::SoftClip arithmetic), its face index per
// corner, and the sequential faces (3f, 3f + 1, 3f + 2)
struct SoftGeometry {
    CpuImage clip;     // {3F,1} x 4
    CpuImage face_id;  // {3F,1} x 1
    CpuImage faces;    // {F,1} x 3
};
SoftGeometry BuildSoftGeometry(const CpuImage& hard_clip, const CpuImage& faces, ImgSize screen,
                               float radius_px);

// inverse-UV inputs: UvAsClip {V,1} x 4 = (u * 2 - 1, v * 2 - 1, 0.5, 1);
// ScreenAttr {V,1} x 4 = (screen x, screen y, 1, 0) of clip positions
CpuImage UvAsClip(const CpuImage& uv);
CpuImage ScreenAttr(const CpuImage& clip, ImgSize screen);

}  // namespace dressi

#endif  // DRESSI_MESH_UTILS_H
