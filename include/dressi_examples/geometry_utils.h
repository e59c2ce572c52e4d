/* dressi_examples/geometry_utils.h -- the examples' mesh and optimisation
 * helpers (the reference's examples/common/geometry_utils.h:11-104: same
 * namespace, names, signatures and layouts), implemented in
 * libdressi_hip.so. Host code; the in-graph transform builds F:: ops. */
#ifndef DRESSI_EXAMPLES_GEOMETRY_UTILS_H
#define DRESSI_EXAMPLES_GEOMETRY_UTILS_H

#include <array>
#include <string>
#include <vector>

#include "asset_utils.h"
#include "dressi/dressi.h"
#include "dressi/mesh_utils.h"

namespace dressi_examples {

// topology builders of the library
using dressi::BuildFaceAdjacency;
using dressi::BuildSoftGeometry;
using dressi::BuildVertexAdjacency;
using dressi::FaceNeighborsTex;
using dressi::SoftGeometry;
using dressi::VertexFacesTex;
using dressi::VertexNeighborsTex;

// welded unit icosphere, uv zero; level 0 = 12 v / 20 f, x4 faces a level
Mesh GenerateIcosphere(uint32_t level);

// lat-long unit sphere, uv = (j / slices, i / stacks); the seam column is
// duplicated and the pole triangles are left out (stacks >= 2, slices >= 3)
Mesh GenerateUvSphere(uint32_t stacks, uint32_t slices);

// each dst vertex's direction from the origin is cast against the control
// mesh's rest triangles; the nearest hit's barycentric weights blend the
// control mesh's deformed positions
dressi::CpuImage TransferDeformationByDirection(const dressi::CpuImage& ctrl_rest_pos,
                                                const dressi::CpuImage& ctrl_faces,
                                                const dressi::CpuImage& ctrl_deformed_pos,
                                                const dressi::CpuImage& dst_pos);

// OBJ with positions and faces (no uv); a path that cannot be opened is
// skipped
void SaveObjMesh(const std::string& path, const Mesh& mesh);

// OBJ with v / vt (vt's v written as 1 - v) / f a/a, plus `<stem>.mtl`
// naming `texture_filename` as map_Kd
void SaveTexturedObjMesh(const std::string& path, const Mesh& mesh,
                         const std::string& texture_filename);

// lambda * (p - mean of its neighbours), zero for isolated vertices
dressi::CpuImage UniformLaplacianGrad(const dressi::CpuImage& pos,
                                      const std::vector<std::vector<uint32_t>>& adj,
                                      float lambda);

// gradient of lambda * sum over adjacent face pairs of (1 - n_f . n_g);
// pairs with a degenerate face (|cross| < 1e-12) are skipped
dressi::CpuImage NormalConsistencyGrad(const dressi::CpuImage& pos,
                                       const dressi::CpuImage& faces,
                                       const std::vector<std::array<uint32_t, 2>>& face_adj,
                                       float lambda);

// adjacent face pairs with n_f . n_g < 0
uint32_t CountFlippedFacePairs(const dressi::CpuImage& pos, const dressi::CpuImage& faces,
                               const std::vector<std::array<uint32_t, 2>>& face_adj);

// g_pos {V,1} x 3 = the first three columns of mvp (column-major),
// transposed, times g_clip {V,1} x 4
dressi::CpuImage ChainRuleClipToPos(const dressi::CpuImage& g_clip, const Mat4& mvp);

// clip {V,1} VEC4 = mvp * (pos, 1) as elementwise F:: ops
dressi::Variable TransformToClipVar(const dressi::Variable& pos, const Mat4& mvp);

struct AdamState {
    std::vector<float> m, v;
    int t = 0;
    float beta1 = 0.9f, beta2 = 0.999f, eps = 1e-8f;
};
// one bias-corrected Adam step; the state resets when the size changes
void AdamStep(AdamState& state, std::vector<float>& params, const std::vector<float>& grad,
              float lr);

}  // namespace dressi_examples

#endif  // DRESSI_EXAMPLES_GEOMETRY_UTILS_H
