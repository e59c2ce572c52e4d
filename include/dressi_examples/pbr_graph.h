/* dressi_examples/pbr_graph.h -- the examples' split-sum PBR rendering graph
 * built from F:: ops (the reference's examples/common/pbr_graph.h:13-107:
 * same namespace, struct names, fields and builder signatures), implemented
 * in libdressi_hip.so. Host code: the builders only create graph nodes; the
 * graph runs wherever it is handed (DressiAD, or the fused PBR plan of the
 * C ABI for the material / environment fit). */
#ifndef DRESSI_EXAMPLES_PBR_GRAPH_H
#define DRESSI_EXAMPLES_PBR_GRAPH_H

#include <vector>

#include "dressi/dressi.h"

namespace dressi_examples {

// per-vertex inputs ({V,1} images except faces {F,1})
struct PbrGeometryLeaves {
    dressi::Variable clip{nullptr};     // VEC4 clip-space positions
    dressi::Variable uvh{nullptr};      // VEC4 (u, v, 1, tangent handedness)
    dressi::Variable normal{nullptr};   // VEC3 world normals
    dressi::Variable tangent{nullptr};  // VEC3 world tangents
    dressi::Variable wpos{nullptr};     // VEC3 world positions
    dressi::Variable faces{nullptr};    // IVEC3 vertex indices
};

// texture-space material maps
struct PbrMaterialLeaves {
    dressi::Variable albedo{nullptr};      // VEC3 linear base colour
    dressi::Variable mr{nullptr};          // VEC3: y roughness, z metallic
    dressi::Variable normal_map{nullptr};  // VEC3 tangent-space normal in [0,1]
    dressi::Variable ao{nullptr};          // VEC3: x ambient occlusion
    dressi::Variable emissive{nullptr};    // VEC3 linear emission
};

// per-view camera frame and the point light ({1,1} VEC3 images)
struct PbrFrameLeaves {
    dressi::Variable cam_pos{nullptr};    // eye position
    dressi::Variable cam_fwd{nullptr};    // unit view direction
    dressi::Variable cam_right{nullptr};  // right axis * tan(fov / 2) * aspect
    dressi::Variable cam_up{nullptr};     // up axis * tan(fov / 2)
    dressi::Variable light_pos{nullptr};  // light position
    dressi::Variable light_col{nullptr};  // radiant intensity
};

// the environment and its split-sum maps
struct PbrIblMaps {
    dressi::Variable env{nullptr};        // VEC3 equirect HDR (linear)
    dressi::Variable irr{nullptr};        // irradiance / pi
    std::vector<dressi::Variable> pref;   // prefiltered levels by roughness
    dressi::Variable lut{nullptr};        // BRDF integration map
};

// irradiance, prefiltered levels (the GGX convolution when the environment
// is optimised, else the sampled prefilter) and the BRDF map of `env`
PbrIblMaps BuildPbrIblMaps(const dressi::Variable& env, bool differentiable_prefilter = false);

// screen-space G-buffer of one view
struct PbrGBuffer {
    dressi::Variable uv{nullptr};      // VEC2 texture coordinates
    dressi::Variable mask{nullptr};    // FLOAT coverage
    dressi::Variable handed{nullptr};  // FLOAT tangent handedness, +-1
    dressi::Variable g_n{nullptr};     // VEC3 interpolated normal (not unit)
    dressi::Variable g_t{nullptr};     // VEC3 interpolated tangent (not unit)
    dressi::Variable g_p{nullptr};     // VEC3 world position
};

PbrGBuffer BuildPbrGBuffer(const PbrGeometryLeaves& geom, dressi::ImgSize screen);

// screen-space results of the shading
struct PbrOutputs {
    dressi::Variable ldr{nullptr};     // VEC3 Reinhard-mapped, gamma 2.2
    dressi::Variable mapped{nullptr};  // VEC3 Reinhard-mapped, linear
    dressi::Variable hdr{nullptr};     // VEC3 shaded surface over the environment
    dressi::Variable mask{nullptr};    // FLOAT coverage
    dressi::Variable uv{nullptr};      // VEC2 G-buffer texture coordinates
    dressi::Variable albedo{nullptr};  // VEC3 sampled albedo
    dressi::Variable normal{nullptr};  // VEC3 shading normal
};

// Cook-Torrance point light + split-sum IBL + emission over the
// environment seen along each pixel's view ray; `inv_uv` is the
// screen-attribute raster that TextureBilinear's backward needs
PbrOutputs BuildPbrShade(const PbrGBuffer& gbuf, const PbrMaterialLeaves& mat,
                         const PbrFrameLeaves& frame, const PbrIblMaps& ibl,
                         const dressi::Variable& inv_uv, dressi::ImgSize screen,
                         bool normal_mapping = true);

// BuildPbrShade of BuildPbrGBuffer
PbrOutputs BuildPbrForward(const PbrGeometryLeaves& geom, const PbrMaterialLeaves& mat,
                           const PbrFrameLeaves& frame, const PbrIblMaps& ibl,
                           const dressi::Variable& inv_uv, dressi::ImgSize screen,
                           bool normal_mapping = true);

}  // namespace dressi_examples

#endif  // DRESSI_EXAMPLES_PBR_GRAPH_H
