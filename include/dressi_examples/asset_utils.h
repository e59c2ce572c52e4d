/* dressi_examples/asset_utils.h -- the examples' asset and matrix helpers
 * (the reference's examples/common/asset_utils.h:11-105: same namespace,
 * names, signatures and layouts) implemented in libdressi_hip.so with zlib
 * as the only dependency, so example code builds offline: compile with
 * `-I include -I include/dressi_examples` and link `-ldressi_hip`.
 *
 * File formats and what is read:
 *  - OBJ (text): v / vt / f records, faces of any size fan-triangulated,
 *    1-based and negative (relative) indices; unwelded per (position,
 *    texcoord) pair in first-use order; vt's v flipped (1 - v).
 *  - glTF 2.0 (.gltf with base64 data URIs or external .bin files, .glb):
 *    the first primitive of the first mesh: POSITION, TEXCOORD_0 (v
 *    flipped), indices; float / uint32 / uint16 / uint8 components.
 *  - OpenEXR (single-part scanline): HALF / FLOAT / UINT channels with NONE,
 *    ZIPS or ZIP compression; R, G, B (a single channel is replicated).
 *    Written as HALF R, G, B with ZIP compression.
 *  - PNG: 8-bit and 16-bit gray, gray + alpha, RGB, RGBA and palette images,
 *    not interlaced; loaded as RGB in [0, 1] (alpha dropped). Written as
 *    8-bit RGB.
 * Errors throw std::runtime_error, as the reference's loaders do. */
#ifndef DRESSI_EXAMPLES_ASSET_UTILS_H
#define DRESSI_EXAMPLES_ASSET_UTILS_H

#include <array>
#include <string>
#include <vector>

#include "dressi/mesh_utils.h"
#include "dressi/types.h"

namespace dressi_examples {

// Unwelded triangle mesh: pos {V,1} x 3, uv {V,1} x 2, faces {F,1} x 3
struct Mesh {
    dressi::CpuImage pos;
    dressi::CpuImage uv;
    dressi::CpuImage faces;
    uint32_t numVertices() const { return pos.width; }
    uint32_t numFaces() const { return faces.width; }
};

// positions centred on the origin with maximum extent 1
Mesh LoadObjMesh(const std::string& path);
Mesh LoadGltfMesh(const std::string& path);

// The first node that has a mesh (its local matrix applied on the CPU), that
// mesh's first primitive and its metallic-roughness material
// (asset_utils.h:30-52 of the reference's examples). uv keeps glTF's V
// (whole-period offsets removed); normal is unit, tangent xyz unit + w the
// handedness, both generated when the file lacks them. Texture slots are
// 3-channel [0, 1] images (width 0 when absent); base_color and emissive
// stay sRGB-encoded.
struct GltfScene {
    Mesh mesh;
    dressi::CpuImage normal;              // {V,1,3}
    dressi::CpuImage tangent;             // {V,1,4}
    dressi::CpuImage base_color;          // sRGB-encoded
    dressi::CpuImage metallic_roughness;  // G = roughness, B = metallic
    dressi::CpuImage normal_map;          // tangent space
    dressi::CpuImage occlusion;           // R = AO
    dressi::CpuImage emissive;            // sRGB-encoded
};
// `normalize`: positions centred with maximum extent 1, as LoadGltfMesh.
GltfScene LoadGltfScene(const std::string& path, bool normalize = true);

// RGB in [0, 1] (PNG or baseline / extended-sequential JPEG)
dressi::CpuImage LoadImageRgb(const std::string& path);
// 3-channel float (EXR)
dressi::CpuImage LoadImageExr(const std::string& path);
void SaveImageExr(const std::string& path, const dressi::CpuImage& img);
// max(v, 0)^2.2
dressi::CpuImage SrgbToLinear(const dressi::CpuImage& img);
// 2x2 means, odd extents round up (the last row / column repeats)
dressi::CpuImage DownsampleHalf(const dressi::CpuImage& img);
// 1- or 3-channel image clamped to [0, 1], 8-bit RGB
void SaveImagePng(const std::string& path, const dressi::CpuImage& img);
// same-size images in a 3-channel grid, `cols` per row (gray replicated)
dressi::CpuImage TileImages(const std::vector<dressi::CpuImage>& imgs, uint32_t cols);

// column-major 4x4 (m[col * 4 + row])
using Mat4 = std::array<float, 16>;
Mat4 Mul(const Mat4& a, const Mat4& b);
Mat4 LookAt(const std::array<float, 3>& eye, const std::array<float, 3>& center,
            const std::array<float, 3>& up);
// Vulkan clip space: y down, depth in [0, 1]
Mat4 PerspectiveVk(float fovy_rad, float aspect, float z_near, float z_far);
// clip {V,1} x 4 = mvp * (pos, 1)
dressi::CpuImage TransformToClip(const dressi::CpuImage& pos, const Mat4& mvp);

using dressi::ScreenAttr;
using dressi::UvAsClip;

}  // namespace dressi_examples

#endif  // DRESSI_EXAMPLES_ASSET_UTILS_H
