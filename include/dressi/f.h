/* dressi/f.h -- the F:: op catalogue of the graph API (the reference's
 * include/dressi/f.h:9-338: same functions and signatures; each op's
 * semantics, backward and float operation order follow the reference's CPU
 * kernel in src/core/f_ops.cpp).
 *
 * Elementwise ops broadcast {1,1} inputs over images and 1-component inputs
 * over vectors. Integer-typed images carry their values as floats. */
#ifndef DRESSI_F_H
#define DRESSI_F_H

#include "dressi/function.h"
#include "dressi/types.h"
#include "dressi/variable.h"

namespace dressi {
namespace F {

// ---- constants ({1,1}) ------------------------------------------------------
Variable Float(float fv);
Variable Vec2(float x, float y);
Variable Vec3(float x, float y, float z);
Variable Vec4(float x, float y, float z, float w);

// ---- arithmetic ---------------------------------------------------------------
Variable Add(const Variable& x0, const Variable& x1);
Variable Sub(const Variable& x0, const Variable& x1);
Variable Mul(const Variable& x0, const Variable& x1);
Variable Div(const Variable& x0, const Variable& x1);
Variable Neg(const Variable& x);

// ---- math (per component) -----------------------------------------------------
Variable Sin(const Variable& x);
Variable Cos(const Variable& x);
Variable Tan(const Variable& x);
Variable Asin(const Variable& x);
Variable Acos(const Variable& x);
Variable Atan(const Variable& x);
Variable Atan2(const Variable& y, const Variable& x);
Variable Exp(const Variable& x);
Variable Exp2(const Variable& x);
Variable Log(const Variable& x);
Variable Log2(const Variable& x);
Variable Sqrt(const Variable& x);
Variable InverseSqrt(const Variable& x);
Variable Abs(const Variable& x);
Variable Sign(const Variable& x);
Variable Floor(const Variable& x);
Variable Fract(const Variable& x);
Variable Mod(const Variable& x, const Variable& m);
Variable Pow(const Variable& x, const Variable& p);
Variable Max(const Variable& x0, const Variable& x1);
Variable Min(const Variable& x0, const Variable& x1);
Variable Clamp(const Variable& x, const Variable& lo, const Variable& hi);
Variable Mix(const Variable& x0, const Variable& x1, const Variable& t);
Variable Step(const Variable& edge, const Variable& x);
Variable SmoothStep(const Variable& e0, const Variable& e1, const Variable& x);
Variable Sigmoid(const Variable& x);

// ---- comparisons (FLOAT 0 / 1, no gradient) -----------------------------------
Variable Less(const Variable& x0, const Variable& x1);
Variable LessEqual(const Variable& x0, const Variable& x1);
Variable Greater(const Variable& x0, const Variable& x1);
Variable GreaterEqual(const Variable& x0, const Variable& x1);

// ---- vectors ------------------------------------------------------------------
Variable Vec2(const Variable& x, const Variable& y);
Variable Vec3(const Variable& x, const Variable& y, const Variable& z);
Variable Vec3(const Variable& xy, const Variable& z);
Variable Vec4(const Variable& x, const Variable& y, const Variable& z, const Variable& w);
Variable Vec4(const Variable& xyz, const Variable& w);
Variable GetX(const Variable& v);
Variable GetY(const Variable& v);
Variable GetZ(const Variable& v);
Variable GetW(const Variable& v);
Variable Dot(const Variable& a, const Variable& b);
Variable Cross(const Variable& a, const Variable& b);
Variable Length(const Variable& v);
Variable Distance(const Variable& a, const Variable& b);
Variable Normalize(const Variable& v);
Variable Reflect(const Variable& incident, const Variable& normal);
Variable CompSum(const Variable& v);  // sum of the components -> FLOAT

// ---- matrices (column-major MAT2..MAT4) ---------------------------------------
Variable MatMul(const Variable& a, const Variable& b);  // MAT x MAT, MAT x VEC
Variable Transpose(const Variable& m);
Variable OuterProduct(const Variable& col, const Variable& row);

// ---- broadcast and reductions -------------------------------------------------
// a {1,1} value replicated over an image of `size` (backward: the sum)
Variable Broadcast(const Variable& x, ImgSize size);
// pixel-wise sum of images (one n-ary node per <= 4 inputs)
Variable SumPixelWise(const Variables& xs);
Variable Sum(const Variable& x);   // whole image -> {1,1}, same vtype (2x2 sums)
Variable Mean(const Variable& x);  // whole image and components -> FLOAT {1,1}
// every pixel and component -> FLOAT {1,1} in one sequential pass; no
// backward (optimizer-side statistics of small arrays)
Variable SumAll(const Variable& x);

// ---- differentiable-rendering ops ----------------------------------------------
Variable StopGradient(const Variable& x);
// raster-pass-only ops of the reference's GLSL backend (fragment depth of a
// custom raster pass); they build graph nodes, but the HIP executor has no
// raster pipeline to run them in and raises DressiError
Variable SetFragDepth(const Variable& depth);
Variable PeelDepth(const Variable& frag_depth, const Variable& prev_frag_depth);

// depth-tested perspective-correct interpolation of a vertex attribute;
// background 0 (cpu_raster.cpp:195-225)
Variable Rasterize(const Variable& vtx_clip_pos, const Variable& vtx_attrib, const Variable& faces,
                   ImgSize screen_size);
// HardSoftRas (VEC4 signed_dist_px, face_id, hard_depth, coverage per pixel;
// cpu_raster.cpp:241-355); differentiable w.r.t. vtx_clip_hard_tex through
// the distance channel
Variable RasterizeSoft(const Variable& vtx_clip_soft, const Variable& face_id,
                       const Variable& faces_soft, const Variable& vtx_clip_hard_tex,
                       const Variable& faces_tex, const Variable& vtx_faces_tex,
                       ImgSize screen_size, float radius_px);
// depth-peeling form: fragments at or in front of prev_shifted_depth
// (+1e-4) are discarded
Variable RasterizeSoft(const Variable& vtx_clip_soft, const Variable& face_id,
                       const Variable& faces_soft, const Variable& vtx_clip_hard_tex,
                       const Variable& faces_tex, const Variable& vtx_faces_tex,
                       const Variable& prev_shifted_depth, ImgSize screen_size, float radius_px);
// face index + 1 per covered pixel, 0 background
Variable RasterizeFaceId(const Variable& vtx_clip_pos, const Variable& vtx_attrib_dummy,
                         const Variable& faces, ImgSize screen_size);
// screen-space edge antialiasing (8-neighbour blend across face-id
// boundaries); differentiable w.r.t. img and vtx_clip; n_samples 0 = exact
// vertex backward, > 0 = stochastic (seeded by `seed`)
Variable AntiAlias(const Variable& img, const Variable& tri_id, const Variable& vtx_clip,
                   const Variable& faces, const Variable& vtx_faces_tex, const Variable& seed,
                   uint32_t n_samples = 8);

// ---- indexed access --------------------------------------------------------------
Variable ScreenCoord(ImgSize size);  // (x + 0.5, y + 0.5), VEC2
// out{F,1} = vtx_attr[faces[f][corner]]; exact backward over vtx_faces_tex
Variable LookupFaces(const Variable& vtx_attr, const Variable& faces_tex,
                     const Variable& vtx_faces_tex, uint32_t corner);
// out(p) = tri_attr[idx(p) - 1] (0 on background); stochastic edge-sample
// backward
Variable FaceFetch(const Variable& tri_attr, const Variable& idx_img, const Variable& tri_prj_0,
                   const Variable& tri_prj_1, const Variable& tri_prj_2, const Variable& seed,
                   float radius_px, uint32_t n_samples = 4);

// ---- in-graph selection -----------------------------------------------------------
// {1,1} = tex(x_index, round(row_idx))
Variable PixelFetch(const Variable& tex, uint32_t x_index, const Variable& row_idx);
// out(p) = atlas(p.x, p.y + round(tile_idx) * tile_h)
Variable TileFetch(const Variable& atlas, const Variable& tile_idx, uint32_t tile_h);

// ---- mesh utilities (forward only) ---------------------------------------------------
Variable SoftClip(const Variable& vtx_clip_hard_tex, const Variable& faces_tex,
                  ImgSize screen_size, float radius_px);
Variable VertexNeighborMean(const Variable& pos_tex, const Variable& vtx_neighbors_tex);
Variable NormalConsistencyFaceTerm(const Variable& pos_tex, const Variable& faces_tex,
                                   const Variable& face_adj_tex);
Variable NormalConsistencyVertexGrad(const Variable& face_term, const Variable& pos_tex,
                                     const Variable& faces_tex, const Variable& vtx_faces_tex);

// ---- textures ---------------------------------------------------------------------
// nearest sampling; gradient to `tex` by the inverse-UV gather of inv_uv
Variable Texture(const Variable& tex, const Variable& uv, const Variable& inv_uv);

// ---- IBL (split-sum, equirect maps) --------------------------------------------------
Variable TextureBilinear(const Variable& tex, const Variable& uv, const Variable& inv_uv);
Variable EquirectSample(const Variable& map, const Variable& dir);
Variable IrradianceConv(const Variable& env, ImgSize out_size);
Variable PrefilterEnv(const Variable& env, ImgSize out_size, float roughness,
                      uint32_t n_samples = 256);
Variable PrefilterConv(const Variable& env, ImgSize out_size, float roughness);
Variable BrdfIntegrationLut(ImgSize size, uint32_t n_samples = 512);
Variable AvgPool2x2(const Variable& x);

}  // namespace F

// ---- operators ----------------------------------------------------------------------
Variable operator+(const Variable& a, const Variable& b);
Variable operator-(const Variable& a, const Variable& b);
Variable operator*(const Variable& a, const Variable& b);
Variable operator/(const Variable& a, const Variable& b);
Variable operator+(const Variable& a, float b);
Variable operator-(const Variable& a, float b);
Variable operator*(const Variable& a, float b);
Variable operator/(const Variable& a, float b);
Variable operator+(float a, const Variable& b);
Variable operator-(float a, const Variable& b);
Variable operator*(float a, const Variable& b);
Variable operator/(float a, const Variable& b);
Variable operator-(const Variable& x);
Variable operator<(const Variable& a, const Variable& b);
Variable operator<(float a, const Variable& b);
Variable operator<(const Variable& a, float b);
Variable operator<=(const Variable& a, const Variable& b);
Variable operator>(const Variable& a, const Variable& b);
Variable operator>=(const Variable& a, const Variable& b);

}  // namespace dressi

#endif  // DRESSI_F_H
