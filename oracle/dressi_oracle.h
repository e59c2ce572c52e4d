/*
 * dressi_oracle.h -- CPU restatement of the reference's HardSoftRas
 * silhouette hot path. TEST INFRASTRUCTURE ONLY: used by tests/, by
 * __graft_entry__.smoke() as the checker, and by bench.py's cpu_baseline
 * leg. The product path (opendressi_amd/, include/dressi_hip.h) never links,
 * loads or calls it.
 *
 * Layout conventions follow the reference: {N,1} arrays are tightly packed
 * logical channels (VEC3 = 3 floats, VEC4 = 4 floats), face indices are
 * stored as floats, {V,deg} adjacency is row-major (d*V + v) with -1 padding,
 * screen images are row-major with row 0 at NDC y = -1.
 */
#ifndef DRESSI_ORACLE_H
#define DRESSI_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scene generation ---------------------------------------------------- */
/* examples/common/geometry_utils.cpp:24-84 (GenerateIcosphere); counts only
 * when pos/faces are NULL */
int or_icosphere(uint32_t level, uint32_t* n_verts, uint32_t* n_faces,
                 float* pos, float* faces);
/* examples/common/asset_utils.cpp:719-766 (Mul, LookAt, PerspectiveVk) */
void or_mat4_mul(const float a[16], const float b[16], float r[16]);
void or_look_at(const float eye[3], const float center[3], const float up[3],
                float m[16]);
void or_perspective_vk(float fovy_rad, float aspect, float z_near,
                       float z_far, float m[16]);
/* SplitMix64 -> Box-Muller standard normals (scene noise; no reference
 * counterpart -- the configs only say "seeded N(0, s)") */
void or_randn(uint64_t seed, uint32_t n, float* out);
/* examples/common/asset_utils.cpp:768-782 (TransformToClip) */
void or_transform_to_clip(const float* pos, uint32_t n_verts,
                          const float mvp[16], float* clip);

/* ---- mesh topology ------------------------------------------------------- */
/* src/core/mesh_utils.cpp:53-71 (VertexFacesTex). Returns max degree;
 * writes deg*V floats when out != NULL and cap >= deg*V. */
uint32_t or_vertex_faces_tex(const float* faces, uint32_t n_faces,
                             uint32_t n_verts, float* out, uint32_t cap);

/* ---- ops (each mirrors one reference op's CPU kernel) ---------------------- */
void or_soft_clip(const float* clip, uint32_t n_verts, const float* faces,
                  uint32_t n_faces, uint32_t w, uint32_t h, float radius,
                  float* out);
void or_rasterize_soft(const float* soft_clip, const float* face_id,
                       const float* faces_soft, const float* hard_clip,
                       uint32_t n_verts, const float* faces_tex,
                       uint32_t n_faces, uint32_t w, uint32_t h, float radius,
                       const float* prev, float* out);
void or_rasterize(const float* clip, uint32_t n_verts, const float* attr,
                  uint32_t n_comp, const float* faces, uint32_t n_faces,
                  uint32_t w, uint32_t h, float* out);
void or_rasterize_face_id(const float* clip, uint32_t n_verts,
                          const float* faces, uint32_t n_faces, uint32_t w,
                          uint32_t h, float* out);
void or_lookup_faces(const float* attr, uint32_t n_comp, const float* faces,
                     uint32_t n_faces, uint32_t corner, float* out);
void or_lookup_faces_bwd(const float* gy, uint32_t n_comp, const float* faces,
                         uint32_t n_faces, const float* vtx_faces,
                         uint32_t n_verts, uint32_t max_deg, uint32_t corner,
                         float* out);
void or_face_fetch(const float* attr, uint32_t n_comp, uint32_t n_faces,
                   const float* idx, uint32_t w, uint32_t h, float* out);
void or_face_fetch_bwd(const float* gy, uint32_t n_comp, const float* idx,
                       uint32_t w, uint32_t h, const float* prj0,
                       const float* prj1, const float* prj2, uint32_t n_faces,
                       float seed, float radius, uint32_t n_samples,
                       float* out);
uint32_t or_wang_hash(uint32_t x);
float or_hash_to_unit(uint32_t f, uint32_t s, uint32_t seed, uint32_t salt);

/* ---- the HardSoftRas silhouette iteration ---------------------------------- */
/* Per-pixel forward of the example's soft-probability chain + silhouette
 * composition + L2 term (examples/silhouette_optimization/run.cpp:253-342,
 * 382-393). `rs` is the RasterizeSoft output image (VEC4), `tri[k]` the
 * LookupFaces outputs {F,4}. Writes pred and the per-view loss image. */
void or_hsr_forward(const float* rs, const float* tri0, const float* tri1,
                    const float* tri2, uint32_t n_faces, const float* target,
                    uint32_t w, uint32_t h, float radius, float* pred,
                    float* view_loss);
/* Per-pixel backward of the same chain: the gradient images (VEC4 {S,S})
 * reaching FaceFetch(tri0/1/2), as the reference's BuildBackward composes
 * them (src/core/build_backward.cpp:62-149). */
void or_hsr_backward(const float* rs, const float* tri0, const float* tri1,
                     const float* tri2, uint32_t n_faces, const float* target,
                     uint32_t w, uint32_t h, float radius, float* gy0,
                     float* gy1, float* gy2);

/* Whole fit, same contract as the reference harness (oracle/ref_harness.cpp
 * refh_hsr_fit): all outputs nullable. `n_threads` > 1 splits the per-view
 * work over POSIX threads (views are independent until the pos gradient). */
int or_hsr_fit(const float* pos0, uint32_t n_verts, const float* faces,
               uint32_t n_faces, const float* tgt_pos, uint32_t n_tverts,
               const float* tgt_faces, uint32_t n_tfaces, const float* mvps,
               uint32_t n_views, uint32_t screen_px, float radius_px,
               uint32_t samples, float lr, uint32_t iters, float* out_pos,
               float* out_m, float* out_v, float* out_t, float* out_loss,
               float* out_grad0, float* out_pred0, float* out_target,
               float* out_rs0, float* out_lossimg0);

/* ---- screen-space antialiasing (technique aa) ------------------------- */
/* src/core/cpu_raster.h:67-80 (AaPair) */
typedef struct {
    float r;
    uint32_t ia, ib;
    float qa[2], qb[2];
    float es, len;
} or_aa_pair;
/* src/core/cpu_raster.cpp:371-454 (EvalAaPair) */
int or_eval_aa_pair(const float* tri, const float* clip, uint32_t n_verts,
                    const float* faces, uint32_t n_faces, uint32_t w, uint32_t h,
                    int sx, int sy, int nx, int ny, or_aa_pair* out);
/* src/core/f_ops.cpp:2480-2579 (AntiAlias) */
void or_antialias(const float* img, uint32_t n_comp, const float* tri,
                  const float* clip, uint32_t n_verts, const float* faces,
                  uint32_t n_faces, uint32_t w, uint32_t h, float* out);
/* src/core/f_ops.cpp:2220-2278 (AntiAliasBwdImg) */
void or_antialias_bwd_img(const float* gy, uint32_t n_comp, const float* tri,
                          const float* clip, uint32_t n_verts, const float* faces,
                          uint32_t n_faces, uint32_t w, uint32_t h, float* out);
/* src/core/f_ops.cpp:2284-2476 (AntiAliasBwdVtx); out {V, wide ? max_deg : 1}
 * VEC4 */
void or_antialias_bwd_vtx(const float* gy, const float* img, uint32_t n_comp,
                          const float* tri, const float* clip, uint32_t n_verts,
                          const float* faces, uint32_t n_faces, const float* vtx_faces,
                          uint32_t max_deg, float seed, uint32_t n_samples, int wide,
                          uint32_t w, uint32_t h, float* out);
/* src/core/f_ops.cpp:1218-1246 (ColSum) */
void or_col_sum(const float* x, uint32_t n_comp, uint32_t w, uint32_t h, float* out);
/* examples/silhouette_optimization/run.cpp:229-238, 346-357, 382-437
 * (technique aa, no regularizers) */
int or_aa_fit(const float* pos0, uint32_t n_verts, const float* faces, uint32_t n_faces,
              const float* tgt_pos, uint32_t n_tverts, const float* tgt_faces,
              uint32_t n_tfaces, const float* mvps, uint32_t n_views, uint32_t screen_px,
              uint32_t samples, float lr, uint32_t iters, float* out_pos, float* out_m,
              float* out_v, float* out_t, float* out_loss, float* out_grad0,
              float* out_pred0, float* out_target, float* out_tri0, float* out_lossimg0);

/* ---- texture path (C3) ---- */
/* examples/common/geometry_utils.cpp:86-131 (GenerateUvSphere); counts only
 * when an output is NULL */
int or_uv_sphere(uint32_t stacks, uint32_t slices, uint32_t* n_verts, uint32_t* n_faces,
                 float* pos, float* uv, float* faces);
/* src/core/mesh_utils.cpp:180-189 (UvAsClip) */
void or_uv_as_clip(const float* uv, uint32_t n_verts, float* clip);
/* src/core/mesh_utils.cpp:191-203 (ScreenAttr) */
void or_screen_attr(const float* clip, uint32_t n_verts, uint32_t w, uint32_t h, float* attr);
/* src/core/f_ops.cpp:2764-2778 (TextureBilinear), ibl_math.h:91-115 */
void or_texture_bilinear(const float* tex, uint32_t tw, uint32_t th, uint32_t n_comp,
                         const float* uv, size_t n_px, float* out);
/* src/core/f_ops.cpp:2605-2639 (F::Texture, nearest clamp-to-edge) */
void or_texture_nearest(const float* tex, uint32_t tw, uint32_t th, uint32_t n_comp,
                        const float* uv, size_t n_px, float* out);
/* src/core/f_ops.cpp:2586-2601 (GatherByInverseUV), glsl_codegen.cpp:658-703 */
void or_gather_inv_uv(const float* gy, uint32_t n_comp, uint32_t sw, uint32_t sh,
                      const float* inv_uv, uint32_t tw, uint32_t th, const float* uv,
                      float* out);
/* src/core/f_ops.cpp:2665-2731 (GatherByInverseUVBilinear) */
void or_gather_inv_uv_bilinear(const float* gy, uint32_t n_comp, uint32_t sw, uint32_t sh,
                               const float* inv_uv, uint32_t tw, uint32_t th, const float* uv,
                               float* out);
/* the C3 texture fit: examples/texture_optimization/run.cpp:112-145 with
 * TextureBilinear, RGBA texture, L2 on RGB, in-graph Adam */
int or_tex_fit(const float* pos, uint32_t n_verts, const float* uv, const float* faces,
               uint32_t n_faces, const float* mvps, uint32_t n_sets, uint32_t n_views,
               uint32_t screen_px, uint32_t tex_w, uint32_t tex_h, const float* gt_tex,
               const float* tex0, float lr, uint32_t iters, float* out_tex, float* out_m,
               float* out_v, float* out_t, float* out_loss, float* out_grad0, float* out_pred0,
               float* out_target0, float* out_lossimg0, float* out_uv0, float* out_invuv0);

/* src/core/f_ops.cpp:1281-1355 (GatherDistGrad): gy, ro {h,w,4}; out wide
 * ? {max_deg, V, 4} : {V, 4} */
void or_gather_dist_grad(const float* gy, const float* ro, const float* clip, uint32_t n_verts,
                         const float* faces, uint32_t n_faces, const float* vtx_faces,
                         uint32_t max_deg, int wide, uint32_t w, uint32_t h, float* out);

/* ---- PBR / IBL (pbr_oracle.c) ------------------------------------------- */
/* EquirectSample (src/core/f_ops.cpp:2921-2964) map {mw,mh} x n at dir {dw,dh}
 * VEC3 -> out {dw,dh} x n; with gy {dw,dh} x n instead the map VJP
 * (EquirectSampleBwd + TileSum, f_ops.cpp:2786-2919) -> out {mw,mh} x n */
int or_equirect_sample(const float* map, uint32_t mw, uint32_t mh, uint32_t n, const float* dir,
                       uint32_t dw, uint32_t dh, const float* gy, float* out);
/* AvgPool2x2 (f_ops.cpp:3411-3415); with gy its VJP -> out {w,h} x n */
int or_avg_pool2x2(const float* x, uint32_t w, uint32_t h, uint32_t n, const float* gy,
                   float* out);
/* IrradianceConv (f_ops.cpp:3006-3087) env {sw,sh} -> {ow,oh}; with gy
 * IrradianceConvBwd (f_ops.cpp:2970-3004) -> {sw,sh} */
int or_irradiance_conv(const float* env, uint32_t sw, uint32_t sh, uint32_t n, uint32_t ow,
                       uint32_t oh, const float* gy, float* out);
/* PrefilterConv (+ PrefilterConvNorm) (f_ops.cpp:3166-3348); with gy
 * PrefilterConvBwd (f_ops.cpp:3207-3262) */
int or_prefilter_conv(const float* env, uint32_t sw, uint32_t sh, uint32_t n, uint32_t ow,
                      uint32_t oh, float roughness, const float* gy, float* out);
/* PrefilterEnv (f_ops.cpp:3089-3157), forward only */
int or_prefilter_env(const float* env, uint32_t sw, uint32_t sh, uint32_t n, uint32_t ow,
                     uint32_t oh, float roughness, uint32_t n_samples, float* out);
/* BrdfIntegrationLut (f_ops.cpp:3350-3409): {w,h} VEC2 */
int or_brdf_lut(uint32_t w, uint32_t h, uint32_t n_samples, float* out);
/* the C5 split-sum PBR/IBL material + environment fit
 * (examples/common/pbr_graph.cpp, src/core/ibl.cpp; in-graph Adam on albedo,
 * mr and env, L1 loss on the Reinhard-mapped image) */
int or_pbr_fit(const float* pos, const float* normal, uint32_t n_verts, const float* uv,
               const float* faces, uint32_t n_faces, const float* mvps, const float* frames,
               const float* light, uint32_t n_views, uint32_t screen_px, uint32_t tex_w,
               uint32_t tex_h, uint32_t env_w, uint32_t env_h, uint32_t levels,
               const float* gt_albedo, const float* gt_mr, const float* gt_env,
               const float* albedo0, const float* mr0, const float* env0, float lr,
               uint32_t iters, float* out_albedo, float* out_mr, float* out_env, float* out_loss,
               float* out_g_albedo0, float* out_g_mr0, float* out_g_env0, float* out_pred0,
               float* out_target0, float* out_mask0);

#ifdef __cplusplus
}
#endif

#endif /* DRESSI_ORACLE_H */
