/*
 * dressi_hip.h -- C ABI of the MI355X-native Dressi-AD hot path.
 *
 * The library (opendressi_amd/libdressi_hip.so) replaces the reference's
 * Vulkan executor seam for the HardSoftRas silhouette path: the GLSL op
 * emitters + generated substages (src/codegen/glsl_codegen.cpp), the packer
 * (src/pack/) and the Vulkan plan/submit/transfer layer
 * (src/vk/executor.h:43-66, src/vk/transfer.h:16-91). Every entry point is
 * plain C: status-code return, sizes explicit, device buffers as raw
 * pointers, streams as opaque handles (hipStream_t). Nothing in a signature
 * is a torch type. Each declaration names the reference interface it
 * replaces (paths relative to the reference checkout).
 *
 * Layout conventions are the reference's logical ones: {N,1} arrays are
 * tightly packed channels (VEC3 = 3 floats, VEC4 = 4 floats), face indices
 * are floats (exact below 2^24), {V,deg} adjacency is row-major (d*V + v)
 * with -1 padding, screen images are row-major, row 0 = NDC y = -1, pixel
 * centres at +0.5, depth = z/w in [0,1].
 *
 * Errors: every call returns DRESSI_OK (0) or a negative dressi_status; the
 * message of the last failure on the calling thread is dressi_last_error()
 * (the reference throws DressiError "msg (file:line)", include/dressi/types.h:110-123).
 * Threading: a context is not thread-safe; calls on one context are
 * externally serialised (reference: src/vk/transfer.cpp:20-21).
 */
#ifndef DRESSI_HIP_H
#define DRESSI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum dressi_status {
    DRESSI_OK = 0,
    DRESSI_ERR_INVALID = -1,     /* bad argument / shape (DRESSI_CHECK) */
    DRESSI_ERR_HIP = -2,         /* HIP runtime failure ("GPU execution failed") */
    DRESSI_ERR_NO_DEVICE = -3,   /* no usable HIP device */
    DRESSI_ERR_UNSUPPORTED = -4  /* configuration outside what is built */
} dressi_status;

/* Message of the last failing call on this thread ("" if none). */
const char* dressi_last_error(void);
/* Library version string. */
const char* dressi_version(void);

/* ------------------------------------------------------------------------ */
/* Context, memory, transfers                                               */
/* ------------------------------------------------------------------------ */
typedef struct dressi_ctx dressi_ctx;

/* Creates a context on `device` with its own default-priority stream.
 * Replaces DressiAD::createContext / CreateVkContext
 * (include/dressi/dressi_ad.h:53-55, src/vk/context.h:11-40). */
int dressi_ctx_create(int device, dressi_ctx** out);
int dressi_ctx_destroy(dressi_ctx* ctx);
/* Use a caller-owned stream (e.g. the current torch stream) instead of the
 * context's own, which is non-blocking. NULL selects the device's null
 * stream, the handle torch reports for its default stream.
 * dressi_ctx_reset_stream restores the context's own stream. */
int dressi_ctx_set_stream(dressi_ctx* ctx, void* stream);
int dressi_ctx_reset_stream(dressi_ctx* ctx);
void* dressi_ctx_stream(dressi_ctx* ctx);
/* Waits for all work queued on the context stream (the reference's fence
 * wait, src/vk/executor.cpp:1020-1027). */
int dressi_ctx_synchronize(dressi_ctx* ctx);
/* Generation of the context's per-op workspaces: it changes whenever a call
 * needs a larger workspace than the context holds and the old one is freed.
 * Device addresses taken from the workspaces (e.g. captured into a hipGraph)
 * are valid only while it stays the same. No reference counterpart (the
 * reference's GpuPlan owns fixed images, src/vk/executor.h:16-38). */
uint64_t dressi_ctx_workspace_generation(dressi_ctx* ctx);
/* Device name (DressiAD::getDeviceName, include/dressi/dressi_ad.h:94-96). */
int dressi_ctx_device_name(dressi_ctx* ctx, char* buf, size_t len);

int dressi_malloc(dressi_ctx* ctx, void** ptr, size_t bytes);
int dressi_free(dressi_ctx* ctx, void* ptr);
/* Stream-ordered copies; the *_sync variants wait for completion.
 * Replace SendImageToDevice / ReceiveImageFromDevice (src/vk/transfer.h:16-91). */
int dressi_memcpy_h2d(dressi_ctx* ctx, void* dst, const void* src, size_t bytes);
int dressi_memcpy_d2h(dressi_ctx* ctx, void* dst, const void* src, size_t bytes);
int dressi_memset(dressi_ctx* ctx, void* dst, int value, size_t bytes);

/* ------------------------------------------------------------------------ */
/* Per-op kernels (device pointers, stream-ordered on the context stream).  */
/* Each reproduces one reference op's CPU semantics exactly.                */
/* ------------------------------------------------------------------------ */

/* F::SoftClip (src/core/f_ops.cpp:1890-1981; GLSL glsl_codegen.cpp:1440-1491):
 * clip {V,1} VEC4, faces {F,1} float VEC3 -> out {3F,1} VEC4. */
int dressi_soft_clip(dressi_ctx* ctx, const float* clip, uint32_t n_verts,
                     const float* faces, uint32_t n_faces, uint32_t width,
                     uint32_t height, float radius_px, float* out);

/* F::RasterizeSoft and its peel overload (src/core/f_ops.cpp:1362-1465,
 * CPU RasterizeSoftCpu src/core/cpu_raster.cpp:241-355; raster stage
 * src/vk/executor.cpp:347-498): tile-binned, depth | face-id resolved
 * per pixel with the reference's tie rule. out {S,S} VEC4 =
 * (signed_dist_px, face_id, hard_z, coverage), background 0.
 * soft_clip {3F,1} VEC4, face_id {3F,1}, faces_soft {F,1} float VEC3,
 * hard_clip {V,1} VEC4, faces_tex {F,1} float VEC3; prev_shifted_depth
 * {S,S} or NULL. */
int dressi_rasterize_soft(dressi_ctx* ctx, const float* soft_clip,
                          const float* face_id, const float* faces_soft,
                          const float* hard_clip, uint32_t n_verts,
                          const float* faces_tex, uint32_t n_faces,
                          uint32_t width, uint32_t height, float radius_px,
                          const float* prev_shifted_depth, float* out);

/* dressi_rasterize_soft without any allocation: no counterpart in the
 * reference. For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments and results as dressi_rasterize_soft; its face records and
 * tile bins live in one fixed 32 MiB device array per GPU instead of the
 * context workspace, so a call needs 256-byte-aligned 176 B + 16 B per face
 * plus 4100 B per 16x16 tile (+256) within 32 MiB (e.g. a 1024x1024 screen
 * with up to ~79k faces) and returns DRESSI_ERR_INVALID beyond that. Every
 * call on one GPU shares that GPU's array: host calls (from any thread)
 * are taken one at a time, and a call on another stream than the GPU's
 * previous call waits for that call's work first. A call made while its
 * stream is captured into a graph is not ordered that way: replays of such
 * a graph race with every other call on the GPU. */
int dressi_rasterize_soft_noalloc(dressi_ctx* ctx, const float* soft_clip,
                                  const float* face_id, const float* faces_soft,
                                  const float* hard_clip, uint32_t n_verts,
                                  const float* faces_tex, uint32_t n_faces,
                                  uint32_t width, uint32_t height, float radius_px,
                                  const float* prev_shifted_depth, float* out);

/* F::Rasterize (src/core/f_ops.cpp:1182-1207, CPU RasterizeHardCpu
 * src/core/cpu_raster.cpp:195-225): depth-tested, perspective-correct
 * attribute interpolation; out {S,S} x n_comp, background 0. */
int dressi_rasterize(dressi_ctx* ctx, const float* clip, uint32_t n_verts,
                     const float* attr, uint32_t n_comp, const float* faces,
                     uint32_t n_faces, uint32_t width, uint32_t height,
                     float* out);

/* F::RasterizeFaceId (src/core/f_ops.cpp:2183-2209, CPU
 * RasterizeFaceIdCpu src/core/cpu_raster.cpp:357-369): float(f)+1, 0 bg. */
int dressi_rasterize_face_id(dressi_ctx* ctx, const float* clip,
                             uint32_t n_verts, const float* faces,
                             uint32_t n_faces, uint32_t width,
                             uint32_t height, float* out);
/* A batch of F::Rasterize in one pass: n_items clip sets clip
 * {n_items, n_verts} x 4 over one face list, attributes shared by the items
 * (attr_per_item 0: {n_verts} x n_comp) or one set per item (1:
 * {n_items, n_verts} x n_comp); out {n_items, S, S} x n_comp, each item's
 * image equal to dressi_rasterize's. face_id (optional, NULL to skip)
 * {n_items, S, S} gets dressi_rasterize_face_id's image of each item from
 * the same pass. No counterpart in the reference (its torch surface batches
 * through one engine graph per batch): the batch entry the torch surface's
 * rasterize uses. */
int dressi_rasterize_batch(dressi_ctx* ctx, const float* clip, uint32_t n_verts,
                           uint32_t n_items, const float* attr, uint32_t n_comp,
                           int attr_per_item, const float* faces, uint32_t n_faces,
                           uint32_t width, uint32_t height, float* out,
                           float* face_id);

/* F::LookupFaces forward / backward (src/core/f_ops.cpp:1521-1619):
 * out{F} = attr[faces[f][corner]]; bwd: per vertex, rows d ascending of
 * vtx_faces {V,max_deg} whose face has the vertex at `corner`. */
int dressi_lookup_faces(dressi_ctx* ctx, const float* attr, uint32_t n_comp,
                        uint32_t n_attr, const float* faces, uint32_t n_faces,
                        uint32_t corner, float* out);
int dressi_lookup_faces_bwd(dressi_ctx* ctx, const float* gy, uint32_t n_comp,
                            const float* faces, uint32_t n_faces,
                            const float* vtx_faces, uint32_t n_verts,
                            uint32_t max_deg, uint32_t corner, float* out);

/* F::FaceFetch forward / backward (src/core/f_ops.cpp:1631-1799; hash
 * :1473-1487). bwd: n_samples > 0 the stochastic Wang-hash edge-sample
 * gather seeded by `seed` (read from device memory, {1,1}), n_samples == 0
 * the exact bbox+-1 scan. */
int dressi_face_fetch(dressi_ctx* ctx, const float* attr, uint32_t n_comp,
                      uint32_t n_faces, const float* idx, uint32_t width,
                      uint32_t height, float* out);
int dressi_face_fetch_bwd(dressi_ctx* ctx, const float* gy, uint32_t n_comp,
                          const float* idx, uint32_t width, uint32_t height,
                          const float* prj0, const float* prj1,
                          const float* prj2, uint32_t n_faces,
                          const float* seed, float radius_px,
                          uint32_t n_samples, float* out);

/* Batched forms of the four entry points above (an extension with no
 * counterpart in the reference: the torch surface's interpolate runs a whole
 * batch per launch). n_items items back to back: attr [item][n_attr] (or
 * [item][n_faces] for FaceFetch) when attr_per_item, else shared; idx and gy
 * images [item][H][W] (x n_comp); prj* [item][F] VEC4 when prj_per_item;
 * seeds [item] (device); gy of LookupFacesBwd [item][F]; outputs [item][...]
 * of the single-item shape. Each item's result equals the single-item
 * call's. n_items <= 65535. */
int dressi_lookup_faces_batch(dressi_ctx* ctx, const float* attr,
                              uint32_t n_comp, uint32_t n_attr,
                              int attr_per_item, const float* faces,
                              uint32_t n_faces, uint32_t corner,
                              uint32_t n_items, float* out);
int dressi_lookup_faces_bwd_batch(dressi_ctx* ctx, const float* gy,
                                  uint32_t n_comp, const float* faces,
                                  uint32_t n_faces, const float* vtx_faces,
                                  uint32_t n_verts, uint32_t max_deg,
                                  uint32_t corner, uint32_t n_items,
                                  float* out);
int dressi_face_fetch_batch(dressi_ctx* ctx, const float* attr,
                            uint32_t n_comp, uint32_t n_faces,
                            int attr_per_item, const float* idx,
                            uint32_t width, uint32_t height, uint32_t n_items,
                            float* out);
int dressi_face_fetch_bwd_batch(dressi_ctx* ctx, const float* gy,
                                uint32_t n_comp, const float* idx,
                                uint32_t width, uint32_t height,
                                const float* prj0, const float* prj1,
                                const float* prj2, int prj_per_item,
                                uint32_t n_faces, const float* seeds,
                                float radius_px, uint32_t n_samples,
                                uint32_t n_items, float* out);

/* F::AntiAlias (src/core/f_ops.cpp:2480-2579; pair rule EvalAaPair,
 * src/core/cpu_raster.cpp:371-454): 8-neighbour screen-space antialiasing of
 * img {S,S} x n_comp (n_comp 1..4) given the face-id image tri {S,S} (float
 * face + 1, 0 bg), clip {V,1} VEC4 and faces {F,3} float ids.
 * c_aa = (c + sum_k [r c + (1 - r) c_n]) / 9. */
int dressi_antialias(dressi_ctx* ctx, const float* img, uint32_t n_comp,
                     const float* tri, const float* clip, uint32_t n_verts,
                     const float* faces, uint32_t n_faces, uint32_t width,
                     uint32_t height, float* out);
/* AntiAliasBwdImg (src/core/f_ops.cpp:2220-2278): d c_aa / d img applied to
 * gy {S,S} x n_comp. */
int dressi_antialias_bwd_img(dressi_ctx* ctx, const float* gy, uint32_t n_comp,
                             const float* tri, const float* clip,
                             uint32_t n_verts, const float* faces,
                             uint32_t n_faces, uint32_t width,
                             uint32_t height, float* out);
/* AntiAliasBwdVtx (src/core/f_ops.cpp:2284-2476): d c_aa / d clip applied
 * to gy. n_samples > 0: the stochastic gather seeded by `seed` (device
 * {1,1}); wide != 0 writes the {V, max_deg} VEC4 partials (row d * V + v, the
 * input of ColSum), else {V,1}. n_samples == 0: the exact sum over every
 * boundary pair, {V,1} VEC4 (wide must be 0). vtx_faces {V,max_deg} float,
 * -1 pad (VertexFacesTex). */
int dressi_antialias_bwd_vtx(dressi_ctx* ctx, const float* gy, const float* img,
                             uint32_t n_comp, const float* tri,
                             const float* clip, uint32_t n_verts,
                             const float* faces, uint32_t n_faces,
                             const float* vtx_faces, uint32_t max_deg,
                             const float* seed, uint32_t n_samples, int wide,
                             uint32_t width, uint32_t height, float* out);
/* F::ColSum (src/core/f_ops.cpp:1218-1246): {W,H} x n_comp -> {W,1}, rows
 * summed in order. */
int dressi_col_sum(dressi_ctx* ctx, const float* x, uint32_t n_comp,
                   uint32_t width, uint32_t height, float* out);

/* Batched forms of the four entry points above (an extension with no
 * counterpart in the reference, which evaluates one image per graph: the
 * torch surface's antialias runs a whole batch per launch). n_items images
 * back to back ([item][H][W] x n_comp, face ids [item][H][W]); clip is
 * [item][V] VEC4 when clip_per_item, else one {V,1} shared by the items;
 * seeds [item] (device); outputs [item][...] of the single-item shape. Each
 * item's result equals the single-item call's. n_items <= 65535. */
int dressi_antialias_batch(dressi_ctx* ctx, const float* img, uint32_t n_comp,
                           const float* tri, const float* clip, uint32_t n_verts,
                           int clip_per_item, const float* faces,
                           uint32_t n_faces, uint32_t width, uint32_t height,
                           uint32_t n_items, float* out);
int dressi_antialias_bwd_img_batch(dressi_ctx* ctx, const float* gy,
                                   uint32_t n_comp, const float* tri,
                                   const float* clip, uint32_t n_verts,
                                   int clip_per_item, const float* faces,
                                   uint32_t n_faces, uint32_t width,
                                   uint32_t height, uint32_t n_items,
                                   float* out);
int dressi_antialias_bwd_vtx_batch(dressi_ctx* ctx, const float* gy,
                                   const float* img, uint32_t n_comp,
                                   const float* tri, const float* clip,
                                   uint32_t n_verts, int clip_per_item,
                                   const float* faces, uint32_t n_faces,
                                   const float* vtx_faces, uint32_t max_deg,
                                   const float* seeds, uint32_t n_samples,
                                   int wide, uint32_t width, uint32_t height,
                                   uint32_t n_items, float* out);
int dressi_col_sum_batch(dressi_ctx* ctx, const float* x, uint32_t n_comp,
                         uint32_t width, uint32_t height, uint32_t n_items,
                         float* out);

/* GatherDistGrad (src/core/f_ops.cpp:1248-1358), the exact backward of
 * RasterizeSoft's dist channel w.r.t. the hard clip positions (RasterizeSoft's
 * own backward is ColSum of the wide form, f_ops.cpp:1448-1455): for every
 * covered pixel of rs {S,S} VEC4 with gy.x != 0 (gy {S,S} VEC4), the
 * argmin-edge gradient of its face's signed distance (envelope theorem)
 * through the screen -> clip Jacobian. wide != 0: out {max_deg, V} VEC4, the
 * contribution of face f to vertex u in u's adjacency row holding f; else
 * out {V,1} VEC4. vtx_faces {V,max_deg} float (-1 pad). As on the
 * reference's GPU path, radius_px bounds each face's pixel scan by its soft
 * triangle's bbox: rs must be RasterizeSoft's output for these clips. */
int dressi_gather_dist_grad(dressi_ctx* ctx, const float* gy, const float* rs,
                            const float* clip, uint32_t n_verts,
                            const float* faces, uint32_t n_faces,
                            const float* vtx_faces, uint32_t max_deg,
                            float radius_px, int wide, uint32_t width,
                            uint32_t height, float* out);

/* ---- split-sum IBL ops (C5) ---- */
/* Maps are equirectangular {w,h} x n_comp (1..4) float images, row 0 at the
 * +Y pole; directions are {dw,dh} VEC3 (any length; zero-length samples 0).
 * Texel-centre directions follow DirFromEquirectUv (src/core/ibl_math.h:
 * 48-54) with the C library's sinf / cosf, so the dense convolutions match
 * the reference's CPU sums bit for bit; per-direction uv use atan2 / acos
 * rounded once (the reference's float library calls can differ by an ulp). */
/* F::EquirectSample (src/core/f_ops.cpp:2921-2964, BilerpWrap
 * src/core/ibl_math.h:58-89): u wraps, v clamps -> out {dw,dh} x n_comp. */
int dressi_equirect_sample(dressi_ctx* ctx, const float* map, uint32_t mw,
                           uint32_t mh, uint32_t n_comp, const float* dir,
                           uint32_t dw, uint32_t dh, float* out);
/* Its VJP w.r.t. the map (EquirectSampleBwd + TileSum, f_ops.cpp:2786-2919):
 * gy {dw,dh} x n_comp -> out {mw,mh} x n_comp, summed in 64-bit fixed point
 * (exact, deterministic). */
int dressi_equirect_sample_bwd(dressi_ctx* ctx, const float* gy,
                               uint32_t n_comp, const float* dir, uint32_t dw,
                               uint32_t dh, uint32_t mw, uint32_t mh,
                               float* out);
/* F::AvgPool2x2 = Reduce2x2Sum * 0.25 (f_ops.cpp:996-1033, 3411-3415):
 * x {w,h} -> out {ceil(w/2), ceil(h/2)}; _bwd: gy {ceil(w/2),ceil(h/2)} ->
 * out {w,h} (UpsampleNearest2x of gy * 0.25, f_ops.cpp:958-994). */
int dressi_avg_pool2x2(dressi_ctx* ctx, const float* x, uint32_t w, uint32_t h,
                       uint32_t n_comp, float* out);
int dressi_avg_pool2x2_bwd(dressi_ctx* ctx, const float* gy, uint32_t w,
                           uint32_t h, uint32_t n_comp, float* out);
/* F::IrradianceConv (f_ops.cpp:3006-3087): env {sw,sh} -> out {ow,oh};
 * _bwd: its transpose IrradianceConvBwd (f_ops.cpp:2970-3004),
 * gy {ow,oh} -> out {sw,sh}. */
int dressi_irradiance_conv(dressi_ctx* ctx, const float* env, uint32_t sw,
                           uint32_t sh, uint32_t n_comp, uint32_t ow,
                           uint32_t oh, float* out);
int dressi_irradiance_conv_bwd(dressi_ctx* ctx, const float* gy, uint32_t ow,
                               uint32_t oh, uint32_t n_comp, uint32_t sw,
                               uint32_t sh, float* out);
/* F::PrefilterConv at roughness r (alpha = max(r, 0.045)^2): its normaliser
 * PrefilterConvNorm (f_ops.cpp:3166-3205) -> norm {ow,oh} FLOAT; the
 * convolution (f_ops.cpp:3264-3348) env {sw,sh} -> out {ow,oh}; its
 * transpose PrefilterConvBwd (f_ops.cpp:3207-3262) gy {ow,oh} -> out {sw,sh}. */
int dressi_prefilter_conv_norm(dressi_ctx* ctx, uint32_t ow, uint32_t oh,
                               uint32_t sw, uint32_t sh, float roughness,
                               float* norm);
int dressi_prefilter_conv(dressi_ctx* ctx, const float* env, uint32_t sw,
                          uint32_t sh, uint32_t n_comp, uint32_t ow,
                          uint32_t oh, float roughness, const float* norm,
                          float* out);
int dressi_prefilter_conv_bwd(dressi_ctx* ctx, const float* gy, uint32_t ow,
                              uint32_t oh, uint32_t n_comp, uint32_t sw,
                              uint32_t sh, float roughness, const float* norm,
                              float* out);
/* F::PrefilterEnv (f_ops.cpp:3089-3157): GGX importance-sampled prefilter
 * with n_samples Hammersley samples, forward only -> out {ow,oh}. */
int dressi_prefilter_env(dressi_ctx* ctx, const float* env, uint32_t sw,
                         uint32_t sh, uint32_t n_comp, uint32_t ow,
                         uint32_t oh, float roughness, uint32_t n_samples,
                         float* out);
/* F::BrdfIntegrationLut (f_ops.cpp:3350-3409): out {w,h} VEC2 (A, B). */
int dressi_brdf_lut(dressi_ctx* ctx, uint32_t w, uint32_t h,
                    uint32_t n_samples, float* out);

/* ---- the fused PBR / IBL fit plan (C5) ---- */
/* The material + environment fit of examples/common/pbr_graph.cpp (shading,
 * normal mapping off, AO 1, emissive 0) with the maps of src/core/ibl.cpp
 * (irradiance 32 x 16 from the env pooled to <= 64 x 32; `levels`
 * PrefilterConv levels from <= 128 x 64, roughness i / (levels - 1); BRDF
 * LUT 256^2 x 512), the L1 loss Mean(|target - pred|) of the Reinhard-mapped
 * image summed over views, and in-graph Adam on the albedo and metallic-
 * roughness textures (clamped to [0,1], as examples/pbr_material_optimization/
 * run.cpp:285-288) and the env (>= 0, as examples/pbr_envmap_optimization/
 * run.cpp:312-317) with one shared step counter. Replaces DressiAD::execStep
 * on that graph (src/dressi_ad.cpp:280-530). Geometry and cameras are static:
 * set_scene precomputes every geometry-only term per view; one step runs the
 * IBL maps, shading forward + backward, the map transposes and Adam. The
 * material gradients are GatherByInverseUVBilinear (f_ops.cpp:2650-2732) of
 * the per-pixel gradients, as a static per-texel gather list. */
typedef struct dressi_pbr_plan dressi_pbr_plan;

typedef struct dressi_pbr_desc {
    uint32_t n_verts, n_faces;
    uint32_t n_views;     /* 1..16 */
    uint32_t width;       /* screen S (square: width == height) */
    uint32_t height;
    uint32_t tex_w, tex_h;  /* albedo / mr textures */
    uint32_t env_w, env_h;  /* equirect env */
    uint32_t levels;      /* prefiltered levels, 2..8 */
    float lr, beta1, beta2, eps;
    uint32_t flags;       /* DRESSI_PBR_* */
} dressi_pbr_desc;

/* keep the predicted (mapped) images of the last step */
#define DRESSI_PBR_KEEP_PRED 1u
/* keep the last step's texture and env gradients */
#define DRESSI_PBR_KEEP_GRAD 2u

int dressi_pbr_create(dressi_ctx* ctx, const dressi_pbr_desc* desc,
                      dressi_pbr_plan** out);
int dressi_pbr_destroy(dressi_pbr_plan* plan);
/* host arrays: pos / normal {V,3}, uv {V,2}, faces {F,3} (float ids),
 * mvps {N,16} column-major, frames {N,12} (cam_pos, cam_fwd,
 * cam_right * tan(fov/2) * aspect, cam_up * tan(fov/2); PbrFrameLeaves,
 * examples/common/pbr_graph.h:46-53), light {6} (position, colour) */
int dressi_pbr_set_scene(dressi_pbr_plan* plan, const float* pos,
                         const float* normal, const float* uv,
                         const float* faces, const float* mvps,
                         const float* frames, const float* light);
/* dressi_pbr_set_scene with each view's clip positions given, clips {N,V,4}
 * view-major, instead of MVP * pos: the example graph's per-view
 * sendImg(clip) (pbr_material_optimization/run.cpp:189-236). No reference
 * counterpart as a call: what DressiAD's route of that graph uses. */
int dressi_pbr_set_scene_clips(dressi_pbr_plan* plan, const float* pos,
                               const float* normal, const float* uv,
                               const float* faces, const float* clips,
                               const float* frames, const float* light);
/* renders the static targets from the ground-truth maps (host VEC3:
 * gt_albedo / gt_mr {tex_h, tex_w, 3}, gt_env {env_h, env_w, 3}); the state
 * must be (re)set afterwards */
int dressi_pbr_set_target(dressi_pbr_plan* plan, const float* gt_albedo,
                          const float* gt_mr, const float* gt_env);
/* parameters (host VEC3, as above), Adam moments cleared, step counter t */
int dressi_pbr_set_state(dressi_pbr_plan* plan, const float* albedo,
                         const float* mr, const float* env, float t);
int dressi_pbr_get_state(dressi_pbr_plan* plan, float* albedo, float* mr,
                         float* env, float* t);
/* The Adam moments m / v of albedo, mr {tex_h, tex_w, 3} and env
 * {env_h, env_w, 3} (host VEC3), in and out: the in-graph Adam's state
 * leaves (addUpdate of run.cpp's optimizer); set after dressi_pbr_set_state,
 * which clears them. No reference counterpart as a call. */
int dressi_pbr_set_adam(dressi_pbr_plan* plan, const float* m_albedo,
                        const float* v_albedo, const float* m_mr,
                        const float* v_mr, const float* m_env,
                        const float* v_env);
int dressi_pbr_get_adam(dressi_pbr_plan* plan, float* m_albedo,
                        float* v_albedo, float* m_mr, float* v_mr,
                        float* m_env, float* v_env);
/* n_iters iterations (a captured hipGraph, replayed) / eager launches */
int dressi_pbr_step(dressi_pbr_plan* plan, uint32_t n_iters);
int dressi_pbr_step_eager(dressi_pbr_plan* plan, uint32_t n_iters);
enum {
    DRESSI_PBR_LOSS = 0,     /* float: the last step's loss */
    DRESSI_PBR_PRED = 1,     /* {N,S,S} float4 mapped rgb (KEEP_PRED) */
    DRESSI_PBR_TARGET = 2,   /* {N,S,S} float4 mapped rgb */
    DRESSI_PBR_G_ALBEDO = 3, /* {T} float4 (KEEP_GRAD) */
    DRESSI_PBR_G_MR = 4,     /* {T} float4 (KEEP_GRAD) */
    DRESSI_PBR_G_ENV = 5,    /* {E} float4 (KEEP_GRAD) */
    DRESSI_PBR_IRR = 6,      /* {32 x 16} float4: the last step's irradiance map */
    DRESSI_PBR_PREF = 7,     /* float4: the prefiltered levels, level-major */
    DRESSI_PBR_GBUF0 = 8     /* {N,S,S} float4 static G-buffer word 0: material
                                uv, n.v, n.l; n.v < 0 marks a background pixel,
                                whose (u, v) is its env lookup (u < 0: none) */
};
int dressi_pbr_buffer(dressi_pbr_plan* plan, int which, void** ptr,
                      size_t* bytes);
int dressi_pbr_read(dressi_pbr_plan* plan, int which, void* host,
                    size_t bytes);
/* in-place eager iterations with a HIP event around each kernel: average
 * microseconds per kernel (the pooling chain counts as one) */
int dressi_pbr_profile(dressi_pbr_plan* plan, uint32_t iters, char* names,
                       size_t name_stride, float* usec, uint32_t cap,
                       uint32_t* n);

/* ---- texture path (C3) ---- */
/* F::TextureBilinear forward (src/core/f_ops.cpp:2736-2780, BilerpClamp
 * src/core/ibl_math.h:91-115): tex {tw,th} x n_comp (1..4) sampled at
 * uv {uw,uh} VEC2 (4-tap, clamp to edge, texel centres at +0.5) ->
 * out {uw,uh} x n_comp. */
int dressi_texture_bilinear(dressi_ctx* ctx, const float* tex, uint32_t tw,
                            uint32_t th, uint32_t n_comp, const float* uv,
                            uint32_t uw, uint32_t uh, float* out);
/* Its backward w.r.t. the texture, GatherByInverseUVBilinear
 * (src/core/f_ops.cpp:2650-2732): per texel the inverse-UV anchor (its own
 * entry of inv_uv {tw,th} VEC4 when .z > 0.5, else the first such entry of
 * the +-4 neighbourhood in row order) and the tent-weighted sum of gy
 * {sw,sh} x n_comp over the 7 x 7 screen pixels around it, weights from
 * uv {sw,sh} VEC2. out {tw,th} x n_comp. */
int dressi_texture_bilinear_bwd(dressi_ctx* ctx, const float* gy,
                                uint32_t n_comp, uint32_t sw, uint32_t sh,
                                const float* inv_uv, uint32_t tw, uint32_t th,
                                const float* uv, float* out);
/* F::Texture forward, nearest (src/core/f_ops.cpp:2605-2639; the reference
 * has only its GLSL texture() read through a nearest, clamp-to-edge sampler,
 * src/vk/executor.cpp:192-202): tex {tw,th} x n_comp (1..4) at texel
 * (clamp(floor(u tw), 0, tw - 1), clamp(floor(v th), 0, th - 1)) for each
 * uv {uw,uh} VEC2 -> out {uw,uh} x n_comp. */
int dressi_texture_nearest(dressi_ctx* ctx, const float* tex, uint32_t tw,
                           uint32_t th, uint32_t n_comp, const float* uv,
                           uint32_t uw, uint32_t uh, float* out);
/* Its backward w.r.t. the texture, GatherByInverseUV (f_ops.cpp:2586-2601,
 * GLSL src/codegen/glsl_codegen.cpp:657-703): per texel the inverse-UV
 * anchor (as for the bilinear gather), then the first screen pixel of the
 * 7 x 7 window around it (row order) whose uv truncates to the texel gives
 * its gradient gy {sw,sh} x n_comp (zero when none). out {tw,th} x n_comp. */
int dressi_texture_nearest_bwd(dressi_ctx* ctx, const float* gy,
                               uint32_t n_comp, uint32_t sw, uint32_t sh,
                               const float* inv_uv, uint32_t tw, uint32_t th,
                               const float* uv, float* out);
/* ScreenAttr (src/core/mesh_utils.cpp:191-203) on the device: clip {V,1}
 * VEC4 -> {V,1} VEC4 (screen x, screen y, 1, 0). */
int dressi_screen_attr(dressi_ctx* ctx, const float* clip, uint32_t n_verts,
                       uint32_t width, uint32_t height, float* out);

/* ------------------------------------------------------------------------ */
/* Host-side mesh topology and scene builders                               */
/* ------------------------------------------------------------------------ */
/* GenerateUvSphere (examples/common/geometry_utils.cpp:86-131): stacks x
 * slices quads with a duplicated seam column and the pole triangles
 * skipped; pos {V,3}, uv {V,2} (u = j / slices, v = i / stacks), faces
 * {F,3} float ids. Counts only when an output is NULL. */
int dressi_uv_sphere(uint32_t stacks, uint32_t slices, uint32_t* n_verts,
                     uint32_t* n_faces, float* pos, float* uv, float* faces);
/* UvAsClip (src/core/mesh_utils.cpp:180-189): uv {V,2} -> clip {V,4}
 * (2u - 1, 2v - 1, 0.5, 1). */
void dressi_uv_as_clip(const float* uv, uint32_t n_verts, float* clip);
/* GenerateIcosphere (examples/common/geometry_utils.cpp:24-84). Counts only
 * when pos/faces are NULL. pos {V,3}, faces {F,3} float ids. */
int dressi_icosphere(uint32_t level, uint32_t* n_verts, uint32_t* n_faces,
                     float* pos, float* faces);
/* VertexFacesTex (src/core/mesh_utils.cpp:53-71): returns max degree in
 * *max_deg; writes max_deg*V floats when out != NULL and cap suffices. */
int dressi_vertex_faces_tex(const float* faces, uint32_t n_faces,
                            uint32_t n_verts, uint32_t* max_deg, float* out,
                            size_t cap);
/* LookAt / PerspectiveVk / Mul (examples/common/asset_utils.cpp:719-766),
 * column-major. */
void dressi_look_at(const float eye[3], const float center[3],
                    const float up[3], float m[16]);
void dressi_perspective_vk(float fovy_rad, float aspect, float z_near,
                           float z_far, float m[16]);
void dressi_mat4_mul(const float a[16], const float b[16], float r[16]);
/* The single-precision exp the kernels use for F::Sigmoid
 * (src/core/f_ops.cpp:564-575 calls std::exp(float)), evaluated on the host:
 * bit-identical to the C library's expf that the reference CPU evaluator
 * calls, so device sigmoids match the reference exactly. */
float dressi_expf(float x);

/* ------------------------------------------------------------------------ */
/* Fused HardSoftRas silhouette iteration                                   */
/* ------------------------------------------------------------------------ */
/* One plan = the reference's GpuPlan for the silhouette example graph
 * (examples/silhouette_optimization/run.cpp:229-437 with technique
 * hardsoftras, peels = 1, no regularizers): per iteration
 *   clip = MVP_v * pos (per view)            TransformToClipVar
 *   SoftClip, RasterizeSoft (StopGradient)    a5, a6
 *   D = mask * sigmoid(dist * 7 / r), pred = max(cov*step(0,dist), D)
 *   loss = sum_v (target_v - pred_v)^2 / (W*H)  (image)
 *   backward: FaceFetchBwd (n samples, seed = t) + LookupFacesBwd + clip->pos
 *   Adam (b1 .9, b2 .999, eps 1e-8), state copy-back
 * captured once into a hipGraph (zero per-iteration host work).
 * Replaces BuildGpuPlan/ExecuteGpuPlan (src/vk/executor.h:43-66) as driven
 * by DressiAD::execStep (src/dressi_ad.cpp:280-530). */
typedef struct dressi_hsr_plan dressi_hsr_plan;

typedef struct dressi_hsr_desc {
    uint32_t n_verts;     /* V of the optimised mesh */
    uint32_t n_faces;     /* F */
    uint32_t n_views;     /* N (>= 1) */
    uint32_t width;       /* screen S (width == height in the configs) */
    uint32_t height;
    float radius_px;      /* soft radius r (3) */
    uint32_t n_samples;   /* FaceFetchBwd samples per face (8) */
    float lr;             /* Adam learning rate */
    float beta1, beta2, eps; /* 0.9, 0.999, 1e-8 */
    uint32_t flags;       /* DRESSI_HSR_* */
} dressi_hsr_desc;

/* Also write per-view pred images each iteration (markOutput(pred)). */
#define DRESSI_HSR_KEEP_PRED 1u
/* Keep d loss / d pos of the last iteration readable (setGradOutputsEnabled,
 * include/dressi/dressi_ad.h:78-87). */
#define DRESSI_HSR_KEEP_GRAD 2u
/* Technique "aa" of the example (run.cpp:231-238, 352-356) instead of
 * HardSoftRas: pred = AntiAlias(Rasterize(clip, 1), RasterizeFaceId(clip),
 * ...), target = StopGradient(AntiAlias of the target mask), vertex
 * gradients from AntiAliasBwdVtx (wide, n_samples, seed t) + ColSum.
 * radius_px is unused; pred is always kept. */
#define DRESSI_HSR_TECHNIQUE_AA 4u

int dressi_hsr_create(dressi_ctx* ctx, const dressi_hsr_desc* desc,
                      dressi_hsr_plan** out);
int dressi_hsr_destroy(dressi_hsr_plan* plan);

/* Static leaves from host memory (sendImg before the first execStep):
 * faces {F,3} float ids, mvps N x 16 column-major. */
int dressi_hsr_set_mesh(dressi_hsr_plan* plan, const float* faces,
                        const float* mvps);
/* Target silhouettes: either uploaded ({N,S,S}) or rasterised once on the
 * GPU from a target mesh: StopGradient(Rasterize(MVP_v * tgt_pos, ones,
 * tgt_faces)) (run.cpp:347-351). */
int dressi_hsr_set_targets(dressi_hsr_plan* plan, const float* targets);
int dressi_hsr_render_targets(dressi_hsr_plan* plan, const float* tgt_pos,
                              uint32_t n_tverts, const float* tgt_faces,
                              uint32_t n_tfaces);
/* Optimiser state pos/m/v {V,3} and t from host (m, v may be NULL = 0). */
int dressi_hsr_set_state(dressi_hsr_plan* plan, const float* pos,
                         const float* m, const float* v, float t);
int dressi_hsr_get_state(dressi_hsr_plan* plan, float* pos, float* m,
                         float* v, float* t);

/* Enqueue `n_iters` iterations on the context stream (graph launches; no
 * host sync). DressiAD::execStep x n (src/dressi_ad.cpp:280-530). */
int dressi_hsr_step(dressi_hsr_plan* plan, uint32_t n_iters);
/* Same, without the hipGraph (eager launches) -- for tests / profiling. */
int dressi_hsr_step_eager(dressi_hsr_plan* plan, uint32_t n_iters);

/* Buffers readable after a step (recvImg): */
enum dressi_hsr_buffer {
    DRESSI_HSR_LOSS = 0,    /* {S,S} float: the loss image */
    DRESSI_HSR_PRED = 1,    /* {N,S,S} float (needs DRESSI_HSR_KEEP_PRED) */
    DRESSI_HSR_TARGET = 2,  /* {N,S,S} float (read only: set_targets and
                               render_targets are its writers, they also
                               refresh the plan's byte copy of 0 / 1 targets) */
    DRESSI_HSR_FACE_ID = 3, /* {N,S,S} uint32: face + 1 of RasterizeSoft, 0 bg;
                               bit 31 set when the winning fragment lies
                               outside its hard triangle (signed dist < 0).
                               Technique aa: RasterizeFaceId, no flag bit */
    DRESSI_HSR_GRAD = 4,    /* {V,3} float (needs DRESSI_HSR_KEEP_GRAD) */
    DRESSI_HSR_POS = 5      /* {V,3} float */
};
/* Device pointer of a plan buffer (zero-copy access) and its size. */
int dressi_hsr_buffer(dressi_hsr_plan* plan, int which, void** ptr,
                      size_t* bytes);
/* Synchronous copy of a plan buffer to host memory. */
int dressi_hsr_read(dressi_hsr_plan* plan, int which, void* host,
                    size_t bytes);
/* Per-kernel profile of the iteration: `iters` (at most 256) eager
 * iterations with HIP events between their kernels on the plan stream;
 * fills up to `cap` kernel names / average microseconds and returns the
 * kernel count in *n. Advances the optimisation by `iters` steps. */
int dressi_hsr_profile(dressi_hsr_plan* plan, uint32_t iters, char* names,
                       size_t name_stride, float* usec, uint32_t cap,
                       uint32_t* n);
/* Entries per soft bin (a 16x16 tile of one view) of the plan. No
 * counterpart in the reference (its binning is the Vulkan rasteriser's): the
 * bins start at 1024 entries; when an iteration's face backward finds a bin
 * past its capacity (that iteration's raster walked every face of the view
 * there: exact but slow), the next dressi_hsr_step / _step_eager grows them
 * to the next power of two holding that count, at most 16384. For tests and
 * diagnostics. */
int dressi_hsr_bin_capacity(dressi_hsr_plan* plan, uint32_t* entries);

/* ------------------------------------------------------------------------ */
/* Fused texture-optimisation iteration (C3)                                */
/* ------------------------------------------------------------------------ */
/* One plan = the GpuPlan of the texture example's graph
 * (examples/texture_optimization/run.cpp:112-145) with TextureBilinear, an
 * RGBA texture, the RGB L2 image loss and the silhouette example's in-graph
 * Adam (run.cpp:404-437): per iteration and view v, with the cameras of set
 * (t mod n_sets) (the example's per-iteration sendImg of moving views):
 *   clip = MVP * pos, inv_uv_attr = ScreenAttr(clip)
 *   g_uv = Rasterize(clip, uv, S), g_mask = Rasterize(clip, 1, S)
 *   inv_uv = Rasterize(UvAsClip(uv), inv_uv_attr, T)
 *   target = g_mask * TextureBilinear(gt_tex, g_uv, inv_uv)  (StopGradient)
 *   pred   = g_mask * TextureBilinear(tex, g_uv, inv_uv)
 *   loss   = sum_v (target - pred)^2 * (c, c, c, 0), c = 1 / S^2  (image)
 *   backward: GatherByInverseUVBilinear per view, summed over views; Adam
 * captured once into a hipGraph. The UV-space raster (which face covers a
 * texel, and its barycentrics) does not depend on the view and is computed
 * once by set_mesh; each view only interpolates its screen attribute. */
typedef struct dressi_tex_plan dressi_tex_plan;

typedef struct dressi_tex_desc {
    uint32_t n_verts;     /* V */
    uint32_t n_faces;     /* F */
    uint32_t n_views;     /* N views per iteration (1..8) */
    uint32_t width;       /* screen S (square) */
    uint32_t height;
    uint32_t tex_w;       /* texture T */
    uint32_t tex_h;
    uint32_t n_sets;      /* camera sets, iteration t uses set t mod n_sets */
    float lr;             /* Adam learning rate */
    float beta1, beta2, eps;
    uint32_t flags;       /* DRESSI_TEX_* */
} dressi_tex_desc;

/* Also write per-view pred / target images (markOutput). */
#define DRESSI_TEX_KEEP_IMAGES 1u
/* Keep d loss / d tex of the last iteration readable. */
#define DRESSI_TEX_KEEP_GRAD 2u
/* The per-view clip positions and ScreenAttr images are the caller's
 * (dressi_tex_set_clips, before each step that changes them) instead of
 * MVP * pos: the example graph's per-iteration sendImg of each view's
 * clip and inverse-UV attribute (texture_optimization/run.cpp:106-109,
 * 166-178). The cameras are then not used. */
#define DRESSI_TEX_EXTERNAL_CLIP 4u

int dressi_tex_create(dressi_ctx* ctx, const dressi_tex_desc* desc,
                      dressi_tex_plan** out);
int dressi_tex_destroy(dressi_tex_plan* plan);
/* Static leaves (sendImg): pos {V,3}, uv {V,2}, faces {F,3} float ids;
 * computes the UV-space raster. */
int dressi_tex_set_mesh(dressi_tex_plan* plan, const float* pos,
                        const float* uv, const float* faces);
/* Cameras: mvps {n_sets, N, 16} column-major. */
int dressi_tex_set_cameras(dressi_tex_plan* plan, const float* mvps);
/* DRESSI_TEX_EXTERNAL_CLIP: clip {N,V} VEC4 and attrs {N,V} VEC4 =
 * ScreenAttr(clip) (z = 1, w = 0 checked), view-major; synchronous. */
int dressi_tex_set_clips(dressi_tex_plan* plan, const float* clips,
                         const float* attrs);
/* The target texture {T} RGBA (gt_tex). */
int dressi_tex_set_target(dressi_tex_plan* plan, const float* gt_tex);
/* Texture and Adam state {T} RGBA from host (m, v may be NULL = 0). */
int dressi_tex_set_state(dressi_tex_plan* plan, const float* tex,
                         const float* m, const float* v, float t);
int dressi_tex_get_state(dressi_tex_plan* plan, float* tex, float* m,
                         float* v, float* t);
/* Enqueue `n_iters` iterations (graph launches / eager launches). */
int dressi_tex_step(dressi_tex_plan* plan, uint32_t n_iters);
int dressi_tex_step_eager(dressi_tex_plan* plan, uint32_t n_iters);

enum dressi_tex_buffer {
    DRESSI_TEX_LOSS = 0,    /* {S,S} VEC4: the loss image */
    DRESSI_TEX_PRED = 1,    /* {N,S,S} VEC4 (DRESSI_TEX_KEEP_IMAGES) */
    DRESSI_TEX_TARGET = 2,  /* {N,S,S} VEC4 (DRESSI_TEX_KEEP_IMAGES) */
    DRESSI_TEX_FACE_ID = 3, /* {N,S,S} uint32: face + 1 of the screen raster */
    DRESSI_TEX_GRAD = 4,    /* {T} VEC4 (DRESSI_TEX_KEEP_GRAD) */
    DRESSI_TEX_TEX = 5,     /* {T} VEC4: the texture */
    DRESSI_TEX_UV = 6       /* {N,S,S} VEC2: g_uv */
};
int dressi_tex_buffer(dressi_tex_plan* plan, int which, void** ptr,
                      size_t* bytes);
int dressi_tex_read(dressi_tex_plan* plan, int which, void* host,
                    size_t bytes);
/* Per-kernel profile: `iters` (<= 256) eager iterations with HIP events
 * between the kernels; advances the optimisation by `iters` steps. */
int dressi_tex_profile(dressi_tex_plan* plan, uint32_t iters, char* names,
                       size_t name_stride, float* usec, uint32_t cap,
                       uint32_t* n);

#ifdef __cplusplus
}
#endif

#endif /* DRESSI_HIP_H */
