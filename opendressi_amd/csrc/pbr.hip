// pbr.hip -- the fused split-sum PBR / IBL material + environment fit (C5):
// the shading graph of examples/common/pbr_graph.cpp (BuildPbrGBuffer +
// BuildPbrShade, normal mapping off, AO 1, emissive 0), the IBL maps of
// src/core/ibl.cpp built from the optimised environment every iteration, the
// L1 loss on the Reinhard-mapped image summed over views, and in-graph Adam
// on the albedo and metallic-roughness textures (clamped to [0,1]) and the
// environment (clamped to >= 0).
//
// Geometry is static, so everything the shading derives from it alone --
// the G-buffer, n.v / n.l / n.h, the Schlick powers, the equirect uv of the
// normal, the reflection and the background ray, the texture gather's
// inverse-UV windows, the map-gradient gather lists and the convolution
// weights -- is computed once at set-up; an iteration reads those, the
// material taps and the maps.
//
// Every floating-point sum is formed in the reference evaluator's order, so
// the fit reproduces its results bit for bit: the convolutions and their
// transposes add over source / map texels in raster order
// (f_ops.cpp:2970-3348), each EquirectSample VJP adds per band of dir rows in
// pixel order and then the bands in order (EquirectSampleBwd + TileSum,
// f_ops.cpp:2785-2919), views are added in view order, and the texture
// gather adds each view's window sum in view order.
//
// One iteration, 11 kernels + the pooling chain (ceil(log2) levels):
//   k_pbr_pool        env -> pooled sources of the irradiance / prefilter maps
//   k_pbr_conv_fwd    IrradianceConv + every PrefilterConv level (static
//                     weight matrices, one wave per colour channel)
//   k_pbr_shade       per pixel: forward, L1 loss, backward; material
//                     gradients and the map-gradient seeds per pixel
//   k_pbr_map_gather  per (map, view, band, texel): the band's partial of the
//                     EquirectSample VJP from a static list of (pixel, tap)
//   k_pbr_tile_sum    per (map, view, texel): the bands' partials in order
//   k_pbr_view_sum    per map texel: the views' sums in order
//   k_pbr_conv_bwd    the convolutions' transposes onto the pooled sources
//   k_pbr_env_adam    pooling VJPs + background gradient, Adam on the env
//   k_pbr_tex_adam    GatherByInverseUVBilinear as a static gather list per
//                     texel (per-view sums), Adam on albedo and mr
//   k_pbr_loss_blocks the loss's Reduce2x2Sum levels over 16 x 16 blocks of
//                     the shading tiles' partials
//   k_pbr_loss        the loss scalar (the remaining levels, CompSum, the
//                     views' SumPixelWise tree), t + 1
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include <hipcub/hipcub.hpp>

#include "dressi_hip.h"
#include "ibl_core.h"
#include "internal.h"
#include "plan.h"

namespace dressi {
namespace {

constexpr uint32_t kPbrMaxLevels = 8;
constexpr uint32_t kPbrMaxViews = 16;
constexpr uint32_t kPbrMaxPool = 12;
constexpr uint32_t kPbrMaxMaps = kPbrMaxLevels + 2;
constexpr int kShadeTile = 16;       // 16 x 16 pixel tile per shading workgroup
constexpr uint32_t kTileSumLds = 4096;  // float4 partials staged per tile-sum round
constexpr uint32_t kMvRows = 256;         // ordered mat-vec: summation steps per LDS tile
constexpr uint32_t kMvCols = 32;          // ordered mat-vec: columns per workgroup (the lanes
                                          // past kMvCols repeat the first ones' work)
constexpr uint32_t kGatherChunk = 1024;  // map gather: positions staged per round
constexpr uint32_t kGatherChains = 256;   // map gather: buckets per workgroup (1 per thread)
constexpr uint32_t kGatherBands = 64;     // map gather: bands per workgroup
// map gather: a workgroup's cost per chunk in units of one sequential entry
constexpr uint32_t kGatherChunkCost = 163;
constexpr uint32_t kGatherMaxChunks = 32;  // map gather: position chunks per workgroup (bands
                                          // with more positions take position lists)
constexpr uint32_t kGatherTile = 16;      // map gather: texel tile of a position-list workgroup
constexpr uint32_t kBandMode = 0xffffffffu;

// One sampled map of the shading and its EquirectSample VJP's layout: the
// VJP adds, per view, k partial maps over bands of `rows` dir rows each
// (EquirectSampleBwd, f_ops.cpp:2823-2919: k doubles until w h k >= 65536 or
// k reaches the dir image's height) and sums them in band order (TileSum).
// Buckets: (view, band, texel) of the map, from `bucket0`; the view sums sit
// in `tot` from `tot0` (view, texel).
struct MapInfo {
    uint32_t w, h, T;     // map size and texels
    uint32_t k, rows;     // bands per view, dir rows per band
    uint32_t bucket0;     // first bucket (view 0, band 0, texel 0)
    uint32_t tot0;        // first view sum (view 0, texel 0)
    uint32_t kind;        // 0 irradiance, 1 prefilter level `level`, 2 background env
    uint32_t level;
};

// One workgroup of the map gather: the non-empty buckets ml_order[a0 .. a0 +
// na) (at most kGatherChains) of nb consecutive (view, band)s of map m from
// vb0 = view k + band. The bands are walked together in nch chunks: chunk c
// stages positions c P .. c P + P - 1 of each band (LDS slots bi P ..), a
// band's positions being its dir pixels in order (the env: the view's
// background pixels). Chunk c's entries of bucket j are mg_ent[coff[c0 + c na
// + j] .. coff[c0 + c na + j + 1]) (chunk-major, then bucket order, then pixel
// order), each (LDS slot << 2) | tap. f0: the set-up's first-entry table.
// A band with more than kGatherMaxChunks chunks of positions is split by
// texel tile instead (position-list mode, nb = 1, bmo != kBandMode): the
// workgroup's positions are only those its buckets read, in order --
// plist[pl0 .. pl0 + npl) as global pixel indices; at set-up a position's
// index in that list is its rank in the workgroup's bitmap of band positions
// (words bm[bmo ..], with exclusive popcount prefixes wpre[bmo ..]).
struct GatherItem {
    uint32_t m, vb0, nb, P;
    uint32_t a0, na, nch, c0;
    uint32_t f0, npl, pl0, bmo;
};

// Index of band position `pos` in a position-list workgroup's list
__device__ __forceinline__ uint32_t list_rank(const uint32_t* bm, const uint32_t* wpre,
                                              uint32_t bmo, uint32_t pos) {
    const uint32_t w = bm[bmo + (pos >> 5)];
    return wpre[bmo + (pos >> 5)] + (uint32_t)__popc(w & ((1u << (pos & 31u)) - 1u));
}

struct PbrDev {
    uint32_t n_views, S, tw, th, ew, eh, levels;
    uint32_t iw, ih, isw, ish, psw, psh;
    uint32_t lw[kPbrMaxLevels], lh[kPbrMaxLevels], loff[kPbrMaxLevels], n_pref;
    const uint4* ltab;  // per level (w, h, texel offset, 0)
    float alpha[kPbrMaxLevels];
    float lr, b1, b2, eps, inv_n, irr_scale;
    float light_col[3];
    // static per (view, pixel)
    const float4* st0;  // fg: (u, v, n.v, n.l); bg: (bg u, bg v, -1, 0)
    const float4* st1;  // (n.h, (1 - v.h)^5, (1 - n.v)^5, dist^2)
    const float4* st2;  // (irr u, irr v, refl u, refl v); u < 0: zero direction
    float4* target;     // mapped target (rgb)
    // map geometry
    const float4* psdir;  // prefilter source directions + sin(theta)
    const float* pnorm;   // PrefilterConvNorm of every prefilter texel
    const float2* lut;
    uint32_t lutw, luth;
    // static convolution weights, summation index major: wf_* [source][output]
    // (forward), wb_* [output][source] (transposes)
    // stored tile-major: column group g (lanes 64 g .. 64 g + 63) holds its
    // rows r of 64 floats at g * rows * 64 + r * 64
    const float *wf_irr, *wb_irr, *wf_pref, *wb_pref;
    // pooling chain: level k (1-based) has size pw[k] x ph[k]
    uint32_t n_pool, irr_pool, pref_pool;
    uint32_t pw[kPbrMaxPool + 1], ph[kPbrMaxPool + 1];
    float4* pool[kPbrMaxPool + 1];  // pool[0] = env
    // state
    float4 *albedo, *mr, *env;
    float4 *am, *av, *mm, *mv, *em, *ev;
    float* t;
    // per iteration
    float4 *irr, *pref;
    float4 *g_irr, *g_pref, *g_bg, *g_isrc, *g_psrc;
    float4* gyA;   // per pixel (g albedo rgb, g roughness)
    float* gyM;    // per pixel g metallic
    float4* mgA;   // per pixel: fg (d loss / d irradiance sample, 0); bg (d loss / d env sample, 0)
    float4* mgB;   // per fg pixel: (d loss / d prefiltered sample before the level weights, roughness)
    float4* loss_part;  // per shading tile: its |diff| sum (Reduce2x2Sum order)
    float4* loss_blk;   // per 16 x 16 block of shading tiles: its sum (same order)
    float* loss;
    float4* pred;  // KEEP_PRED
    float4 *g_tex_a, *g_tex_m, *g_env;  // KEEP_GRAD
    const uint32_t* csr_off;  // per texel, into csr
    const uint2* csr;         // (global pixel, weight bits)
    // map-gradient gather lists
    const MapInfo* minfo;
    uint32_t n_maps, n_buckets, n_tot;
    const uint32_t* ml_order;  // per (map, view, band) its non-empty buckets, bucket order
    const uint32_t* ml_off;   // per bucket, into the sorted entries (n_buckets + 1)
    const uint32_t* bg_pix;   // per view from bg_base[v]: the background pixels in order
    const uint32_t* plist;    // position-list workgroups' positions (global pixel indices)
    const uint32_t* bg_base;  // per view (n_views + 1)
    const struct GatherItem* gitems;  // the gather's workgroups
    uint32_t n_gitems;
    const uint32_t* coff;     // per item, chunk-major: its buckets' entry runs
    const uint16_t* mg_ent;   // the entries, chunk-major per item
    float4* mpart;            // per bucket (maps with k > 1)
    float4* mtot;             // per (map, view, texel)
    const uint4* tsum_work;   // tile-sum work items (map, view, first texel, texels)
    uint32_t n_tsum;
    uint32_t n_ig, n_pg;      // convolution workgroups: irradiance, prefilter
    uint32_t n_isg, n_psg;    // transposes: irradiance sources, prefilter sources
    const float2* bc_tab;
    uint32_t bc_len;
    uint32_t* done;
    int target_mode;  // render the target: forward only, write `target`
};

__device__ __forceinline__ float4 f4_zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }

__device__ __forceinline__ void fetch4(const Taps& t, const float4* data, float* out3) {
    float a0 = 0.f, a1 = 0.f, a2 = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float4 q = data[t.idx[k]];
        a0 += t.w[k] * q.x;
        a1 += t.w[k] * q.y;
        a2 += t.w[k] * q.z;
    }
    out3[0] = a0;
    out3[1] = a1;
    out3[2] = a2;
}

// ---------------------------------------------------------------------------
// Set-up kernels
// ---------------------------------------------------------------------------

// clip = MVP * (pos, 1), column-major MVP (TransformToClip,
// examples/common/asset_utils.cpp:768-782)
__global__ __launch_bounds__(256) void k_pbr_clip(const float* pos, uint32_t n, const float* mvp,
                                                  float4* clip) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) {
        return;
    }
    const float p[4] = {pos[i * 3 + 0], pos[i * 3 + 1], pos[i * 3 + 2], 1.f};
    float r[4];
#pragma unroll
    for (int row = 0; row < 4; row++) {
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            acc += mvp[k * 4 + row] * p[k];
        }
        r[row] = acc;
    }
    clip[i] = make_float4(r[0], r[1], r[2], r[3]);
}

__device__ __forceinline__ V3f safe_normalize(V3f v) {
    const float s = 1.f / sqrtf(dot3(v, v) + 1e-12f);
    return V3f{v.x * s, v.y * s, v.z * s};
}

// powf(x, 5) as the C library rounds it (x in [0, 1])
__device__ __forceinline__ float pow5(float x) { return libm::pow5f(x); }

// Static per-pixel terms of one view from its G-buffer (BuildPbrGBuffer,
// pbr_graph.cpp:34-45, and the geometry-only part of BuildPbrShade,
// :62-129): the shading normal, view / light / half vectors and their
// clamped dots, the Schlick powers, the equirect uv of the normal, of the
// reflection and of the background ray.
struct StaticArgs {
    const float4* g_uvh;   // {S,S} (u, v, mask, handedness)
    const float* g_n;      // {S,S} VEC3
    const float* g_p;      // {S,S} VEC3
    float frame[12];       // cam_pos, cam_fwd, cam_right, cam_up
    float light_pos[3];
    uint32_t S;
    float4 *st0, *st1, *st2;
};

__global__ __launch_bounds__(256) void k_pbr_static(StaticArgs a) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.S * a.S) {
        return;
    }
    const uint32_t x = i % a.S, y = i / a.S;
    const float4 uvh = a.g_uvh[i];
    const V3f cam = mk3(a.frame[0], a.frame[1], a.frame[2]);
    const V3f fwd = mk3(a.frame[3], a.frame[4], a.frame[5]);
    const V3f right = mk3(a.frame[6], a.frame[7], a.frame[8]);
    const V3f up = mk3(a.frame[9], a.frame[10], a.frame[11]);
    // background ray through the pixel centre (ScreenCoord, ndc)
    const float ndc_x = ((float)x + 0.5f) * (2.f / (float)a.S) - 1.f;
    const float ndc_y = ((float)y + 0.5f) * (2.f / (float)a.S) - 1.f;
    const V3f ray = mk3(fwd.x + right.x * ndc_x - up.x * ndc_y,
                        fwd.y + right.y * ndc_x - up.y * ndc_y,
                        fwd.z + right.z * ndc_x - up.z * ndc_y);
    if (uvh.z == 0.f) {
        float bu = -1.f, bv = 0.f;
        dir_to_equirect(ray, &bu, &bv);
        a.st0[i] = make_float4(bu, bv, -1.f, 0.f);
        a.st1[i] = f4_zero();
        a.st2[i] = f4_zero();
        return;
    }
    const V3f gn = mk3(a.g_n[i * 3 + 0], a.g_n[i * 3 + 1], a.g_n[i * 3 + 2]);
    const V3f gp = mk3(a.g_p[i * 3 + 0], a.g_p[i * 3 + 1], a.g_p[i * 3 + 2]);
    const V3f n = safe_normalize(gn);
    const V3f v = safe_normalize(mk3(cam.x - gp.x, cam.y - gp.y, cam.z - gp.z));
    const V3f tl = mk3(a.light_pos[0] - gp.x, a.light_pos[1] - gp.y, a.light_pos[2] - gp.z);
    const V3f l = safe_normalize(tl);
    const V3f h = safe_normalize(mk3(v.x + l.x, v.y + l.y, v.z + l.z));
    const float ndv0 = dot3(n, v), dd = dot3(tl, tl);
    const float ndl0 = dot3(n, l), ndh0 = dot3(n, h), vdh0 = dot3(v, h);
    const float ndv = ndv0 < 1e-4f ? 1e-4f : ndv0;
    const float dist2 = dd < 1e-4f ? 1e-4f : dd;
    const float ndl = ndl0 < 0.f ? 0.f : ndl0;
    const float ndh = ndh0 < 0.f ? 0.f : ndh0;
    const float vdh = vdh0 < 0.f ? 0.f : vdh0;
    // Reflect(-v, n) = I - (2 dot(n, I)) n
    const V3f I = mk3(-v.x, -v.y, -v.z);
    const float t2 = 2.f * dot3(n, I);
    const V3f refl = mk3(I.x - t2 * n.x, I.y - t2 * n.y, I.z - t2 * n.z);
    float iu = -1.f, iv = 0.f, ru = -1.f, rv = 0.f;
    dir_to_equirect(n, &iu, &iv);
    dir_to_equirect(refl, &ru, &rv);
    a.st0[i] = make_float4(uvh.x, uvh.y, ndv, ndl);
    a.st1[i] = make_float4(ndh, pow5(1.f - vdh), pow5(1.f - ndv), dist2);
    a.st2[i] = make_float4(iu, iv, ru, rv);
}

// GatherByInverseUVBilinear (src/core/f_ops.cpp:2665-2731) as a static list:
// per texel and view, the anchor (own inverse-UV entry, else the first
// covered one of the +-4 neighbourhood in row order) and the 7 x 7 screen
// window around it in row order, keeping the foreground pixels whose tent
// weight is > 0. Pass 0 counts, pass 1 fills (same order).
struct CsrArgs {
    const float4* inv;   // {N,T} inverse-UV tables
    const float2* g_uv;  // {N,S,S} raster uv (0 on the background)
    const float* mask;   // {N,S,S}
    uint32_t n_views, S, tw, th;
    uint32_t* count;     // {T}
    const uint32_t* off; // {T} (pass 1)
    uint2* csr;
};

template <int PASS>
__global__ __launch_bounds__(256) void k_pbr_csr(CsrArgs a) {
    const uint32_t ti = blockIdx.x * blockDim.x + threadIdx.x;
    if (ti >= a.tw * a.th) {
        return;
    }
    const int tx = (int)(ti % a.tw), ty = (int)(ti / a.tw);
    const int tw = (int)a.tw, th = (int)a.th, S = (int)a.S;
    const size_t npx = (size_t)a.S * a.S;
    uint32_t n = 0;
    uint32_t w_at = PASS ? a.off[ti] : 0u;
    for (uint32_t view = 0; view < a.n_views; view++) {
        const float4* inv = a.inv + (size_t)view * a.tw * a.th;
        float4 iv = inv[ti];
        for (int ny = -4; ny <= 4 && iv.z < 0.5f; ny++) {
            for (int nx = -4; nx <= 4; nx++) {
                const int px = tx + nx, py = ty + ny;
                if (px < 0 || py < 0 || px >= tw || py >= th) {
                    continue;
                }
                iv = inv[py * tw + px];
                if (iv.z > 0.5f) {
                    break;
                }
            }
        }
        if (iv.z <= 0.5f) {
            continue;
        }
        const int scx = (int)iv.x, scy = (int)iv.y;
        for (int dy = -3; dy <= 3; dy++) {
            for (int dx = -3; dx <= 3; dx++) {
                const int spx = scx + dx, spy = scy + dy;
                if (spx < 0 || spy < 0 || spx >= S || spy >= S) {
                    continue;
                }
                const size_t p = (size_t)view * npx + (size_t)spy * S + spx;
                const float2 suv = a.g_uv[p];
                const float stx = suv.x * (float)tw - 0.5f;
                const float sty = suv.y * (float)th - 0.5f;
                const float aa = 1.f - fabsf(stx - (float)tx);
                const float bb = 1.f - fabsf(sty - (float)ty);
                const float w = (aa > 0.f ? aa : 0.f) * (bb > 0.f ? bb : 0.f);
                if (w > 0.f && a.mask[p] != 0.f) {
                    if (PASS) {
                        a.csr[w_at++] = make_uint2((uint32_t)p, __float_as_uint(w));
                    }
                    n++;
                }
            }
        }
    }
    if (!PASS) {
        a.count[ti] = n;
    }
}

// The static convolution weights of one map (f_ops.cpp:3006-3087,
// 3207-3348): per (output texel o, source texel s) with output direction
// r_o, source direction d_s and sin(theta_s), c = dot(r_o, d_s) in the
// reference's float order;
//   irradiance: wf = wb = max(c, 0) sin(theta_s)
//   prefilter:  w = GgxConvWeight(c, alpha_o), wf = w sin(theta_s),
//               wb = w / max(norm_o, 1e-12) where w > 0, else 0
// wf is a matrix of rows s, columns o; wb of rows o, columns s (rows: the
// index each ordered sum runs over); both tile-major in column groups of
// kMvCols, zero past the last column. A zero weight adds nothing to a sum of finite
// terms.
__global__ __launch_bounds__(256) void k_pbr_weights(const float4* odir, uint32_t no,
                                                     const float4* sdir, uint32_t ns,
                                                     const float* norm, float* wf, float* wb) {
    const uint32_t o = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t sidx = blockIdx.y;
    if (o >= no) {
        return;
    }
    const float4 r = odir[o];
    const float4 sd = sdir[sidx];
    const float c = r.x * sd.x + r.y * sd.y + r.z * sd.z;
    float f, b;
    if (!norm) {
        f = (c < 0.f ? 0.f : c) * sd.w;
        b = f;
    } else {
        const float w = ggx_conv_weight(c, r.w);
        f = w * sd.w;
        const float nt = norm[o];
        b = w > 0.f ? w / (nt < 1e-12f ? 1e-12f : nt) : 0.f;
    }
    // tile-major: wf rows are sources (no outputs per row), wb rows outputs
    wf[((size_t)(o / kMvCols) * ns + sidx) * kMvCols + (o % kMvCols)] = f;
    wb[((size_t)(sidx / kMvCols) * no + o) * kMvCols + (sidx % kMvCols)] = b;
}

// Keys of the map-gradient gather lists: per (view, pixel) in pixel order,
// per map, per bilinear tap in the reference's order (dy outer, dx inner),
// the bucket (view, band of the pixel's row, tap texel) of the map's
// EquirectSample VJP, or kNoBucket when the pixel adds nothing there (see
// k_pbr_map_gather); the value is (pixel << 2) | tap. A stable sort by key
// then lists every bucket's entries in pixel order.
constexpr uint32_t kNoBucket = 0xffffffffu;

struct ListArgs {
    const float4 *st0, *st2;
    const MapInfo* minfo;
    uint32_t n_maps, n_views, S;
    uint32_t no_key;
    const uint32_t* bg_idx;  // per pixel: its index among its view's background pixels
    uint32_t* keys;
    uint32_t* vals;
    uint32_t* count;
};

__global__ __launch_bounds__(256) void k_pbr_list_keys(ListArgs a) {
    const size_t npx = (size_t)a.S * a.S;
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= npx * a.n_views) {
        return;
    }
    const uint32_t v = (uint32_t)(q / npx);
    const uint32_t p = (uint32_t)(q % npx);
    const uint32_t y = p / a.S;
    const float4 s0 = a.st0[q], s2 = a.st2[q];
    const bool fg = s0.z >= 0.f;
    for (uint32_t m = 0; m < a.n_maps; m++) {
        const MapInfo mi = a.minfo[m];
        bool ok;
        float u, vv;
        if (mi.kind == 0) {
            ok = fg && s2.x >= 0.f;
            u = s2.x;
            vv = s2.y;
        } else if (mi.kind == 1) {
            ok = fg && s2.z >= 0.f;
            u = s2.z;
            vv = s2.w;
        } else {
            ok = !fg && s0.x >= 0.f;
            u = s0.x;
            vv = s0.y;
        }
        const float sx = u * (float)mi.w - 0.5f;
        const float sy = vv * (float)mi.h - 0.5f;
        const int ix = (int)floorf(sx), iy = (int)floorf(sy);
        const uint32_t band = y / mi.rows;
        for (uint32_t k = 0; k < 4; k++) {
            const size_t o = (q * a.n_maps + m) * 4 + k;
            uint32_t key = a.no_key;
            if (ok) {
                int x = ix + (int)(k & 1u);
                if (x < 0) x += (int)mi.w;
                if (x >= (int)mi.w) x -= (int)mi.w;
                int yy = iy + (int)(k >> 1);
                yy = yy < 0 ? 0 : (yy > (int)mi.h - 1 ? (int)mi.h - 1 : yy);
                key = mi.bucket0 + (v * mi.k + band) * mi.T + (uint32_t)yy * mi.w + (uint32_t)x;
                atomicAdd(&a.count[key], 1u);
            }
            a.keys[o] = key;
            a.vals[o] = ((mi.kind == 2 && ok ? a.bg_idx[q] : p) << 2) | k;
        }
    }
}

// The positions of (view, band) vb of a map: pixels pbase .. pbase + npos - 1
// of view v (the env: bg_pix[pbase ..]); a sorted entry's position is its
// value >> 2 minus posoff.
struct BandPos {
    uint32_t v, pbase, npos, posoff;
};

__device__ __forceinline__ BandPos band_pos(const MapInfo& mi, uint32_t vb, uint32_t S,
                                            const uint32_t* bg_base) {
    BandPos r;
    r.v = vb / mi.k;
    if (mi.kind == 2) {
        r.pbase = bg_base[r.v];
        r.npos = bg_base[r.v + 1] - r.pbase;
        r.posoff = 0;
    } else {
        const uint32_t band = vb % mi.k;
        const uint32_t r0 = band * mi.rows < S ? band * mi.rows : S;
        const uint32_t r1 = r0 + mi.rows < S ? r0 + mi.rows : S;
        r.pbase = r0 * S;
        r.npos = (r1 - r0) * S;
        r.posoff = r0 * S;
    }
    return r;
}

// Background pixels that sample the env (zero-length rays excluded), as
// k_pbr_list_keys selects them: flags for their per-view exclusive scan
// (bg_idx), then the per-view lists of their pixels.
__global__ __launch_bounds__(256) void k_pbr_bg_flags(const float4* st0, size_t n, uint32_t* flag) {
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q < n) {
        const float4 s0 = st0[q];
        flag[q] = (!(s0.z >= 0.f) && s0.x >= 0.f) ? 1u : 0u;
    }
}

__global__ __launch_bounds__(256) void k_pbr_bg_fill(const uint32_t* flag, const uint32_t* idx,
                                                     uint32_t npx, uint32_t base, uint32_t* bg_pix) {
    const uint32_t p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p < npx && flag[p]) {
        bg_pix[base + idx[p]] = p;
    }
}

// Position-list workgroups, step 1: the band positions their buckets' sorted
// entries read, as bits of the workgroup's bitmap (cleared before).
__global__ __launch_bounds__(256) void k_pbr_list_bits(const GatherItem* items, uint32_t n_items,
                                                       const MapInfo* minfo, uint32_t S,
                                                       const uint32_t* bg_base,
                                                       const uint32_t* order, const uint32_t* off,
                                                       const uint32_t* ent, uint32_t* bm) {
    const uint32_t it = blockIdx.y;
    if (it >= n_items) {
        return;
    }
    const GatherItem g = items[it];
    const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
    if (g.bmo == kBandMode || j >= g.na) {
        return;
    }
    const MapInfo mi = minfo[g.m];
    const uint32_t b = order[g.a0 + j];
    const BandPos bp = band_pos(mi, (b - mi.bucket0) / mi.T, S, bg_base);
    for (uint32_t e = off[b]; e < off[b + 1]; e++) {
        const uint32_t pos = (ent[e] >> 2) - bp.posoff;
        atomicOr(&bm[g.bmo + (pos >> 5)], 1u << (pos & 31u));
    }
}

// Step 2, one workgroup per item: the exclusive popcount prefix of every
// bitmap word and the list length npl[item].
__global__ __launch_bounds__(256) void k_pbr_list_count(const GatherItem* items,
                                                        uint32_t n_items, const MapInfo* minfo,
                                                        uint32_t S, const uint32_t* bg_base,
                                                        const uint32_t* bm, uint32_t* wpre,
                                                        uint32_t* npl) {
    __shared__ uint32_t sc[256];
    const uint32_t it = blockIdx.x;
    if (it >= n_items) {
        return;
    }
    const GatherItem g = items[it];
    if (g.bmo == kBandMode) {
        return;
    }
    const MapInfo mi = minfo[g.m];
    const uint32_t words = (band_pos(mi, g.vb0, S, bg_base).npos + 31u) / 32u;
    const uint32_t t = threadIdx.x;
    uint32_t carry = 0;
    for (uint32_t w0 = 0; w0 < words; w0 += 256u) {
        const uint32_t c = w0 + t < words ? (uint32_t)__popc(bm[g.bmo + w0 + t]) : 0u;
        sc[t] = c;
        __syncthreads();
        // inclusive Hillis-Steele scan
        for (uint32_t o = 1; o < 256u; o <<= 1) {
            const uint32_t add = t >= o ? sc[t - o] : 0u;
            __syncthreads();
            sc[t] += add;
            __syncthreads();
        }
        if (w0 + t < words) {
            wpre[g.bmo + w0 + t] = carry + sc[t] - c;
        }
        carry += sc[255];
        __syncthreads();
    }
    if (t == 0) {
        npl[it] = carry;
    }
}

// Step 3: the lists themselves, in band-position order, as global pixel
// indices (view base + the position's pixel, the env's via bg_pix).
__global__ __launch_bounds__(256) void k_pbr_list_fill(const GatherItem* items, uint32_t n_items,
                                                       const MapInfo* minfo, uint32_t S,
                                                       const uint32_t* bg_base,
                                                       const uint32_t* bg_pix, const uint32_t* bm,
                                                       const uint32_t* wpre, uint32_t* plist) {
    const uint32_t it = blockIdx.y;
    if (it >= n_items) {
        return;
    }
    const GatherItem g = items[it];
    if (g.bmo == kBandMode) {
        return;
    }
    const MapInfo mi = minfo[g.m];
    const BandPos bp = band_pos(mi, g.vb0, S, bg_base);
    const uint32_t words = (bp.npos + 31u) / 32u;
    const size_t vbase = (size_t)bp.v * S * S;
    for (uint32_t w = blockIdx.x * blockDim.x + threadIdx.x; w < words;
         w += gridDim.x * blockDim.x) {
        uint32_t bits = bm[g.bmo + w];
        uint32_t r = g.pl0 + wpre[g.bmo + w];
        while (bits) {
            const uint32_t pos = w * 32u + (uint32_t)__builtin_ctz(bits);
            bits &= bits - 1u;
            plist[r++] = (uint32_t)(vbase + (mi.kind == 2 ? bg_pix[bp.pbase + pos]
                                                          : bp.pbase + pos));
        }
    }
}

// Per gather item and bucket j (thread): the first sorted entry of each chunk
// (positions c P .. of the bucket's band), fo[f0 + c na + j] for c = 0 .. nch
// (nch: the list's end), and the chunk's entry count cnt[c0 + c na + j].
__global__ __launch_bounds__(256) void k_pbr_chunk_first(const GatherItem* items,
                                                         uint32_t n_items, const MapInfo* minfo,
                                                         uint32_t S, const uint32_t* bg_base,
                                                         const uint32_t* order, const uint32_t* off,
                                                         const uint32_t* ent, const uint32_t* bm,
                                                         const uint32_t* wpre, uint32_t* fo,
                                                         uint32_t* cnt) {
    const uint32_t it = blockIdx.y;
    if (it >= n_items) {
        return;
    }
    const GatherItem g = items[it];
    const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= g.na) {
        return;
    }
    const MapInfo mi = minfo[g.m];
    const uint32_t b = order[g.a0 + j];
    const BandPos bp = band_pos(mi, (b - mi.bucket0) / mi.T, S, bg_base);
    uint32_t k = 0;
    const uint32_t e1 = off[b + 1];
    for (uint32_t e = off[b]; e < e1; e++) {
        uint32_t pos = (ent[e] >> 2) - bp.posoff;
        if (g.bmo != kBandMode) {
            pos = list_rank(bm, wpre, g.bmo, pos);
        }
        while (k <= g.nch && k * g.P <= pos) {
            fo[g.f0 + k * g.na + j] = e;
            k++;
        }
    }
    while (k <= g.nch) {
        fo[g.f0 + k * g.na + j] = e1;
        k++;
    }
    for (uint32_t c = 0; c < g.nch; c++) {
        cnt[g.c0 + c * g.na + j] = fo[g.f0 + (c + 1) * g.na + j] - fo[g.f0 + c * g.na + j];
    }
}

// The chunk-major entries: bucket j's entries of chunk c from coff[c0 + c na
// + j], in pixel order, each (LDS slot of the position) << 2 | tap.
__global__ __launch_bounds__(256) void k_pbr_chunk_fill(const GatherItem* items, uint32_t n_items,
                                                        const MapInfo* minfo, uint32_t S,
                                                        const uint32_t* bg_base,
                                                        const uint32_t* order, const uint32_t* ent,
                                                        const uint32_t* bm, const uint32_t* wpre,
                                                        const uint32_t* fo, const uint32_t* coff,
                                                        uint16_t* out) {
    const uint32_t it = blockIdx.y;
    if (it >= n_items) {
        return;
    }
    const GatherItem g = items[it];
    const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= g.na) {
        return;
    }
    const MapInfo mi = minfo[g.m];
    const uint32_t b = order[g.a0 + j];
    const uint32_t vb = (b - mi.bucket0) / mi.T;
    const BandPos bp = band_pos(mi, vb, S, bg_base);
    const uint32_t slot0 = (vb - g.vb0) * g.P;
    for (uint32_t c = 0; c < g.nch; c++) {
        const uint32_t x0 = fo[g.f0 + c * g.na + j], x1 = fo[g.f0 + (c + 1) * g.na + j];
        const uint32_t dst = coff[g.c0 + c * g.na + j];
        for (uint32_t e = x0; e < x1; e++) {
            const uint32_t v = ent[e];
            uint32_t pos = (v >> 2) - bp.posoff;
            if (g.bmo != kBandMode) {
                pos = list_rank(bm, wpre, g.bmo, pos);
            }
            const uint32_t l = slot0 + pos - c * g.P;
            out[dst + (e - x0)] = (uint16_t)((l << 2) | (v & 3u));
        }
    }
}

// ---------------------------------------------------------------------------
// Iteration kernels
// ---------------------------------------------------------------------------

// One level of the pooling chain (Reduce2x2Sum * 0.25, zero padding): level
// `lvl` from level lvl - 1.
__global__ __launch_bounds__(256) void k_pbr_pool(PbrDev d, uint32_t lvl) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t ow = d.pw[lvl], oh = d.ph[lvl];
    if (i >= ow * oh) {
        return;
    }
    const uint32_t w = d.pw[lvl - 1], h = d.ph[lvl - 1];
    const float4* src = d.pool[lvl - 1];
    const uint32_t ox = i % ow, oy = i / ow;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f;
    for (uint32_t dy = 0; dy < 2; dy++) {
        for (uint32_t dx = 0; dx < 2; dx++) {
            const uint32_t px = 2 * ox + dx, py = 2 * oy + dy;
            if (px < w && py < h) {
                const float4 q = src[py * w + px];
                a0 += q.x;
                a1 += q.y;
                a2 += q.z;
            }
        }
    }
    d.pool[lvl][i] = make_float4(a0 * 0.25f, a1 * 0.25f, a2 * 0.25f, 0.f);
}

// Ordered mat-vec in tiles of kMvRows summation steps x kMvCols lanes,
// double-buffered in LDS (128 KB of weights + the x rows): the workgroup's
// next tile is in flight while its three waves (one per colour channel) add
// the current one.
constexpr uint32_t kMvThreads = 192;
constexpr uint32_t kMvVec = kMvRows * kMvCols / 4;                    // float4 per weight tile
constexpr uint32_t kMvPer = (kMvVec + kMvThreads - 1) / kMvThreads;  // per thread
constexpr uint32_t kMvXPer = (kMvRows + kMvThreads - 1) / kMvThreads;

struct MvLds {
    float w[2][kMvRows][kMvCols];
    float x[2][3][kMvRows];  // planar: channel c of rows 4j .. 4j + 3 in one 16-byte read
};

struct MvRegs {
    float4 w[kMvPer];
    float4 x[kMvXPer];
};

// rows [r, r + n) (n <= kMvRows) of the weights of one column group (the
// group's rows of kMvCols floats stored contiguously: `Wg` points at its row
// 0) and of x
__device__ __forceinline__ void mv_fetch(const float* __restrict__ Wg,
                                         const float4* __restrict__ x, uint32_t r, uint32_t n,
                                         MvRegs& g) {
    const float4* w4 = (const float4*)(Wg + (size_t)r * kMvCols);
#pragma unroll
    for (uint32_t i = 0; i < kMvPer; i++) {
        const uint32_t f = threadIdx.x + i * kMvThreads;
        const uint32_t row = f / (kMvCols / 4);
        g.w[i] = (f < kMvVec && row < n) ? w4[f] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (uint32_t i = 0; i < kMvXPer; i++) {
        const uint32_t row = threadIdx.x + i * kMvThreads;
        g.x[i] = row < n ? x[r + row] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

__device__ __forceinline__ void mv_store(MvLds& L, int b, const MvRegs& g) {
#pragma unroll
    for (uint32_t i = 0; i < kMvPer; i++) {
        const uint32_t f = threadIdx.x + i * kMvThreads;
        if (f < kMvVec) {
            const uint32_t row = f / (kMvCols / 4), c4 = f % (kMvCols / 4);
            *(float4*)&L.w[b][row][c4 * 4] = g.w[i];
        }
    }
#pragma unroll
    for (uint32_t i = 0; i < kMvXPer; i++) {
        const uint32_t row = threadIdx.x + i * kMvThreads;
        if (row < kMvRows) {
            L.x[b][0][row] = g.x[i].x;
            L.x[b][1][row] = g.x[i].y;
            L.x[b][2][row] = g.x[i].z;
        }
    }
}

// sum over rows r in [r0, r1) of x[r].c * W(r, lane), from 0 in row order,
// for the calling lane and the wave's channel c; W(r, l) = Wg[r * kMvCols + l]
// (one column group, tile-major). Every thread of the workgroup calls it (it
// synchronises the workgroup).
__device__ float mv_segment(MvLds& L, const float* __restrict__ Wg,
                            const float4* __restrict__ x, uint32_t r0, uint32_t r1) {
    const uint32_t lane = (threadIdx.x & 63u) % kMvCols;
    const uint32_t c = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t n = r1 - r0;
    const uint32_t tiles = (n + kMvRows - 1) / kMvRows;
    MvRegs g;
    mv_fetch(Wg, x, r0, n < kMvRows ? n : kMvRows, g);
    mv_store(L, 0, g);
    __syncthreads();
    float acc = 0.f;
    for (uint32_t t = 0; t < tiles; t++) {
        const uint32_t done = t * kMvRows;
        const uint32_t rows = n - done < kMvRows ? n - done : kMvRows;
        const bool next = t + 1 < tiles;
        if (next) {
            const uint32_t rest = n - done - kMvRows;
            mv_fetch(Wg, x, r0 + done + kMvRows, rest < kMvRows ? rest : kMvRows, g);
        }
        const int b = (int)(t & 1u);
        const float* xs = L.x[b][c];
        uint32_t i = 0;
        // 16 rows' LDS reads in flight, then their products added in order
        for (; i + 16 <= rows; i += 16) {
            float wv[16], xv[16];
#pragma unroll
            for (uint32_t u = 0; u < 16; u += 4) {
                const float4 q = *(const float4*)&xs[i + u];
                xv[u] = q.x;
                xv[u + 1] = q.y;
                xv[u + 2] = q.z;
                xv[u + 3] = q.w;
            }
#pragma unroll
            for (uint32_t u = 0; u < 16; u++) {
                wv[u] = L.w[b][i + u][lane];
            }
#pragma unroll
            for (uint32_t u = 0; u < 16; u++) {
                acc += xv[u] * wv[u];
            }
        }
        for (; i < rows; i++) {
            acc += xs[i] * L.w[b][i][lane];
        }
        if (next) {
            mv_store(L, b ^ 1, g);
        }
        __syncthreads();
    }
    return acc;
}

// Adds rows [i0, i1) of tile b to acc (lane's column, channel c) in row
// order, 16 rows' LDS reads in flight where the rows are 4-aligned.
__device__ __forceinline__ void mv_rows(const MvLds& L, int b, uint32_t c, uint32_t lane,
                                        uint32_t i0, uint32_t i1, float& acc) {
    const float* xs = L.x[b][c];
    uint32_t i = i0;
    for (; i < i1 && (i & 3u); i++) {
        acc += xs[i] * L.w[b][i][lane];
    }
    for (; i + 16 <= i1; i += 16) {
        float wv[16], xv[16];
#pragma unroll
        for (uint32_t u = 0; u < 16; u += 4) {
            const float4 q = *(const float4*)&xs[i + u];
            xv[u] = q.x;
            xv[u + 1] = q.y;
            xv[u + 2] = q.z;
            xv[u + 3] = q.w;
        }
#pragma unroll
        for (uint32_t u = 0; u < 16; u++) {
            wv[u] = L.w[b][i + u][lane];
        }
#pragma unroll
        for (uint32_t u = 0; u < 16; u++) {
            acc += xv[u] * wv[u];
        }
    }
    for (; i < i1; i++) {
        acc += xs[i] * L.w[b][i][lane];
    }
}

// The prefilter transpose's per-level sums in one tile stream: rows [0, n)
// are the levels' texels, level-major (level i ends at lend(i)); each
// level's sum runs from 0 in row order and is added to `a` times st at the
// level's end, in level order -- the sums of one mv_segment per level, with
// the next level's first tile in flight while the previous level ends.
__device__ float mv_levels(MvLds& L, const float* __restrict__ Wg, const float4* __restrict__ x,
                           const PbrDev& d, float st) {
    const uint32_t lane = (threadIdx.x & 63u) % kMvCols;
    const uint32_t c = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t n = d.n_pref;
    const uint32_t tiles = (n + kMvRows - 1) / kMvRows;
    const auto lend = [&](uint32_t i) { return d.loff[i] + d.lw[i] * d.lh[i]; };
    MvRegs g;
    mv_fetch(Wg, x, 0u, n < kMvRows ? n : kMvRows, g);
    mv_store(L, 0, g);
    __syncthreads();
    float a = 0.f, acc = 0.f;
    uint32_t lvl = 0, le = lend(0);
    for (uint32_t t = 0; t < tiles; t++) {
        const uint32_t base = t * kMvRows;
        const uint32_t rows = n - base < kMvRows ? n - base : kMvRows;
        const bool next = t + 1 < tiles;
        if (next) {
            const uint32_t rest = n - base - kMvRows;
            mv_fetch(Wg, x, base + kMvRows, rest < kMvRows ? rest : kMvRows, g);
        }
        const int b = (int)(t & 1u);
        uint32_t i = 0;
        while (i < rows) {
            const uint32_t e = le - base < rows ? le - base : rows;
            mv_rows(L, b, c, lane, i, e, acc);
            i = e;
            if (base + i == le) {
                a += acc * st;
                acc = 0.f;
                lvl++;
                le = lvl < d.levels ? lend(lvl) : 0xffffffffu;
            }
        }
        if (next) {
            mv_store(L, b ^ 1, g);
        }
        __syncthreads();
    }
    return a;
}

// IrradianceConv and every PrefilterConv level (f_ops.cpp:3006-3087,
// 3264-3348): out[o] = (sum_s e[s] * w(o, s)) * 2 pi / (sw sh) for the
// irradiance map, (sum_s e[s] * w(o, s)) / max(norm[o], 1e-12) for a
// prefilter texel, the sums over the pooled source in raster order from 0.
// The weights (cos+ sin(theta) / GGX sin(theta)) are static: wf_*
// [source][output], rows of ld_* floats. A workgroup holds 64 outputs; wave
// c computes colour channel c.
__global__ __launch_bounds__(192) void k_pbr_conv_fwd(PbrDev d) {
    __shared__ MvLds L;
    const bool irr = blockIdx.x < d.n_ig;
    const uint32_t n_out = irr ? d.iw * d.ih : d.n_pref;
    const uint32_t n_src = irr ? d.isw * d.ish : d.psw * d.psh;
    const uint32_t col0 = (irr ? blockIdx.x : blockIdx.x - d.n_ig) * kMvCols;
    const uint32_t o = col0 + (threadIdx.x & 63u) % kMvCols;
    const uint32_t c = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const float4* src = irr ? d.pool[d.irr_pool] : d.pool[d.pref_pool];
    const float* Wg = (irr ? d.wf_irr : d.wf_pref) + (size_t)col0 * n_src;  // group's rows
    const float acc = mv_segment(L, Wg, src, 0, n_src);
    if (o >= n_out || (threadIdx.x & 63u) >= kMvCols) {
        return;
    }
    if (irr) {
        ((float*)d.irr)[(size_t)o * 4 + c] = acc * d.irr_scale;
    } else {
        const float nt = d.pnorm[o];
        ((float*)d.pref)[(size_t)o * 4 + c] = acc / (nt < 1e-12f ? 1e-12f : nt);
    }
}

// F::Sum (f_ops.cpp:1037-1043) reduces an image by Reduce2x2Sum levels
// (f_ops.cpp:999-1033: each output texel adds its 2x2 source block from 0
// in row order, a missing row or column adding nothing) down to 1 x 1. On a
// 16 x 16-aligned block that is a quadtree whose four lowest levels lie in
// the block; zero padding is exact (the sums start at +0).
struct QuadLds {
    float4 q[256], q1[64], q2[16], q3[4];
};

__device__ __forceinline__ float4 quad4(const float4& a, const float4& b, const float4& c,
                                        const float4& e) {
    float4 r;
    r.x = (((0.f + a.x) + b.x) + c.x) + e.x;
    r.y = (((0.f + a.y) + b.y) + c.y) + e.y;
    r.z = (((0.f + a.z) + b.z) + c.z) + e.z;
    r.w = 0.f;
    return r;
}

// The 16 x 16 block in L.q (row-major) reduced by four Reduce2x2Sum levels;
// the result in thread 0. Every thread of the 256-thread workgroup calls it.
__device__ float4 quad_reduce16(QuadLds& L) {
    const uint32_t t = threadIdx.x;
    __syncthreads();
    if (t < 64) {
        const uint32_t i = (t >> 3) * 32u + (t & 7u) * 2u;
        L.q1[t] = quad4(L.q[i], L.q[i + 1], L.q[i + 16], L.q[i + 17]);
    }
    __syncthreads();
    if (t < 16) {
        const uint32_t i = (t >> 2) * 16u + (t & 3u) * 2u;
        L.q2[t] = quad4(L.q1[i], L.q1[i + 1], L.q1[i + 8], L.q1[i + 9]);
    }
    __syncthreads();
    if (t < 4) {
        const uint32_t i = (t >> 1) * 8u + (t & 1u) * 2u;
        L.q3[t] = quad4(L.q2[i], L.q2[i + 1], L.q2[i + 4], L.q2[i + 5]);
    }
    __syncthreads();
    float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
    if (t == 0) {
        r = quad4(L.q3[0], L.q3[1], L.q3[2], L.q3[3]);
    }
    __syncthreads();  // L is reused by the caller
    return r;
}

// Per pixel (a 16 x 16 tile of one view per workgroup): the shading
// forward, the L1 loss and its backward (the derivation of the reference's
// autodiff of pbr_graph.cpp:47-137 through Div / Mul / Add / Max / Mix /
// Clamp / Pow / Abs, f_ops.cpp:235-537); in target mode the forward only.
// Outputs per pixel: the material gradients (gyA, gyM) and the seeds of the
// map-gradient VJPs (mgA, mgB) that k_pbr_map_gather spreads over the maps.
// The prefilter levels with a tent weight 1 - |lod - i| >= 0 are among
// floor(lod) - 1 .. floor(lod) + 1: three register slots.
__global__ __launch_bounds__(256) void k_pbr_shade(PbrDev d) {
    __shared__ QuadLds lq;
    const uint32_t tiles = (d.S + kShadeTile - 1) / kShadeTile;
    const uint32_t view = blockIdx.x / (tiles * tiles);
    const uint32_t tile = blockIdx.x % (tiles * tiles);
    const uint32_t x = (tile % tiles) * kShadeTile + (threadIdx.x % kShadeTile);
    const uint32_t y = (tile / tiles) * kShadeTile + (threadIdx.x / kShadeTile);
    const bool valid = x < d.S && y < d.S;
    const size_t npx = (size_t)d.S * d.S;
    const size_t p = (size_t)view * npx + (size_t)(valid ? y * d.S + x : 0);
    const int L = (int)d.levels;
    const bool train = !d.target_mode;
    // ---- forward --------------------------------------------------------
    const float4 s0 = valid ? d.st0[p] : make_float4(0.f, 0.f, -1.f, 0.f);
    const bool fg = valid && s0.z >= 0.f;
    float hdr[3] = {0.f, 0.f, 0.f};
    bool act[3] = {false, false, false};
    int li[3] = {0, 0, 0};
    float xs[3] = {0.f, 0.f, 0.f}, ws[3] = {0.f, 0.f, 0.f}, Ps[3][3];
    float a[3] = {0.f, 0.f, 0.f}, mr[3] = {0.f, 0.f, 0.f}, irr[3] = {0.f, 0.f, 0.f};
    float pref[3] = {0.f, 0.f, 0.f}, lut[2] = {0.f, 0.f};
    float ao = 0.f, rough = 0.f, metal = 0.f, lod = 0.f;
    float4 s1 = f4_zero(), s2 = f4_zero();
#pragma unroll
    for (int j = 0; j < 3; j++) {
        Ps[j][0] = Ps[j][1] = Ps[j][2] = 0.f;
    }
    if (valid && !fg) {
        if (s0.x >= 0.f) {
            fetch4(taps_wrap((int)d.ew, (int)d.eh, s0.x, s0.y), d.env, hdr);
        }
    } else if (fg) {
        s1 = d.st1[p];
        s2 = d.st2[p];
        const Taps tt = taps_clamp((int)d.tw, (int)d.th, s0.x, s0.y);
        fetch4(tt, d.albedo, a);
        fetch4(tt, d.mr, mr);
        ao = 0.f;
        ao += tt.w[0] * 1.f;
        ao += tt.w[1] * 1.f;
        ao += tt.w[2] * 1.f;
        ao += tt.w[3] * 1.f;
        rough = mr[1] < 0.045f ? 0.045f : (mr[1] > 1.f ? 1.f : mr[1]);
        metal = mr[2];
        if (s2.x >= 0.f) {
            fetch4(taps_wrap((int)d.iw, (int)d.ih, s2.x, s2.y), d.irr, irr);
        }
        lod = rough * (float)(L - 1);
        const int base = (int)floorf(lod) - 1;
#pragma unroll
        for (int j = 0; j < 3; j++) {
            const int i = base + j;
            li[j] = i;
            if (i < 0 || i >= L) {
                continue;
            }
            xs[j] = 1.f - fabsf(lod - (float)i);
            ws[j] = xs[j] < 0.f ? 0.f : (xs[j] > 1.f ? 1.f : xs[j]);
            if (xs[j] >= 0.f && s2.z >= 0.f) {
                act[j] = true;
                const uint4 lv = d.ltab[i];
                fetch4(taps_wrap((int)lv.x, (int)lv.y, s2.z, s2.w), d.pref + lv.z, Ps[j]);
                pref[0] += Ps[j][0] * ws[j];
                pref[1] += Ps[j][1] * ws[j];
                pref[2] += Ps[j][2] * ws[j];
            }
        }
        {
            const Taps tl = taps_clamp((int)d.lutw, (int)d.luth, s0.z, rough);
            float a0 = 0.f, a1 = 0.f;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float2 q = d.lut[tl.idx[k]];
                a0 += tl.w[k] * q.x;
                a1 += tl.w[k] * q.y;
            }
            lut[0] = a0;
            lut[1] = a1;
        }
    }
    // shading terms (foreground)
    const float ndv = s0.z, ndl = s0.w, ndh = s1.x, p5v = s1.y, p5n = s1.z, dist2 = s1.w;
    float f0[3], F[3], kd[3], fib[3], kdi[3], R0[3];
    const float alpha = rough * rough;
    const float alpha2 = alpha * alpha;
    const float dd = ndh * ndh * (alpha2 - 1.f) + 1.f;
    const float D = alpha2 / (kIblPi * dd * dd);
    const float kk = (rough + 1.f) * (rough + 1.f) / 8.f;
    const float gvd = ndv * (1.f - kk) + kk;
    const float g_v = ndv / gvd;
    const float ndlc = ndl < 1e-4f ? 1e-4f : ndl;
    const float gld = ndlc * (1.f - kk) + kk;
    const float g_l = ndlc / gld;
    const float den = 4.f * ndv * ndl + 1e-4f;
    const float Sd = D * g_v * g_l / den;
    if (fg) {
#pragma unroll
        for (int c = 0; c < 3; c++) {
            f0[c] = 0.04f + (a[c] - 0.04f) * metal;
            F[c] = f0[c] + (1.f - f0[c]) * p5v;
            kd[c] = (1.f - F[c]) * (1.f - metal);
            R0[c] = d.light_col[c] / dist2;
            const float mx = (1.f - rough) < f0[c] ? f0[c] : (1.f - rough);
            fib[c] = f0[c] + (mx - f0[c]) * p5n;
            kdi[c] = (1.f - fib[c]) * (1.f - metal);
            const float lo = (kd[c] * a[c] / kIblPi + F[c] * Sd) * R0[c] * ndl;
            const float spec_ibl = pref[c] * (f0[c] * lut[0] + lut[1]);
            const float amb = (kdi[c] * irr[c] * a[c] + spec_ibl) * ao;
            hdr[c] = (lo + amb) + 0.f;
        }
    }
    float mapped[3];
#pragma unroll
    for (int c = 0; c < 3; c++) {
        mapped[c] = hdr[c] / (hdr[c] + 1.f);
    }
    if (!train) {
        if (valid) {
            d.target[p] = make_float4(mapped[0], mapped[1], mapped[2], 0.f);
        }
        return;
    }
    if (valid && d.pred) {
        d.pred[p] = make_float4(mapped[0], mapped[1], mapped[2], 0.f);
    }
    // ---- loss and d loss / d hdr -----------------------------------------
    float gh[3] = {0.f, 0.f, 0.f};
    float lc[3] = {0.f, 0.f, 0.f};  // |diff| per channel (0 off the screen)
    if (valid) {
        const float4 tg = d.target[p];
        const float tv[3] = {tg.x, tg.y, tg.z};
#pragma unroll
        for (int c = 0; c < 3; c++) {
            const float diff = tv[c] - mapped[c];
            lc[c] = fabsf(diff);
            const float sg = (float)((diff > 0.f) - (diff < 0.f));
            const float gm = -(d.inv_n * sg);
            gh[c] = gm / (hdr[c] + 1.f) - gm * hdr[c] / ((hdr[c] + 1.f) * (hdr[c] + 1.f));
        }
    }
    // ---- backward ---------------------------------------------------------
    float ga[3] = {0.f, 0.f, 0.f}, gmet = 0.f, gr = 0.f, gS = 0.f;
    float g_irr[3] = {0.f, 0.f, 0.f}, gpref[3] = {0.f, 0.f, 0.f};
    if (fg) {
#pragma unroll
        for (int c = 0; c < 3; c++) {
            const float gs = gh[c];
            const float q = gs * R0[c] * ndl;
            ga[c] += q * kd[c] / kIblPi;
            const float gkd = q * a[c] / kIblPi;
            const float gF = q * Sd - gkd * (1.f - metal);
            gS += q * F[c];
            gmet -= gkd * (1.f - F[c]);
            const float u = gs * ao;
            g_irr[c] = u * kdi[c] * a[c];
            ga[c] += u * kdi[c] * irr[c];
            const float gkdi = u * irr[c] * a[c];
            gpref[c] = u * (f0[c] * lut[0] + lut[1]);
            float gf0 = u * pref[c] * lut[0];
            const float gfib = -gkdi * (1.f - metal);
            gmet -= gkdi * (1.f - fib[c]);
            const bool pick_r = (1.f - rough) >= f0[c];
            gf0 += gfib * (1.f - p5n) + (pick_r ? 0.f : gfib * p5n);
            if (pick_r) {
                gr -= gfib * p5n;
            }
            gf0 += gF * (1.f - p5v);
            ga[c] += gf0 * metal;
            gmet += gf0 * (a[c] - 0.04f);
        }
        float glod = 0.f;
#pragma unroll
        for (int j = 0; j < 3; j++) {
            if (!act[j] || xs[j] > 1.f) {
                continue;
            }
            const float gw = gpref[0] * Ps[j][0] + gpref[1] * Ps[j][1] + gpref[2] * Ps[j][2];
            const float dl = lod - (float)li[j];
            const float sgn = (float)((dl > 0.f) - (dl < 0.f));
            glod -= gw * sgn;
        }
        {
            // level floor(lod) + 2: lod - i rounds to exactly -1 when lod lies
            // within half an ulp below an integer, and its weight clamp(0, 0,
            // 1) = 0 adds nothing forward, but Clamp's backward passes the
            // gradient at its bounds (Step(lo, x) * Step(x, hi)); it comes
            // last in level order, with dl < 0
            const int i = li[2] + 1;
            if (i < L && s2.z >= 0.f && 1.f - fabsf(lod - (float)i) >= 0.f) {
                const uint4 lv = d.ltab[i];
                float P3[3];
                fetch4(taps_wrap((int)lv.x, (int)lv.y, s2.z, s2.w), d.pref + lv.z, P3);
                const float gw = gpref[0] * P3[0] + gpref[1] * P3[1] + gpref[2] * P3[2];
                glod -= gw * -1.f;
            }
        }
        gr += glod * (float)(L - 1);
        const float gD = gS * g_v * g_l / den;
        const float ggv = gS * D * g_l / den;
        const float ggl = gS * D * g_v / den;
        const float galpha2 =
                gD * (1.f / (kIblPi * dd * dd) - 2.f * alpha2 * ndh * ndh / (kIblPi * dd * dd * dd));
        gr += galpha2 * 2.f * alpha * 2.f * rough;
        const float gk = ggv * (-ndv * (1.f - ndv) / (gvd * gvd)) +
                         ggl * (-ndlc * (1.f - ndlc) / (gld * gld));
        gr += gk * (rough + 1.f) / 4.f;
        if (!(mr[1] >= 0.045f && 1.f >= mr[1])) {
            gr = 0.f;
        }
    }
    if (valid) {
        d.gyA[p] = make_float4(ga[0], ga[1], ga[2], gr);
        d.gyM[p] = gmet;
        // seeds of the map VJPs: the irradiance sample's gradient (fg) or the
        // background env sample's (bg: d hdr / d env sample = 1); the
        // prefiltered sample's before the level weights, with the roughness
        // the level weights come from
        d.mgA[p] = fg ? make_float4(g_irr[0], g_irr[1], g_irr[2], 0.f)
                      : make_float4(gh[0], gh[1], gh[2], 0.f);
        if (fg) {
            d.mgB[p] = make_float4(gpref[0], gpref[1], gpref[2], rough);
        }
    }
    // ---- loss partial of the tile: Sum's first four Reduce2x2Sum levels ---
    lq.q[threadIdx.x] = make_float4(lc[0], lc[1], lc[2], 0.f);
    const float4 tsum = quad_reduce16(lq);
    if (threadIdx.x == 0) {
        d.loss_part[blockIdx.x] = tsum;
    }
}

// The map of a bucket (maps are few; their buckets are contiguous)
__device__ __forceinline__ uint32_t map_of_bucket(const PbrDev& d, uint32_t b) {
    uint32_t m = 0;
    while (m + 1 < d.n_maps && b >= d.minfo[m + 1].bucket0) {
        m++;
    }
    return m;
}

// EquirectSampleBwd's band partials (f_ops.cpp:2862-2904) of up to 256
// (map, view, band, texel) buckets of consecutive bands, one per thread: each
// from 0, the bucket's list entries (pixel, tap) in pixel order, each adding
// gy * w with the tap's bilinear weight w = (dx ? fx : 1 - fx) * (dy ? fy :
// 1 - fy) of the pixel's direction uv (fx = (u w - 0.5) - floor(u w - 0.5),
// f_ops.cpp:2874-2892) and its gy: the irradiance sample's gradient, the
// prefiltered sample's times the level's tent weight clamp(1 - |lod - i|, 0,
// 1), or the background env sample's. Entries whose gy is always 0 are not
// listed (background pixels of the material maps, pixels with a zero-length
// direction), which changes no sum that starts at +0.
// The bands are walked together in chunks: each chunk's per-position tap
// weights and gy are staged in LDS once for all the buckets (an entry value
// (slot << 2) | tap indexes its weight directly), with the chunk's entries;
// the next chunk's loads are in flight while every thread adds its bucket's
// entries of this chunk in order, four per step with their LDS loads issued
// together.
__global__ __launch_bounds__(256) void k_pbr_map_gather(PbrDev d) {
    constexpr uint32_t kPer = kGatherChunk / 256u;            // position slots per thread
    constexpr uint32_t kWords = (4u * kGatherChunk) / 8u + 1u;  // 16-byte entry words per chunk
    constexpr uint32_t kWper = (kWords + 255u) / 256u;
    static_assert(kWper == 3, "the entry words are staged in three registers per thread");
    __shared__ float sw[4 * kGatherChunk];  // per slot and tap: the bilinear weight
    __shared__ float4 sg[kGatherChunk];     // per slot: gy (xyz)
    __shared__ uint4 sew[kWper * 256u];     // the chunk's entries from an aligned start
    __shared__ uint32_t bvpx[kGatherBands], bbase[kGatherBands], bnpos[kGatherBands];
    const uint16_t* se = (const uint16_t*)sew;
    const GatherItem it = d.gitems[blockIdx.x];
    const MapInfo mi = d.minfo[it.m];
    const uint32_t tid = threadIdx.x;
    if (tid < it.nb) {
        const BandPos bp = band_pos(mi, it.vb0 + tid, d.S, d.bg_base);
        bvpx[tid] = bp.v * d.S * d.S;
        bbase[tid] = bp.pbase;
        bnpos[tid] = bp.npos;
    }
    __syncthreads();
    const float fw = (float)mi.w, fh = (float)mi.h;
    const float lod_scale = (float)(d.levels - 1), lvl = (float)mi.level;
    // the map's uv pair of a position: st0.xy (background env), st2.xy
    // (irradiance) or st2.zw (prefilter levels)
    const float2* uvsrc = (const float2*)(mi.kind == 2 ? d.st0 : d.st2) + (mi.kind == 1 ? 1 : 0);
    const float4* gsrc = mi.kind == 1 ? d.mgB : d.mgA;
    const uint32_t nch = it.nch, P = it.P, nslot = it.nb * it.P;
    const uint32_t* coff = d.coff + it.c0;
    const bool mine = tid < it.na;
    const bool listed = it.bmo != kBandMode;  // positions from the workgroup's list (nb = 1)
    // this thread's position slots: band and position within the chunk
    uint32_t sbi0, sbi1, sbi2, sbi3;
    sbi0 = tid < nslot ? tid / P : 0u;
    sbi1 = tid + 256u < nslot ? (tid + 256u) / P : 0u;
    sbi2 = tid + 512u < nslot ? (tid + 512u) / P : 0u;
    sbi3 = tid + 768u < nslot ? (tid + 768u) / P : 0u;
    static_assert(kPer == 4, "four position slots per thread");
    // chunk data in flight: positions, entry words, this bucket's entry range
    float2 rs[kPer];
    float4 rg[kPer];
    bool rv[kPer];
    uint4 rw0, rw1, rw2;
    uint32_t rx0 = 0, rx1 = 0, ra0 = 0;
    // one chunk further ahead: the positions' pixel indices (from the
    // position list or the background list) and the chunk's entry run, so
    // that a chunk's loads depend on no load of their own
    uint32_t pq[kPer];
    bool pv[kPer];
    uint32_t prun0 = 0, prun1 = 0;
#define DRESSI_GATHER_PRE(CC)                                                                    \
    {                                                                                            \
        const uint32_t cp_ = (CC);                                                               \
        _Pragma("unroll") for (uint32_t r = 0; r < kPer; r++) {                                  \
            const uint32_t u = tid + 256u * r;                                                   \
            const uint32_t bi = r == 0 ? sbi0 : (r == 1 ? sbi1 : (r == 2 ? sbi2 : sbi3));       \
            const uint32_t pos = cp_ * P + (u - bi * P);                                         \
            if (listed) {                                                                        \
                pv[r] = pos < it.npl;                                                            \
                pq[r] = pv[r] ? d.plist[it.pl0 + pos] : 0u;                                      \
            } else {                                                                             \
                pv[r] = u < nslot && pos < bnpos[bi];                                            \
                pq[r] = pv[r] ? bvpx[bi] + (mi.kind == 2 ? d.bg_pix[bbase[bi] + pos]             \
                                                         : bbase[bi] + pos)                      \
                              : 0u;                                                              \
            }                                                                                    \
        }                                                                                        \
        prun0 = coff[cp_ * it.na];                                                               \
        prun1 = coff[(cp_ + 1) * it.na]; /* the next block's first: the end */                   \
    }
#define DRESSI_GATHER_FETCH(CC)                                                                  \
    {                                                                                            \
        const uint32_t cc_ = (CC);                                                               \
        _Pragma("unroll") for (uint32_t r = 0; r < kPer; r++) {                                  \
            rv[r] = pv[r];                                                                       \
            if (rv[r]) {                                                                         \
                rs[r] = uvsrc[2u * pq[r]];                                                       \
                rg[r] = gsrc[pq[r]];                                                             \
            }                                                                                    \
        }                                                                                        \
        ra0 = prun0 & ~7u;                                                                       \
        const uint32_t nw_ = (prun1 - ra0 + 7u) / 8u;                                            \
        const uint4* src_ = (const uint4*)(d.mg_ent + ra0);                                      \
        const uint4 z4_ = make_uint4(0u, 0u, 0u, 0u);                                            \
        rw0 = tid < nw_ ? src_[tid] : z4_;                                                       \
        rw1 = tid + 256u < nw_ ? src_[tid + 256u] : z4_;                                         \
        rw2 = tid + 512u < nw_ ? src_[tid + 512u] : z4_;                                         \
        rx0 = mine ? coff[cc_ * it.na + tid] : 0u;                                               \
        rx1 = mine ? coff[cc_ * it.na + tid + 1] : 0u;                                           \
        if (cc_ + 1 < nch) {                                                                     \
            DRESSI_GATHER_PRE(cc_ + 1u)                                                          \
        }                                                                                        \
    }
    float a0 = 0.f, a1 = 0.f, a2 = 0.f;
    if (nch > 0) {
        DRESSI_GATHER_PRE(0u)
        DRESSI_GATHER_FETCH(0u)
    }
    for (uint32_t c = 0; c < nch; c++) {
        __syncthreads();  // the previous chunk's readers are done
#pragma unroll
        for (uint32_t r = 0; r < kPer; r++) {
            if (rv[r]) {
                const uint32_t u = tid + 256u * r;
                const float2 st = rs[r];
                const float4 g = rg[r];
                const float uu = st.x;
                const float vv = st.y;
                const float sx = uu * fw - 0.5f;
                const float sy = vv * fh - 0.5f;
                const float fx = sx - floorf(sx);
                const float fy = sy - floorf(sy);
                float g0 = g.x, g1 = g.y, g2 = g.z;
                if (mi.kind == 1) {
                    const float xl = 1.f - fabsf(g.w * lod_scale - lvl);
                    const float wl = xl < 0.f ? 0.f : (xl > 1.f ? 1.f : xl);
                    g0 = g0 * wl;
                    g1 = g1 * wl;
                    g2 = g2 * wl;
                }
                const float ex = 1.f - fx, ey = 1.f - fy;
                sw[4u * u + 0u] = ex * ey;
                sw[4u * u + 1u] = fx * ey;
                sw[4u * u + 2u] = ex * fy;
                sw[4u * u + 3u] = fx * fy;
                sg[u] = make_float4(g0, g1, g2, 0.f);
            }
        }
        sew[tid] = rw0;
        sew[tid + 256u] = rw1;
        sew[tid + 512u] = rw2;
        const uint32_t x1 = rx1 - ra0;  // this bucket's entries in the staged words
        uint32_t x = rx0 - ra0;
        __syncthreads();
        if (c + 1 < nch) {  // chunk c + 1's loads, in flight while this chunk is summed
            DRESSI_GATHER_FETCH(c + 1u)
        }
        if (x + 8u <= x1) {
            // batches of 8 entries, software-pipelined: the next batch's LDS
            // reads are in flight while this batch's products are added in
            // order
            float w[8];
            float4 g[8];
#pragma unroll
            for (uint32_t r = 0; r < 8; r++) {
                const uint32_t e = se[x + r];
                w[r] = sw[e];
                g[r] = sg[e >> 2];
            }
            for (; x + 16u <= x1; x += 8u) {
                uint32_t en[8];
#pragma unroll
                for (uint32_t r = 0; r < 8; r++) {
                    en[r] = se[x + 8u + r];
                }
                float c0[8], c1[8], c2[8];
#pragma unroll
                for (uint32_t r = 0; r < 8; r++) {
                    c0[r] = g[r].x * w[r];
                    c1[r] = g[r].y * w[r];
                    c2[r] = g[r].z * w[r];
                }
#pragma unroll
                for (uint32_t r = 0; r < 8; r++) {
                    w[r] = sw[en[r]];
                    g[r] = sg[en[r] >> 2];
                }
#pragma unroll
                for (uint32_t r = 0; r < 8; r++) {
                    a0 += c0[r];
                    a1 += c1[r];
                    a2 += c2[r];
                }
            }
#pragma unroll
            for (uint32_t r = 0; r < 8; r++) {
                a0 += g[r].x * w[r];
                a1 += g[r].y * w[r];
                a2 += g[r].z * w[r];
            }
            x += 8u;
        }
        for (; x + 4u <= x1; x += 4u) {
            float c0[4], c1[4], c2[4];
#pragma unroll
            for (uint32_t r = 0; r < 4; r++) {
                const uint32_t e = se[x + r];
                const float w = sw[e];
                const float4 g = sg[e >> 2];
                c0[r] = g.x * w;
                c1[r] = g.y * w;
                c2[r] = g.z * w;
            }
#pragma unroll
            for (uint32_t r = 0; r < 4; r++) {
                a0 += c0[r];
                a1 += c1[r];
                a2 += c2[r];
            }
        }
        for (; x < x1; x++) {
            const uint32_t e = se[x];
            const float w = sw[e];
            const float4 g = sg[e >> 2];
            a0 += g.x * w;
            a1 += g.y * w;
            a2 += g.z * w;
        }
    }
#undef DRESSI_GATHER_FETCH
#undef DRESSI_GATHER_PRE
    if (mine) {
        const uint32_t b = d.ml_order[it.a0 + tid];
        const float4 res = make_float4(a0, a1, a2, 0.f);
        if (mi.k == 1) {
            const uint32_t t = (b - mi.bucket0) % mi.T;
            const uint32_t v = (b - mi.bucket0) / mi.T;
            d.mtot[mi.tot0 + v * mi.T + t] = res;
        } else {
            d.mpart[b] = res;
        }
    }
}

// TileSum (f_ops.cpp:2786-2821) of one (map, view) over a run of texels: from
// 0, the band partials in band order. The workgroup stages rounds of
// partials in LDS (coalesced), then one thread per texel adds them.
__global__ __launch_bounds__(256) void k_pbr_tile_sum(PbrDev d) {
    __shared__ float4 buf[kTileSumLds];
    const uint4 wi = d.tsum_work[blockIdx.x];
    const MapInfo mi = d.minfo[wi.x];
    const uint32_t v = wi.y, t0 = wi.z, cnt = wi.w;
    const uint32_t per = kTileSumLds / cnt;  // bands per round
    const float4* part = d.mpart + mi.bucket0 + (size_t)v * mi.k * mi.T + t0;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f;
    for (uint32_t b0 = 0; b0 < mi.k; b0 += per) {
        const uint32_t nb = mi.k - b0 < per ? mi.k - b0 : per;
        // all of the round's loads in flight, then the LDS stores
        constexpr uint32_t kPer = kTileSumLds / 256u;
        float4 r[kPer];
#pragma unroll
        for (uint32_t u = 0; u < kPer; u++) {
            const uint32_t j = threadIdx.x + u * 256u;
            r[u] = j < nb * cnt ? part[(size_t)(b0 + j / cnt) * mi.T + j % cnt]
                                : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        __syncthreads();
#pragma unroll
        for (uint32_t u = 0; u < kPer; u++) {
            buf[threadIdx.x + u * 256u] = r[u];
        }
        __syncthreads();
        if (threadIdx.x < cnt) {
            // eight bands' LDS reads in flight, then added in band order
            uint32_t band = 0;
            for (; band + 8u <= nb; band += 8u) {
                float4 q[8];
#pragma unroll
                for (uint32_t u = 0; u < 8; u++) {
                    q[u] = buf[(band + u) * cnt + threadIdx.x];
                }
#pragma unroll
                for (uint32_t u = 0; u < 8; u++) {
                    a0 += q[u].x;
                    a1 += q[u].y;
                    a2 += q[u].z;
                }
            }
            for (; band < nb; band++) {
                const float4 q = buf[band * cnt + threadIdx.x];
                a0 += q.x;
                a1 += q.y;
                a2 += q.z;
            }
        }
    }
    if (threadIdx.x < cnt) {
        d.mtot[mi.tot0 + v * mi.T + t0 + threadIdx.x] = make_float4(a0, a1, a2, 0.f);
    }
}

// The map gradients: per texel, the views' VJP results added in view order
// from 0 (the irradiance map, every prefilter level, the background env).
__global__ __launch_bounds__(256) void k_pbr_view_sum(PbrDev d) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t ni = d.iw * d.ih, ne = d.ew * d.eh;
    if (i >= ni + d.n_pref + ne) {
        return;
    }
    float4* out;
    uint32_t m, t;
    if (i < ni) {
        m = 0;
        t = i;
        out = d.g_irr + t;
    } else if (i < ni + d.n_pref) {
        const uint32_t j = i - ni;
        m = 1;
        while (m < d.levels && j >= d.loff[m]) {
            m++;
        }
        t = j - d.loff[m - 1];
        out = d.g_pref + j;
    } else {
        m = d.levels + 1;
        t = i - ni - d.n_pref;
        out = d.g_bg + t;
    }
    const MapInfo mi = d.minfo[m];
    float a0 = 0.f, a1 = 0.f, a2 = 0.f;
    for (uint32_t v = 0; v < d.n_views; v++) {
        const float4 q = d.mtot[mi.tot0 + v * mi.T + t];
        a0 += q.x;
        a1 += q.y;
        a2 += q.z;
    }
    *out = make_float4(a0, a1, a2, 0.f);
}

// The convolutions' transposes (IrradianceConvBwd f_ops.cpp:2970-3004,
// PrefilterConvBwd :3207-3262): per pooled source texel s, irradiance
// (sum_o g[o] w(o, s)) * 2 pi / (sw sh); prefilter, per level in order,
// (sum_t g[t] w(t, s) / max(norm[t], 1e-12)) * sin(theta_s), the levels
// added in level order from 0. Sums over the map texels in raster order;
// static weights wb_* [map texel][source]; wave c computes channel c.
__global__ __launch_bounds__(192) void k_pbr_conv_bwd(PbrDev d) {
    __shared__ MvLds L;
    const bool irr = blockIdx.x < d.n_isg;
    const uint32_t n_src = irr ? d.isw * d.ish : d.psw * d.psh;
    const uint32_t col0 = (irr ? blockIdx.x : blockIdx.x - d.n_isg) * kMvCols;
    const uint32_t s = col0 + (threadIdx.x & 63u) % kMvCols;
    const uint32_t c = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool ok = s < n_src && (threadIdx.x & 63u) < kMvCols;
    if (irr) {
        const float acc = mv_segment(L, d.wb_irr + (size_t)col0 * (d.iw * d.ih), d.g_irr, 0,
                                     d.iw * d.ih);
        if (ok) {
            ((float*)d.g_isrc)[(size_t)s * 4 + c] = acc * d.irr_scale;
        }
        return;
    }
    const float st = d.psdir[ok ? s : 0u].w;
    const float a = mv_levels(L, d.wb_pref + (size_t)col0 * d.n_pref, d.g_pref, d, st);
    if (ok) {
        ((float*)d.g_psrc)[(size_t)s * 4 + c] = a;
    }
}

__device__ __forceinline__ void adam_bias(const PbrDev& d, float t_new, float* bc1, float* bc2) {
    if (t_new >= 1.f && t_new <= (float)d.bc_len && t_new == floorf(t_new)) {
        const float2 bc = d.bc_tab[(uint32_t)t_new - 1];
        *bc1 = bc.x;
        *bc2 = bc.y;
    } else {
        *bc1 = 1.f - powf(d.b1, t_new);
        *bc2 = 1.f - powf(d.b2, t_new);
    }
}

// Adam on a float4 (first 3 channels) with the clamp of the parameter
__device__ __forceinline__ void adam3(const PbrDev& d, float bc1, float bc2, const float* g,
                                      float4* x4, float4* m4, float4* v4, bool unit) {
    const float4 x = *x4, m = *m4, v = *v4;
    float xi[3] = {x.x, x.y, x.z}, mi[3] = {m.x, m.y, m.z}, vi[3] = {v.x, v.y, v.z};
    const float cb1 = 1.f - d.b1, cb2 = 1.f - d.b2;
#pragma unroll
    for (int c = 0; c < 3; c++) {
        const float mn = mi[c] * d.b1 + g[c] * cb1;
        const float vn = vi[c] * d.b2 + g[c] * g[c] * cb2;
        const float step = (mn / bc1) / (sqrtf(vn / bc2) + d.eps) * d.lr;
        const float xn = xi[c] - step;
        xi[c] = unit ? (xn < 0.f ? 0.f : (xn > 1.f ? 1.f : xn)) : (xn < 0.f ? 0.f : xn);
        mi[c] = mn;
        vi[c] = vn;
    }
    *x4 = make_float4(xi[0], xi[1], xi[2], x.w);
    *m4 = make_float4(mi[0], mi[1], mi[2], 0.f);
    *v4 = make_float4(vi[0], vi[1], vi[2], 0.f);
}

// Per env texel: the background gradient (view sums of the env VJP), then
// the pooling chains' VJPs (UpsampleNearest2x of gy * 0.25 per level,
// f_ops.cpp:958-994) of the irradiance and of the prefilter source added in
// that order, Adam (env >= 0).
__global__ __launch_bounds__(256) void k_pbr_env_adam(PbrDev d) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= d.ew * d.eh) {
        return;
    }
    const uint32_t x = i % d.ew, y = i / d.ew;
    const float4 gb = d.g_bg[i];
    float g[3] = {gb.x, gb.y, gb.z};
    {
        const uint32_t sx = x >> d.irr_pool, sy = y >> d.irr_pool;
        const float4 q = d.g_isrc[sy * d.isw + sx];
        float c3[3] = {q.x, q.y, q.z};
        for (uint32_t l = 0; l < d.irr_pool; l++) {
            c3[0] *= 0.25f;
            c3[1] *= 0.25f;
            c3[2] *= 0.25f;
        }
        g[0] += c3[0];
        g[1] += c3[1];
        g[2] += c3[2];
    }
    {
        const uint32_t sx = x >> d.pref_pool, sy = y >> d.pref_pool;
        const float4 q = d.g_psrc[sy * d.psw + sx];
        float c3[3] = {q.x, q.y, q.z};
        for (uint32_t l = 0; l < d.pref_pool; l++) {
            c3[0] *= 0.25f;
            c3[1] *= 0.25f;
            c3[2] *= 0.25f;
        }
        g[0] += c3[0];
        g[1] += c3[1];
        g[2] += c3[2];
    }
    if (d.g_env) {
        d.g_env[i] = make_float4(g[0], g[1], g[2], 0.f);
    }
    float bc1, bc2;
    adam_bias(d, *d.t + 1.f, &bc1, &bc2);
    adam3(d, bc1, bc2, g, &d.env[i], &d.em[i], &d.ev[i], false);
}

// Per texel: the static gather list (GatherByInverseUVBilinear, view by
// view: each view's window sum from 0, then the views added in order), Adam
// on albedo and mr.
__global__ __launch_bounds__(256) void k_pbr_tex_adam(PbrDev d) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= d.tw * d.th) {
        return;
    }
    const uint32_t npx = d.S * d.S;
    float ga[3] = {0.f, 0.f, 0.f}, gr = 0.f, gm = 0.f;
    float pa[3] = {0.f, 0.f, 0.f}, pr = 0.f, pm = 0.f;
    const uint32_t e0 = d.csr_off[i], e1 = d.csr_off[i + 1];
    uint32_t view = e0 < e1 ? d.csr[e0].x / npx : 0u;
    for (uint32_t e = e0; e < e1; e++) {
        const uint2 en = d.csr[e];
        const uint32_t ev = en.x / npx;
        if (ev != view) {
            ga[0] += pa[0];
            ga[1] += pa[1];
            ga[2] += pa[2];
            gr += pr;
            gm += pm;
            pa[0] = pa[1] = pa[2] = pr = pm = 0.f;
            view = ev;
        }
        const float w = __uint_as_float(en.y);
        const float4 g = d.gyA[en.x];
        pa[0] += g.x * w;
        pa[1] += g.y * w;
        pa[2] += g.z * w;
        pr += g.w * w;
        pm += d.gyM[en.x] * w;
    }
    ga[0] += pa[0];
    ga[1] += pa[1];
    ga[2] += pa[2];
    gr += pr;
    gm += pm;
    const float gmr[3] = {0.f, gr, gm};
    if (d.g_tex_a) {
        d.g_tex_a[i] = make_float4(ga[0], ga[1], ga[2], 0.f);
        d.g_tex_m[i] = make_float4(0.f, gr, gm, 0.f);
    }
    float bc1, bc2;
    adam_bias(d, *d.t + 1.f, &bc1, &bc2);
    adam3(d, bc1, bc2, ga, &d.albedo[i], &d.am[i], &d.av[i], true);
    adam3(d, bc1, bc2, gmr, &d.mr[i], &d.mm[i], &d.mv[i], true);
}

// The loss's next four Reduce2x2Sum levels: one workgroup per 16 x 16 block
// of a view's shading-tile partials (a `tiles` x `tiles` grid, zero outside).
__global__ __launch_bounds__(256) void k_pbr_loss_blocks(PbrDev d, uint32_t tiles) {
    __shared__ QuadLds L;
    const uint32_t nside = (tiles + 15u) / 16u;
    const uint32_t view = blockIdx.x / (nside * nside), b = blockIdx.x % (nside * nside);
    const uint32_t x = (b % nside) * 16u + (threadIdx.x & 15u);
    const uint32_t y = (b / nside) * 16u + (threadIdx.x >> 4);
    L.q[threadIdx.x] = x < tiles && y < tiles
                               ? d.loss_part[((size_t)view * tiles + y) * tiles + x]
                               : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 r = quad_reduce16(L);
    if (threadIdx.x == 0) {
        d.loss_blk[blockIdx.x] = r;
    }
}

// The loss scalar and the step counter. Per view, F::Mean of the |diff|
// image (f_ops.cpp:1045-1050): Sum's remaining Reduce2x2Sum levels over the
// block sums (an `nside` x `nside` grid, reduced 16 x 16 blocks at a time,
// block-aligned, so the quadtree is Sum's), then CompSum (from 0, components
// in order, f_ops.cpp:743-770) times 1 / (W H 3); the views' losses added by
// SumPixelWise's tree (f_ops.cpp:893-950: groups of at most four, each from 0
// in order, a lone entry passed up).
constexpr uint32_t kLossGrid = 1024;  // a level's block sums in LDS
__global__ __launch_bounds__(256) void k_pbr_loss(PbrDev d, uint32_t nside) {
    __shared__ QuadLds L;
    __shared__ float4 grid[2][kLossGrid];
    __shared__ float vl[kPbrMaxViews];
    const uint32_t t = threadIdx.x;
    for (uint32_t view = 0; view < d.n_views; view++) {
        uint32_t side = nside, cur = 0;
        // the view's block sums into LDS
        for (uint32_t i = t; i < nside * nside; i += 256u) {
            grid[0][i] = d.loss_blk[(size_t)view * nside * nside + i];
        }
        __syncthreads();
        while (side > 1) {
            const uint32_t ns = (side + 15u) / 16u;
            for (uint32_t b = 0; b < ns * ns; b++) {
                const uint32_t x = (b % ns) * 16u + (t & 15u);
                const uint32_t y = (b / ns) * 16u + (t >> 4);
                L.q[t] = x < side && y < side ? grid[cur][y * side + x]
                                              : make_float4(0.f, 0.f, 0.f, 0.f);
                const float4 r = quad_reduce16(L);
                if (t == 0) {
                    grid[cur ^ 1u][b] = r;
                }
            }
            __syncthreads();
            cur ^= 1u;
            side = ns;
        }
        if (t == 0) {
            const float4 s = grid[cur][0];
            float acc = 0.f;
            acc += s.x;
            acc += s.y;
            acc += s.z;
            vl[view] = acc * d.inv_n;
        }
        __syncthreads();
    }
    if (t == 0) {
        float lv[kPbrMaxViews];
        uint32_t n = d.n_views;
        for (uint32_t i = 0; i < n; i++) {
            lv[i] = vl[i];
        }
        while (n > 1) {
            uint32_t m = 0;
            for (uint32_t i = 0; i < n; i += 4) {
                const uint32_t k = n - i < 4u ? n - i : 4u;
                if (k == 1) {
                    lv[m++] = lv[i];
                } else {
                    float acc = 0.f;
                    for (uint32_t j = 0; j < k; j++) {
                        acc += lv[i + j];
                    }
                    lv[m++] = acc;
                }
            }
            n = m;
        }
        d.loss[0] = lv[0];
        *d.t = *d.t + 1.f;
    }
}

// Kernel list of one iteration (the pooling chain counts as one entry)
constexpr int kPbrKernels = 11;
const char* const kPbrKernelNames[kPbrKernels] = {
        "k_pbr_pool",     "k_pbr_conv_fwd", "k_pbr_shade",       "k_pbr_map_gather",
        "k_pbr_tile_sum", "k_pbr_view_sum", "k_pbr_conv_bwd",    "k_pbr_env_adam",
        "k_pbr_tex_adam", "k_pbr_loss_blocks", "k_pbr_loss"};
// index of each kernel in the launch switch
enum PbrK {
    kKPool = 0, kKConvFwd, kKShade, kKGather, kKTileSum, kKViewSum, kKConvBwd, kKEnvAdam,
    kKTexAdam, kKLossBlocks, kKLoss
};

uint32_t loss_tiles(const PbrDev& d) { return (d.S + kShadeTile - 1) / kShadeTile; }
uint32_t loss_nside(const PbrDev& d) { return (loss_tiles(d) + 15u) / 16u; }

uint32_t shade_blocks(const PbrDev& d) {
    const uint32_t tiles = (d.S + kShadeTile - 1) / kShadeTile;
    return tiles * tiles * d.n_views;
}

int launch_pbr_kernel(const PbrDev& d, hipStream_t s, int k) {
    switch (k) {
        case kKPool:
            for (uint32_t l = 1; l <= d.n_pool; l++) {
                const uint32_t n = d.pw[l] * d.ph[l];
                hipLaunchKernelGGL(k_pbr_pool, dim3(div_up(n, 256)), dim3(256), 0, s, d, l);
                DRESSI_CHECK_LAUNCH();
            }
            return DRESSI_OK;
        case kKConvFwd:
            hipLaunchKernelGGL(k_pbr_conv_fwd, dim3(d.n_ig + d.n_pg), dim3(kMvThreads), 0, s, d);
            break;
        case kKShade:
            hipLaunchKernelGGL(k_pbr_shade, dim3(shade_blocks(d)), dim3(256), 0, s, d);
            break;
        case kKGather:
            if (d.n_gitems == 0) {
                return DRESSI_OK;
            }
            hipLaunchKernelGGL(k_pbr_map_gather, dim3(d.n_gitems), dim3(256), 0, s, d);
            break;
        case kKTileSum:
            if (d.n_tsum == 0) {
                return DRESSI_OK;
            }
            hipLaunchKernelGGL(k_pbr_tile_sum, dim3(d.n_tsum), dim3(256), 0, s, d);
            break;
        case kKViewSum:
            hipLaunchKernelGGL(k_pbr_view_sum,
                               dim3(div_up(d.iw * d.ih + d.n_pref + d.ew * d.eh, 256)), dim3(256),
                               0, s, d);
            break;
        case kKConvBwd:
            hipLaunchKernelGGL(k_pbr_conv_bwd, dim3(d.n_isg + d.n_psg), dim3(kMvThreads), 0, s,
                               d);
            break;
        case kKEnvAdam:
            hipLaunchKernelGGL(k_pbr_env_adam, dim3(div_up(d.ew * d.eh, 256)), dim3(256), 0, s,
                               d);
            break;
        case kKTexAdam:
            hipLaunchKernelGGL(k_pbr_tex_adam, dim3(div_up(d.tw * d.th, 256)), dim3(256), 0, s,
                               d);
            break;
        case kKLossBlocks:
            hipLaunchKernelGGL(k_pbr_loss_blocks,
                               dim3(d.n_views * loss_nside(d) * loss_nside(d)), dim3(256), 0, s, d,
                               loss_tiles(d));
            break;
        default:
            hipLaunchKernelGGL(k_pbr_loss, dim3(1), dim3(256), 0, s, d, loss_nside(d));
            break;
    }
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

}  // namespace
}  // namespace dressi

using namespace dressi;

struct dressi_pbr_plan {
    dressi_ctx* ctx = nullptr;
    dressi_pbr_desc desc{};
    PbrDev d{};
    std::vector<void*> allocs;
    bool scene_set = false, target_set = false, state_set = false;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    hipStream_t graph_stream = nullptr;
    uint32_t csr_len = 0;
    uint64_t ml_len = 0;  // map-gradient gather list entries
    // set_scene's allocations (freed when the scene is set again)
    std::vector<void*> scene_allocs;
};

namespace {

template <typename T>
int pbr_alloc(dressi_pbr_plan* p, T** out, size_t count) {
    void* ptr = nullptr;
    DRESSI_TRY_HIP(hipMalloc(&ptr, sizeof(T) * (count ? count : 1)));
    p->allocs.push_back(ptr);
    *out = (T*)ptr;
    return DRESSI_OK;
}

template <typename T>
int pbr_upload(dressi_pbr_plan* p, T** out, const std::vector<T>& v) {
    if (int rc = pbr_alloc(p, out, v.size())) return rc;
    DRESSI_TRY_HIP(hipMemcpy(*out, v.data(), sizeof(T) * v.size(), hipMemcpyHostToDevice));
    return DRESSI_OK;
}

void pbr_drop_graph(dressi_pbr_plan* p) {
    if (p->exec) {
        hipGraphExecDestroy(p->exec);
        p->exec = nullptr;
    }
    if (p->graph) {
        hipGraphDestroy(p->graph);
        p->graph = nullptr;
    }
}

int pbr_ready(dressi_pbr_plan* p) {
    DRESSI_REQUIRE(p, "NULL plan");
    DRESSI_REQUIRE(p->scene_set, "dressi_pbr_set_scene() must be called before stepping");
    DRESSI_REQUIRE(p->target_set, "dressi_pbr_set_target() must be called before stepping");
    DRESSI_REQUIRE(p->state_set, "dressi_pbr_set_state() must be called before stepping");
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    return DRESSI_OK;
}

int pbr_enqueue(dressi_pbr_plan* p, hipStream_t s) {
    for (int k = 0; k < kPbrKernels; k++) {
        if (int rc = launch_pbr_kernel(p->d, s, k)) return rc;
    }
    return DRESSI_OK;
}

// One iteration for graph capture: after the shading, the texture gather +
// Adam and the loss's block sums run on `side` beside the environment's chain
// (map gathers, tile and view sums, transposed convolutions, env Adam): the
// two read and write disjoint buffers (both only read t), and both join
// before the loss kernel advances t.
int pbr_enqueue_forked(dressi_pbr_plan* p, hipStream_t s, hipStream_t side, hipEvent_t fork,
                       hipEvent_t join) {
    for (int k : {kKPool, kKConvFwd, kKShade}) {
        if (int rc = launch_pbr_kernel(p->d, s, k)) return rc;
    }
    DRESSI_TRY_HIP(hipEventRecord(fork, s));
    DRESSI_TRY_HIP(hipStreamWaitEvent(side, fork, 0));
    if (int rc = launch_pbr_kernel(p->d, side, kKTexAdam)) return rc;
    if (int rc = launch_pbr_kernel(p->d, side, kKLossBlocks)) return rc;
    DRESSI_TRY_HIP(hipEventRecord(join, side));
    for (int k : {kKGather, kKTileSum, kKViewSum, kKConvBwd, kKEnvAdam}) {
        if (int rc = launch_pbr_kernel(p->d, s, k)) return rc;
    }
    DRESSI_TRY_HIP(hipStreamWaitEvent(s, join, 0));
    return launch_pbr_kernel(p->d, s, kKLoss);
}

// host VEC3 {n} -> device float4 {n} (w = 0)
int upload3(float4* dst, const float* src, size_t n) {
    std::vector<float4> v(n);
    for (size_t i = 0; i < n; i++) {
        v[i] = make_float4(src[i * 3 + 0], src[i * 3 + 1], src[i * 3 + 2], 0.f);
    }
    DRESSI_TRY_HIP(hipMemcpy(dst, v.data(), sizeof(float4) * n, hipMemcpyHostToDevice));
    return DRESSI_OK;
}

int download3(float* dst, const float4* src, size_t n) {
    std::vector<float4> v(n);
    DRESSI_TRY_HIP(hipMemcpy(v.data(), src, sizeof(float4) * n, hipMemcpyDeviceToHost));
    for (size_t i = 0; i < n; i++) {
        dst[i * 3 + 0] = v[i].x;
        dst[i * 3 + 1] = v[i].y;
        dst[i * 3 + 2] = v[i].z;
    }
    return DRESSI_OK;
}

// The IBL pass of the target: the env's pooled sources and maps through the
// iteration's pool / conv kernels on temporary buffers
int render_target(dressi_pbr_plan* p, const float* gt_env) {
    PbrDev t = p->d;
    const size_t ne = (size_t)t.ew * t.eh;
    std::vector<void*> tmp;
    auto talloc = [&](void** q, size_t b) -> int {
        DRESSI_TRY_HIP(hipMalloc(q, b ? b : 4));
        tmp.push_back(*q);
        return DRESSI_OK;
    };
    int rc = DRESSI_OK;
    void* q = nullptr;
    if (!rc) rc = talloc(&q, sizeof(float4) * ne);
    if (!rc) {
        t.pool[0] = (float4*)q;
        t.env = (float4*)q;
        rc = upload3(t.pool[0], gt_env, ne);
    }
    for (uint32_t l = 1; l <= t.n_pool && !rc; l++) {
        rc = talloc(&q, sizeof(float4) * t.pw[l] * t.ph[l]);
        t.pool[l] = (float4*)q;
    }
    if (!rc) rc = talloc(&q, sizeof(float4) * t.iw * t.ih);
    t.irr = (float4*)q;
    if (!rc) rc = talloc(&q, sizeof(float4) * t.n_pref);
    t.pref = (float4*)q;
    t.target_mode = 1;
    hipStream_t s = p->ctx->stream;
    if (!rc) rc = launch_pbr_kernel(t, s, kKPool);
    if (!rc) rc = launch_pbr_kernel(t, s, kKConvFwd);
    if (!rc) rc = launch_pbr_kernel(t, s, kKShade);
    hipError_t e = hipStreamSynchronize(s);
    for (void* b : tmp) hipFree(b);
    if (!rc && e != hipSuccess) {
        set_error("target render failed: %s", hipGetErrorString(e));
        rc = DRESSI_ERR_HIP;
    }
    return rc;
}

// Static gather lists of the map-gradient VJPs (see k_pbr_map_gather) and the
// bookkeeping of their sums: per map the EquirectSampleBwd layout, every
// (view, pixel, map, tap) entry keyed by its bucket, a stable radix sort
// (pixel order kept within a bucket), bucket offsets from the counts, the
// tile-sum work items. Allocations go to p->scene_allocs.
int build_map_lists(dressi_pbr_plan* p) {
    PbrDev& d = p->d;
    hipStream_t s = p->ctx->stream;
    const uint32_t N = d.n_views, S = d.S;
    const size_t npx = (size_t)S * S;
    for (void* q : p->scene_allocs) hipFree(q);
    p->scene_allocs.clear();
    auto salloc = [&](void** q, size_t b) -> int {
        DRESSI_TRY_HIP(hipMalloc(q, b ? b : 4));
        p->scene_allocs.push_back(*q);
        return DRESSI_OK;
    };
    // EquirectSampleBwd's band count for a map of w x h over S dir rows
    const auto bands = [&](uint32_t w, uint32_t h) {
        uint32_t k = 1;
        while ((size_t)w * h * k < 65536 && k < S) {
            k *= 2;
        }
        return k;
    };
    std::vector<MapInfo> mis;
    uint64_t nb = 0, nt = 0;
    const auto add = [&](uint32_t w, uint32_t h, uint32_t kind, uint32_t level) {
        MapInfo m{};
        m.w = w;
        m.h = h;
        m.T = w * h;
        m.k = bands(w, h);
        m.rows = (S + m.k - 1) / m.k;
        m.bucket0 = (uint32_t)nb;
        m.tot0 = (uint32_t)nt;
        m.kind = kind;
        m.level = level;
        nb += (uint64_t)N * m.k * m.T;
        nt += (uint64_t)N * m.T;
        mis.push_back(m);
    };
    add(d.iw, d.ih, 0, 0);
    for (uint32_t i = 0; i < d.levels; i++) {
        add(d.lw[i], d.lh[i], 1, i);
    }
    add(d.ew, d.eh, 2, 0);
    DRESSI_REQUIRE(nb < (1ull << 31), "too many map-gradient buckets");
    uint32_t key_bits = 1;
    while ((1ull << key_bits) <= nb) {
        key_bits++;
    }
    const uint32_t n_maps = (uint32_t)mis.size();
    const size_t items = (size_t)N * npx * n_maps * 4;
    int rc = DRESSI_OK;
    void *minfo = nullptr, *off = nullptr, *part = nullptr, *tot = nullptr, *work = nullptr;
    if (!rc) rc = salloc(&minfo, sizeof(MapInfo) * n_maps);
    if (!rc) rc = salloc(&part, sizeof(float4) * nb);
    if (!rc) rc = salloc(&tot, sizeof(float4) * nt);
    if (!rc) rc = salloc(&off, sizeof(uint32_t) * (nb + 1));
    if (rc) return rc;
    DRESSI_TRY_HIP(hipMemcpy(minfo, mis.data(), sizeof(MapInfo) * n_maps, hipMemcpyHostToDevice));
    // temporaries: keys / values (two copies for the sort), counts, sort scratch
    std::vector<void*> tmp;
    auto talloc = [&](void** q, size_t b) -> int {
        DRESSI_TRY_HIP(hipMalloc(q, b ? b : 4));
        tmp.push_back(*q);
        return DRESSI_OK;
    };
    // background pixels that sample the env, per view (the env lists'
    // positions)
    std::vector<uint32_t> n_bg(N, 0), bg_base(N + 1, 0);
    void *bgflag = nullptr, *bgidx = nullptr, *bgscr = nullptr, *bgpix = nullptr;
    if (!rc) rc = talloc(&bgflag, sizeof(uint32_t) * N * npx);
    if (!rc) rc = talloc(&bgidx, sizeof(uint32_t) * N * npx);
    if (!rc) {
        size_t sb = 0;
        hipLaunchKernelGGL(k_pbr_bg_flags, dim3(div_up((uint32_t)(N * npx), 256)), dim3(256), 0, s,
                           d.st0, (size_t)N * npx, (uint32_t*)bgflag);
        hipError_t e = hipGetLastError();
        if (e == hipSuccess) {
            e = hipcub::DeviceScan::ExclusiveSum(nullptr, sb, (const uint32_t*)bgflag,
                                                 (uint32_t*)bgidx, (int)npx, s);
        }
        if (e == hipSuccess) e = hipMalloc(&bgscr, sb ? sb : 4);
        if (e == hipSuccess) tmp.push_back(bgscr);
        for (uint32_t v = 0; v < N && e == hipSuccess; v++) {
            e = hipcub::DeviceScan::ExclusiveSum(bgscr, sb, (const uint32_t*)bgflag + v * npx,
                                                 (uint32_t*)bgidx + v * npx, (int)npx, s);
            uint32_t last[2] = {0, 0};
            if (e == hipSuccess) {
                e = hipMemcpyAsync(&last[0], (uint32_t*)bgidx + v * npx + npx - 1, 4,
                                   hipMemcpyDeviceToHost, s);
            }
            if (e == hipSuccess) {
                e = hipMemcpyAsync(&last[1], (uint32_t*)bgflag + v * npx + npx - 1, 4,
                                   hipMemcpyDeviceToHost, s);
            }
            if (e == hipSuccess) e = hipStreamSynchronize(s);
            n_bg[v] = last[0] + last[1];
            bg_base[v + 1] = bg_base[v] + n_bg[v];
        }
        if (e != hipSuccess) {
            set_error("background pixel lists failed: %s", hipGetErrorString(e));
            rc = DRESSI_ERR_HIP;
        }
    }
    if (!rc) rc = salloc(&bgpix, sizeof(uint32_t) * bg_base[N]);
    void* bgbase = nullptr;
    if (!rc) rc = salloc(&bgbase, sizeof(uint32_t) * (N + 1));
    if (!rc && hipMemcpy(bgbase, bg_base.data(), sizeof(uint32_t) * (N + 1),
                         hipMemcpyHostToDevice) != hipSuccess) {
        set_error("background pixel bases upload failed");
        rc = DRESSI_ERR_HIP;
    }
    for (uint32_t v = 0; v < N && !rc; v++) {
        hipLaunchKernelGGL(k_pbr_bg_fill, dim3(div_up((uint32_t)npx, 256)), dim3(256), 0, s,
                           (const uint32_t*)bgflag + v * npx, (const uint32_t*)bgidx + v * npx,
                           (uint32_t)npx, bg_base[v], (uint32_t*)bgpix);
    }
    void *k0 = nullptr, *k1 = nullptr, *v0 = nullptr, *v1 = nullptr, *cnt = nullptr, *scr = nullptr;
    if (!rc) rc = talloc(&k0, sizeof(uint32_t) * items);
    if (!rc) rc = talloc(&k1, sizeof(uint32_t) * items);
    if (!rc) rc = talloc(&v0, sizeof(uint32_t) * items);
    if (!rc) rc = talloc(&v1, sizeof(uint32_t) * items);
    if (!rc) rc = talloc(&cnt, sizeof(uint32_t) * nb);
    size_t scr_bytes = 0;
    if (!rc) {
        hipError_t e = hipMemsetAsync(cnt, 0, sizeof(uint32_t) * nb, s);
        ListArgs la{};
        la.st0 = d.st0;
        la.st2 = d.st2;
        la.minfo = (const MapInfo*)minfo;
        la.n_maps = n_maps;
        la.n_views = N;
        la.S = S;
        la.no_key = (uint32_t)((1ull << key_bits) - 1);
        la.bg_idx = (const uint32_t*)bgidx;
        la.keys = (uint32_t*)k0;
        la.vals = (uint32_t*)v0;
        la.count = (uint32_t*)cnt;
        if (e == hipSuccess) {
            hipLaunchKernelGGL(k_pbr_list_keys, dim3(div_up((uint32_t)(N * npx), 256)), dim3(256), 0,
                               s, la);
            e = hipGetLastError();
        }
        if (e == hipSuccess) {
            e = hipcub::DeviceRadixSort::SortPairs(nullptr, scr_bytes, (const uint32_t*)k0,
                                                   (uint32_t*)k1, (const uint32_t*)v0,
                                                   (uint32_t*)v1, (int)items, 0, (int)key_bits, s);
        }
        if (e != hipSuccess) {
            set_error("map gather list keys failed: %s", hipGetErrorString(e));
            rc = DRESSI_ERR_HIP;
        }
    }
    if (!rc) rc = talloc(&scr, scr_bytes);
    std::vector<uint32_t> c(nb), o(nb + 1);
    if (!rc) {
        hipError_t e = hipcub::DeviceRadixSort::SortPairs(
                scr, scr_bytes, (const uint32_t*)k0, (uint32_t*)k1, (const uint32_t*)v0,
                (uint32_t*)v1, (int)items, 0, (int)key_bits, s);
        if (e == hipSuccess) e = hipMemcpyAsync(c.data(), cnt, sizeof(uint32_t) * nb,
                                                hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) {
            set_error("map gather list sort failed: %s", hipGetErrorString(e));
            rc = DRESSI_ERR_HIP;
        }
    }
    uint64_t total = 0;
    if (!rc) {
        for (size_t i = 0; i < nb; i++) {
            o[i] = (uint32_t)total;
            total += c[i];
        }
        o[nb] = (uint32_t)total;
        if (total >= (1ull << 32)) {
            set_error("map gather lists too long (%llu entries)", (unsigned long long)total);
            rc = DRESSI_ERR_UNSUPPORTED;
        }
    }
    void* ent = v1;  // the sorted entries (set-up only)
    if (!rc) {
        hipError_t e = hipMemcpyAsync(off, o.data(), sizeof(uint32_t) * (nb + 1),
                                      hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) {
            set_error("map gather list fill failed: %s", hipGetErrorString(e));
            rc = DRESSI_ERR_HIP;
        }
    }
    // the gather's workgroups: per (map, view, band) its non-empty buckets in
    // bucket order, at most kGatherChains per workgroup, over the band's
    // positions; the longest first. Then the per-chunk entry runs: first
    // entries and counts per (item, chunk, bucket), their exclusive scan in
    // item / chunk / bucket order, the entries copied there. The partials of
    // the empty buckets stay 0 (cleared here).
    void *order = nullptr, *gbuf = nullptr, *coff = nullptr, *ment = nullptr;
    std::vector<GatherItem> gi;
    if (!rc) {
        std::vector<uint32_t> ord;
        uint64_t n_fo = 0, n_c = 0;
        // the positions of (view, band) vb, as band_pos derives them
        const auto band_npos = [&](const MapInfo& mi, uint32_t vb) -> uint32_t {
            if (mi.kind == 2) {
                return n_bg[vb / mi.k];
            }
            const uint32_t band = vb % mi.k;
            const uint32_t r0 = std::min(band * mi.rows, S);
            const uint32_t r1 = std::min(r0 + mi.rows, S);
            return (r1 - r0) * S;
        };
        GatherItem cur{};
        uint32_t cur_max = 0;
        uint64_t n_bmw = 0;  // bitmap words of the position-list workgroups
        // chunks per workgroup: kGatherMaxChunks, or DRESSI_PBR_GATHER_CHUNKS
        // (tests use 1 to take position lists at small sizes)
        uint64_t max_chunks = kGatherMaxChunks;
        if (const char* ev = getenv("DRESSI_PBR_GATHER_CHUNKS")) {
            const long v = strtol(ev, nullptr, 10);
            if (v >= 1 && v <= 4096) max_chunks = (uint64_t)v;
        }
        const uint64_t pos_cap = (uint64_t)kGatherChunk * max_chunks;
        const auto flush = [&]() {
            if (cur.na == 0) {
                cur = GatherItem{};
                cur_max = 0;
                return;
            }
            cur.P = kGatherChunk / cur.nb;
            cur.nch = (cur_max + cur.P - 1) / cur.P;
            cur.bmo = kBandMode;
            gi.push_back(cur);
            cur = GatherItem{};
            cur_max = 0;
        };
        for (uint32_t m = 0; m < n_maps; m++) {
            const MapInfo& mi = mis[m];
            for (uint32_t vb = 0; vb < N * mi.k; vb++) {
                const uint64_t b0 = mi.bucket0 + (uint64_t)vb * mi.T;
                const uint32_t first = (uint32_t)ord.size();
                for (uint32_t t = 0; t < mi.T; t++) {
                    if (c[b0 + t]) ord.push_back((uint32_t)(b0 + t));
                }
                const uint32_t n_here = (uint32_t)ord.size() - first;
                const uint32_t npos = band_npos(mi, vb);
                if (n_here == 0) {
                    flush();  // a workgroup's bands are consecutive and non-empty
                    continue;
                }
                if ((uint64_t)npos > pos_cap) {
                    // position-list workgroups: the band's buckets by texel
                    // tile (at most kGatherTile^2 = kGatherChains each)
                    flush();
                    const uint32_t tx = (mi.w + kGatherTile - 1) / kGatherTile;
                    const auto tile_of = [&](uint32_t b) {
                        const uint32_t t = (b - mi.bucket0) % mi.T;
                        return (t / mi.w) / kGatherTile * tx + (t % mi.w) / kGatherTile;
                    };
                    std::stable_sort(ord.begin() + first, ord.end(),
                                     [&](uint32_t x, uint32_t y) { return tile_of(x) < tile_of(y); });
                    for (uint32_t a = 0; a < n_here;) {
                        uint32_t e = a + 1;
                        while (e < n_here && tile_of(ord[first + e]) == tile_of(ord[first + a])) {
                            e++;
                        }
                        GatherItem li{};
                        li.m = m;
                        li.vb0 = vb;
                        li.nb = 1;
                        li.P = kGatherChunk;
                        li.a0 = first + a;
                        li.na = e - a;
                        li.bmo = (uint32_t)n_bmw;
                        n_bmw += (npos + 31u) / 32u;
                        gi.push_back(li);
                        a = e;
                    }
                    continue;
                }
                if (n_here > kGatherChains) {
                    // a band of its own, split into workgroups of kGatherChains
                    flush();
                    for (uint32_t a = 0; a < n_here; a += kGatherChains) {
                        cur.m = m;
                        cur.vb0 = vb;
                        cur.nb = 1;
                        cur.a0 = first + a;
                        cur.na = std::min(kGatherChains, n_here - a);
                        cur_max = npos;
                        flush();
                    }
                    continue;
                }
                if (cur.na + n_here > kGatherChains || cur.nb == kGatherBands ||
                    (uint64_t)(cur.nb + 1) * std::max(cur_max, npos) > pos_cap) {
                    flush();
                }
                if (cur.na == 0) {
                    cur.m = m;
                    cur.vb0 = vb;
                    cur.a0 = first;
                }
                cur.nb++;
                cur.na += n_here;
                cur_max = std::max(cur_max, npos);
            }
            flush();
        }
        // position-list workgroups: bitmaps of the positions their entries
        // read, the word prefixes, the lengths (to the host: they set nch)
        // and the lists
        void *bm = nullptr, *wpre = nullptr, *lgi = nullptr, *lnpl = nullptr, *plist = nullptr;
        if (!rc) rc = salloc(&order, sizeof(uint32_t) * std::max<size_t>(ord.size(), 1));
        if (!rc && hipMemcpy(order, ord.data(), sizeof(uint32_t) * ord.size(),
                             hipMemcpyHostToDevice) != hipSuccess) {
            set_error("map gather bucket order upload failed");
            rc = DRESSI_ERR_HIP;
        }
        uint32_t max_na0 = 1;
        for (const GatherItem& g : gi) max_na0 = std::max(max_na0, g.na);
        if (!rc && n_bmw) {
            std::vector<uint32_t> npl(gi.size(), 0);
            rc = talloc(&bm, sizeof(uint32_t) * n_bmw);
            if (!rc) rc = talloc(&wpre, sizeof(uint32_t) * n_bmw);
            if (!rc) rc = talloc(&lgi, sizeof(GatherItem) * gi.size());
            if (!rc) rc = talloc(&lnpl, sizeof(uint32_t) * gi.size());
            hipError_t e = hipSuccess;
            if (!rc) {
                e = hipMemcpy(lgi, gi.data(), sizeof(GatherItem) * gi.size(),
                              hipMemcpyHostToDevice);
                if (e == hipSuccess) e = hipMemsetAsync(bm, 0, sizeof(uint32_t) * n_bmw, s);
                if (e == hipSuccess) e = hipMemsetAsync(lnpl, 0, sizeof(uint32_t) * gi.size(), s);
                if (e == hipSuccess) {
                    hipLaunchKernelGGL(k_pbr_list_bits,
                                       dim3(div_up(max_na0, 256), (uint32_t)gi.size()), dim3(256),
                                       0, s, (const GatherItem*)lgi, (uint32_t)gi.size(),
                                       (const MapInfo*)minfo, S, (const uint32_t*)bgbase,
                                       (const uint32_t*)order, (const uint32_t*)off,
                                       (const uint32_t*)ent, (uint32_t*)bm);
                    e = hipGetLastError();
                }
                if (e == hipSuccess) {
                    hipLaunchKernelGGL(k_pbr_list_count, dim3((uint32_t)gi.size()), dim3(256), 0,
                                       s, (const GatherItem*)lgi, (uint32_t)gi.size(),
                                       (const MapInfo*)minfo, S, (const uint32_t*)bgbase,
                                       (const uint32_t*)bm, (uint32_t*)wpre, (uint32_t*)lnpl);
                    e = hipGetLastError();
                }
                if (e == hipSuccess) e = hipMemcpyAsync(npl.data(), lnpl,
                                                        sizeof(uint32_t) * gi.size(),
                                                        hipMemcpyDeviceToHost, s);
                if (e == hipSuccess) e = hipStreamSynchronize(s);
            }
            uint64_t n_pl = 0;
            if (!rc && e == hipSuccess) {
                for (size_t i = 0; i < gi.size(); i++) {
                    if (gi[i].bmo == kBandMode) continue;
                    gi[i].npl = npl[i];
                    gi[i].pl0 = (uint32_t)n_pl;
                    gi[i].nch = (npl[i] + gi[i].P - 1) / gi[i].P;
                    n_pl += npl[i];
                }
                if (n_pl >= (1ull << 31)) {
                    set_error("map gather position lists too long");
                    rc = DRESSI_ERR_UNSUPPORTED;
                }
            }
            if (!rc && e == hipSuccess) rc = salloc(&plist, sizeof(uint32_t) * n_pl);
            if (!rc && e == hipSuccess) {
                e = hipMemcpy(lgi, gi.data(), sizeof(GatherItem) * gi.size(),
                              hipMemcpyHostToDevice);
                if (e == hipSuccess) {
                    hipLaunchKernelGGL(k_pbr_list_fill, dim3(16, (uint32_t)gi.size()), dim3(256), 0,
                                       s, (const GatherItem*)lgi, (uint32_t)gi.size(),
                                       (const MapInfo*)minfo, S, (const uint32_t*)bgbase,
                                       (const uint32_t*)bgpix, (const uint32_t*)bm,
                                       (const uint32_t*)wpre, (uint32_t*)plist);
                    e = hipGetLastError();
                }
            }
            if (!rc && e != hipSuccess) {
                set_error("map gather position lists failed: %s", hipGetErrorString(e));
                rc = DRESSI_ERR_HIP;
            }
        }
        d.plist = (const uint32_t*)plist;
        // chunk tables: per item (nch + 1) first entries and nch counts per bucket
        for (GatherItem& g : gi) {
            g.c0 = (uint32_t)n_c;
            g.f0 = (uint32_t)n_fo;
            n_c += (uint64_t)g.nch * g.na;
            n_fo += (uint64_t)(g.nch + 1) * g.na;
        }
        if (n_fo >= (1ull << 31)) {
            set_error("map gather chunk tables too large");
            rc = DRESSI_ERR_UNSUPPORTED;
        }
        std::stable_sort(gi.begin(), gi.end(), [](const GatherItem& x, const GatherItem& y) {
            return x.nch > y.nch;
        });
        uint32_t max_na = 1;
        for (const GatherItem& g : gi) max_na = std::max(max_na, g.na);
        void *fo = nullptr, *ccnt = nullptr, *cscr = nullptr;
        if (!rc) rc = salloc(&gbuf, sizeof(GatherItem) * std::max<size_t>(gi.size(), 1));
        if (!rc) rc = salloc(&coff, sizeof(uint32_t) * (n_c + 1));
        if (!rc) rc = salloc(&ment, sizeof(uint16_t) * (total + 16));  // + the last 16-byte word
        if (!rc) rc = talloc(&fo, sizeof(uint32_t) * n_fo);
        if (!rc) rc = talloc(&ccnt, sizeof(uint32_t) * (n_c + 1));
        size_t cs_bytes = 0;
        if (!rc) {
            hipError_t e = hipMemcpy(gbuf, gi.data(), sizeof(GatherItem) * gi.size(),
                                     hipMemcpyHostToDevice);
            if (e == hipSuccess) e = hipMemset(part, 0, sizeof(float4) * nb);
            if (e == hipSuccess) e = hipMemset(tot, 0, sizeof(float4) * nt);
            if (e == hipSuccess) e = hipMemset((uint32_t*)ccnt + n_c, 0, sizeof(uint32_t));
            if (e == hipSuccess && !gi.empty()) {
                hipLaunchKernelGGL(k_pbr_chunk_first,
                                   dim3(div_up(max_na, 256), (uint32_t)gi.size()), dim3(256), 0,
                                   s, (const GatherItem*)gbuf, (uint32_t)gi.size(),
                                   (const MapInfo*)minfo, S, (const uint32_t*)bgbase,
                                   (const uint32_t*)order, (const uint32_t*)off,
                                   (const uint32_t*)ent, (const uint32_t*)bm,
                                   (const uint32_t*)wpre, (uint32_t*)fo, (uint32_t*)ccnt);
                e = hipGetLastError();
            }
            if (e == hipSuccess) {
                e = hipcub::DeviceScan::ExclusiveSum(nullptr, cs_bytes, (const uint32_t*)ccnt,
                                                     (uint32_t*)coff, (int)(n_c + 1), s);
            }
            if (e == hipSuccess) e = hipMalloc(&cscr, cs_bytes ? cs_bytes : 4);
            if (e == hipSuccess) {
                tmp.push_back(cscr);
                e = hipcub::DeviceScan::ExclusiveSum(cscr, cs_bytes, (const uint32_t*)ccnt,
                                                     (uint32_t*)coff, (int)(n_c + 1), s);
            }
            if (e == hipSuccess && !gi.empty()) {
                hipLaunchKernelGGL(k_pbr_chunk_fill,
                                   dim3(div_up(max_na, 256), (uint32_t)gi.size()), dim3(256), 0,
                                   s, (const GatherItem*)gbuf, (uint32_t)gi.size(),
                                   (const MapInfo*)minfo, S, (const uint32_t*)bgbase,
                                   (const uint32_t*)order, (const uint32_t*)ent,
                                   (const uint32_t*)bm, (const uint32_t*)wpre,
                                   (const uint32_t*)fo, (const uint32_t*)coff, (uint16_t*)ment);
                e = hipGetLastError();
            }
            if (e == hipSuccess) e = hipStreamSynchronize(s);
            // dispatch order: the longest workgroups first. A workgroup's
            // time is close to kGatherChunkCost per chunk (staging and
            // synchronisation) plus one unit per entry of each chunk's
            // longest bucket (its lanes wait for the longest sequential
            // sum): measured on the 1024^2 x 6-view fit, 6.0 us per chunk
            // and 37 ns per entry.
            std::vector<uint32_t> hc(n_c);
            if (e == hipSuccess && n_c) {
                e = hipMemcpy(hc.data(), ccnt, sizeof(uint32_t) * n_c, hipMemcpyDeviceToHost);
            }
            if (e == hipSuccess && !gi.empty()) {
                std::vector<uint64_t> cost(gi.size());
                for (size_t i = 0; i < gi.size(); i++) {
                    const GatherItem& g = gi[i];
                    uint64_t t = (uint64_t)kGatherChunkCost * g.nch;
                    for (uint32_t c = 0; c < g.nch; c++) {
                        const uint32_t* q = hc.data() + g.c0 + (size_t)c * g.na;
                        t += *std::max_element(q, q + g.na);
                    }
                    cost[i] = t;
                }
                std::vector<uint32_t> idx(gi.size());
                for (uint32_t i = 0; i < (uint32_t)gi.size(); i++) idx[i] = i;
                std::stable_sort(idx.begin(), idx.end(),
                                 [&](uint32_t x, uint32_t y) { return cost[x] > cost[y]; });
                std::vector<GatherItem> sorted(gi.size());
                for (size_t i = 0; i < gi.size(); i++) sorted[i] = gi[idx[i]];
                gi.swap(sorted);
                e = hipMemcpy(gbuf, gi.data(), sizeof(GatherItem) * gi.size(),
                              hipMemcpyHostToDevice);
            }
            if (e != hipSuccess) {
                set_error("map gather work set-up failed: %s", hipGetErrorString(e));
                rc = DRESSI_ERR_HIP;
            }
        }
    }
    for (void* q : tmp) hipFree(q);
    if (rc) return rc;
    // tile sums: per map with k > 1, per view, runs of <= 256 texels, short
    // enough that a workgroup stages its k bands in about two rounds (a
    // round's loads are a round trip; maps with many bands take short runs)
    std::vector<uint4> wk;
    for (uint32_t m = 0; m < n_maps; m++) {
        if (mis[m].k == 1) continue;
        const uint32_t fit = std::max<uint32_t>(8u, 2u * kTileSumLds / mis[m].k);
        const uint32_t run = std::min<uint32_t>({mis[m].T, 256u, fit});
        for (uint32_t v = 0; v < N; v++) {
            for (uint32_t t0 = 0; t0 < mis[m].T; t0 += run) {
                wk.push_back(make_uint4(m, v, t0, std::min(run, mis[m].T - t0)));
            }
        }
    }
    if (!wk.empty()) {
        if ((rc = salloc(&work, sizeof(uint4) * wk.size()))) return rc;
        DRESSI_TRY_HIP(hipMemcpy(work, wk.data(), sizeof(uint4) * wk.size(),
                                 hipMemcpyHostToDevice));
    }
    d.minfo = (const MapInfo*)minfo;
    d.n_maps = n_maps;
    d.n_buckets = (uint32_t)nb;
    d.n_tot = (uint32_t)nt;
    d.ml_off = (const uint32_t*)off;
    d.ml_order = (const uint32_t*)order;
    d.bg_pix = (const uint32_t*)bgpix;
    d.bg_base = (const uint32_t*)bgbase;
    d.gitems = (const GatherItem*)gbuf;
    d.n_gitems = (uint32_t)gi.size();
    d.coff = (const uint32_t*)coff;
    d.mg_ent = (const uint16_t*)ment;
    d.mpart = (float4*)part;
    d.mtot = (float4*)tot;
    d.tsum_work = (const uint4*)work;
    d.n_tsum = (uint32_t)wk.size();
    p->ml_len = total;
    return DRESSI_OK;
}

}  // namespace

extern "C" {

int dressi_pbr_create(dressi_ctx* ctx, const dressi_pbr_desc* desc, dressi_pbr_plan** out) {
    DRESSI_REQUIRE(ctx && desc && out, "bad arguments");
    DRESSI_REQUIRE(desc->n_verts > 0 && desc->n_faces > 0, "empty mesh");
    DRESSI_REQUIRE(desc->n_views >= 1 && desc->n_views <= kPbrMaxViews,
                   "n_views must be in [1, %u]", kPbrMaxViews);
    DRESSI_REQUIRE(desc->width > 0 && desc->width == desc->height,
                   "the screen must be square (width == height > 0)");
    // the map-gradient list set-up sorts (pixel, map, tap) entries of every
    // view with 32-bit item counts
    DRESSI_REQUIRE((uint64_t)desc->n_views * desc->width * desc->height * (kPbrMaxLevels + 2) * 4 <
                           (1ull << 31),
                   "too many pixels (views x width x height x (levels + 2) x 4 must be < 2^31)");
    // the loss kernel keeps a level of 16 x 16-tile block sums in LDS
    DRESSI_REQUIRE(desc->width <= 8192, "the screen must be at most 8192 px wide");
    DRESSI_REQUIRE(desc->tex_w > 0 && desc->tex_h > 0 &&
                           (uint64_t)desc->tex_w * desc->tex_h < (1ull << 28),
                   "bad texture size");
    DRESSI_REQUIRE(desc->env_w > 0 && desc->env_h > 0 &&
                           desc->env_w < 8192 && desc->env_h < 8192,
                   "bad env size");
    DRESSI_REQUIRE(desc->levels >= 2 && desc->levels <= kPbrMaxLevels,
                   "levels must be in [2, %u]", kPbrMaxLevels);
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    dressi_pbr_plan* p = new dressi_pbr_plan();
    p->ctx = ctx;
    p->desc = *desc;
    PbrDev& d = p->d;
    d.n_views = desc->n_views;
    d.S = desc->width;
    d.tw = desc->tex_w;
    d.th = desc->tex_h;
    d.ew = desc->env_w;
    d.eh = desc->env_h;
    d.levels = desc->levels;
    d.lr = desc->lr;
    d.b1 = desc->beta1;
    d.b2 = desc->beta2;
    d.eps = desc->eps;
    d.inv_n = 1.f / ((float)d.S * (float)d.S * 3.f);
    // pooling chain (src/core/ibl.cpp:14-20): irradiance source <= 64 x 32,
    // prefilter source <= 128 x 64 (halving, sizes rounding up)
    d.pw[0] = d.ew;
    d.ph[0] = d.eh;
    uint32_t n = 0;
    while ((d.pw[n] > 64 || d.ph[n] > 32) && n < kPbrMaxPool) {
        d.pw[n + 1] = (d.pw[n] + 1) / 2;
        d.ph[n + 1] = (d.ph[n] + 1) / 2;
        n++;
    }
    d.n_pool = n;
    d.irr_pool = n;
    d.pref_pool = 0;
    while (d.pw[d.pref_pool] > 128 || d.ph[d.pref_pool] > 64) d.pref_pool++;
    d.isw = d.pw[d.irr_pool];
    d.ish = d.ph[d.irr_pool];
    d.psw = d.pw[d.pref_pool];
    d.psh = d.ph[d.pref_pool];
    d.iw = 32;
    d.ih = 16;
    d.irr_scale = kIblTwoPi / ((float)d.isw * (float)d.ish);
    uint32_t w = std::min(128u, d.psw), h = std::min(64u, d.psh), off = 0;
    for (uint32_t i = 0; i < d.levels; i++) {
        d.lw[i] = w;
        d.lh[i] = h;
        d.loff[i] = off;
        const float r = (float)i / (float)(d.levels - 1);
        const float rr = r > 0.045f ? r : 0.045f;
        d.alpha[i] = rr * rr;
        off += w * h;
        w = w > 1 ? w / 2 : 1;
        h = h > 1 ? h / 2 : 1;
    }
    d.n_pref = off;
    std::vector<uint4> ltab(d.levels);
    for (uint32_t i = 0; i < d.levels; i++) ltab[i] = make_uint4(d.lw[i], d.lh[i], d.loff[i], 0u);
    d.lutw = 256;
    d.luth = 256;
    const size_t N = d.n_views, npx = (size_t)d.S * d.S, T = (size_t)d.tw * d.th;
    const size_t E = (size_t)d.ew * d.eh;
    int rc = DRESSI_OK;
    float4* st = nullptr;
    if (!rc) rc = pbr_alloc(p, &st, N * npx * 3);
    d.st0 = st;
    d.st1 = st + N * npx;
    d.st2 = st + 2 * N * npx;
    if (!rc) rc = pbr_alloc(p, &d.target, N * npx);
    for (float4** q : {&d.albedo, &d.mr, &d.am, &d.av, &d.mm, &d.mv}) {
        if (!rc) rc = pbr_alloc(p, q, T);
    }
    for (float4** q : {&d.env, &d.em, &d.ev}) {
        if (!rc) rc = pbr_alloc(p, q, E);
    }
    d.pool[0] = d.env;
    for (uint32_t l = 1; l <= d.n_pool && !rc; l++) {
        rc = pbr_alloc(p, &d.pool[l], (size_t)d.pw[l] * d.ph[l]);
    }
    if (!rc) rc = pbr_alloc(p, &d.t, 1);
    if (!rc) rc = pbr_alloc(p, &d.done, 1);
    if (!rc) rc = pbr_alloc(p, &d.irr, (size_t)d.iw * d.ih);
    if (!rc) rc = pbr_alloc(p, &d.pref, d.n_pref);
    if (!rc) rc = pbr_alloc(p, &d.g_irr, (size_t)d.iw * d.ih);
    if (!rc) rc = pbr_alloc(p, &d.g_pref, d.n_pref);
    if (!rc) rc = pbr_alloc(p, &d.g_bg, E);
    if (!rc) rc = pbr_alloc(p, &d.g_isrc, (size_t)d.isw * d.ish);
    if (!rc) rc = pbr_alloc(p, &d.g_psrc, (size_t)d.psw * d.psh);
    if (!rc) rc = pbr_alloc(p, &d.gyA, N * npx);
    if (!rc) rc = pbr_alloc(p, &d.gyM, N * npx);
    if (!rc) rc = pbr_alloc(p, &d.mgA, N * npx);
    if (!rc) rc = pbr_alloc(p, &d.mgB, N * npx);
    if (!rc) rc = pbr_alloc(p, &d.loss_part, shade_blocks(d));
    if (!rc) rc = pbr_alloc(p, &d.loss_blk, (size_t)d.n_views * loss_nside(d) * loss_nside(d));
    if (!rc) rc = pbr_alloc(p, &d.loss, 1);
    if (!rc && (desc->flags & DRESSI_PBR_KEEP_PRED)) rc = pbr_alloc(p, &d.pred, N * npx);
    if (!rc && (desc->flags & DRESSI_PBR_KEEP_GRAD)) {
        rc = pbr_alloc(p, &d.g_tex_a, T);
        if (!rc) rc = pbr_alloc(p, &d.g_tex_m, T);
        if (!rc) rc = pbr_alloc(p, &d.g_env, E);
    }
    if (!rc) {
        uint4* lt = nullptr;
        rc = pbr_upload(p, &lt, ltab);
        d.ltab = lt;
    }
    // static maps: prefilter normalisers and the BRDF LUT, through the
    // per-op entry points on the plan's context; then the convolution weights
    // from the texel-centre direction tables (the reference's float bits, see
    // ibl_core.h)
    if (!rc) {
        float* pn = nullptr;
        rc = pbr_alloc(p, &pn, d.n_pref);
        for (uint32_t i = 0; i < d.levels && !rc; i++) {
            const float r = (float)i / (float)(d.levels - 1);
            rc = dressi_prefilter_conv_norm(ctx, d.lw[i], d.lh[i], d.psw, d.psh, r,
                                            pn + d.loff[i]);
        }
        d.pnorm = pn;
        float2* lut = nullptr;
        if (!rc) rc = pbr_alloc(p, &lut, (size_t)d.lutw * d.luth);
        if (!rc) rc = dressi_brdf_lut(ctx, d.lutw, d.luth, 512, (float*)lut);
        d.lut = lut;
    }
    if (!rc) {
        std::vector<float4> idir = host_equirect_dirs(d.iw, d.ih);
        std::vector<float4> isdir = host_equirect_dirs(d.isw, d.ish);
        std::vector<float4> psdir = host_equirect_dirs(d.psw, d.psh);
        std::vector<float4> pdir;
        for (uint32_t i = 0; i < d.levels; i++) {
            std::vector<float4> lv = host_equirect_dirs(d.lw[i], d.lh[i]);
            for (float4& q : lv) q.w = d.alpha[i];
            pdir.insert(pdir.end(), lv.begin(), lv.end());
        }
        float4 *a = nullptr, *b = nullptr, *c = nullptr, *e = nullptr;
        rc = pbr_upload(p, &a, idir);
        if (!rc) rc = pbr_upload(p, &b, isdir);
        if (!rc) rc = pbr_upload(p, &c, pdir);
        if (!rc) rc = pbr_upload(p, &e, psdir);
        d.psdir = e;
        const uint32_t ni = d.iw * d.ih, nis = d.isw * d.ish, nps = d.psw * d.psh;
        // tile-major, the column count rounded up to whole groups of kMvCols
        const auto cols = [](uint32_t n) { return (size_t)div_up(n, kMvCols) * kMvCols; };
        const size_t bfi = (size_t)nis * cols(ni), bbi = (size_t)ni * cols(nis);
        const size_t bfp = (size_t)nps * cols(d.n_pref), bbp = (size_t)d.n_pref * cols(nps);
        float *wfi = nullptr, *wbi = nullptr, *wfp = nullptr, *wbp = nullptr;
        if (!rc) rc = pbr_alloc(p, &wfi, bfi);
        if (!rc) rc = pbr_alloc(p, &wbi, bbi);
        if (!rc) rc = pbr_alloc(p, &wfp, bfp);
        if (!rc) rc = pbr_alloc(p, &wbp, bbp);
        if (!rc) {
            hipError_t err = hipSuccess;
            for (const auto& [q, n] : {std::pair<float*, size_t>{wfi, bfi}, {wbi, bbi}, {wfp, bfp},
                                      {wbp, bbp}}) {
                if (err == hipSuccess) err = hipMemsetAsync(q, 0, n * sizeof(float), ctx->stream);
            }
            if (err == hipSuccess) {
                hipLaunchKernelGGL(k_pbr_weights, dim3(div_up(ni, 256), nis), dim3(256), 0,
                                   ctx->stream, a, ni, b, nis, (const float*)nullptr, wfi, wbi);
                hipLaunchKernelGGL(k_pbr_weights, dim3(div_up(d.n_pref, 256), nps), dim3(256), 0,
                                   ctx->stream, c, d.n_pref, e, nps, d.pnorm, wfp, wbp);
                err = hipGetLastError();
            }
            if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
            if (err != hipSuccess) {
                set_error("static IBL maps failed: %s", hipGetErrorString(err));
                rc = DRESSI_ERR_HIP;
            }
        }
        d.wf_irr = wfi;
        d.wb_irr = wbi;
        d.wf_pref = wfp;
        d.wb_pref = wbp;
        d.n_ig = div_up(ni, kMvCols);
        d.n_pg = div_up(d.n_pref, kMvCols);
        d.n_isg = div_up(nis, kMvCols);
        d.n_psg = div_up(nps, kMvCols);
    }
    if (!rc) {
        float2* bc = nullptr;
        std::vector<float2> tab(kBiasTableLen);
        for (uint32_t i = 0; i < kBiasTableLen; i++) {
            const float tn = (float)(i + 1);
            tab[i] = make_float2(1.f - powf(desc->beta1, tn), 1.f - powf(desc->beta2, tn));
        }
        rc = pbr_upload(p, &bc, tab);
        d.bc_tab = bc;
        d.bc_len = kBiasTableLen;
    }
    if (rc) {
        for (void* q : p->allocs) hipFree(q);
        delete p;
        return rc;
    }
    *out = p;
    return DRESSI_OK;
}

int dressi_pbr_destroy(dressi_pbr_plan* p) {
    if (!p) return DRESSI_OK;
    hipSetDevice(p->ctx->device);
    hipStreamSynchronize(p->ctx->stream);
    pbr_drop_graph(p);
    for (void* q : p->allocs) hipFree(q);
    for (void* q : p->scene_allocs) hipFree(q);
    delete p;
    return DRESSI_OK;
}

namespace {

// set_scene with the clip positions from MVP * pos (mvps) or given (clips)
int pbr_set_scene(dressi_pbr_plan* p, const float* pos, const float* normal, const float* uv,
                  const float* faces, const float* mvps, const float* clips,
                  const float* frames, const float* light) {
    DRESSI_REQUIRE(p && pos && normal && uv && faces && (mvps || clips) && frames && light,
                   "bad arguments");
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    PbrDev& d = p->d;
    dressi_ctx* ctx = p->ctx;
    hipStream_t s = ctx->stream;
    const uint32_t V = p->desc.n_verts, Fn = p->desc.n_faces, N = d.n_views, S = d.S;
    const size_t npx = (size_t)S * S, T = (size_t)d.tw * d.th;
    d.light_col[0] = light[3];
    d.light_col[1] = light[4];
    d.light_col[2] = light[5];
    std::vector<float> uvh((size_t)V * 4), uvc((size_t)V * 4);
    for (uint32_t i = 0; i < V; i++) {
        uvh[i * 4 + 0] = uv[i * 2 + 0];
        uvh[i * 4 + 1] = uv[i * 2 + 1];
        uvh[i * 4 + 2] = 1.f;
        uvh[i * 4 + 3] = 1.f;
    }
    dressi_uv_as_clip(uv, V, uvc.data());
    // temporaries
    std::vector<void*> tmp;
    int rc = DRESSI_OK;
    auto talloc = [&](void** q, size_t b) -> int {
        DRESSI_TRY_HIP(hipMalloc(q, b ? b : 4));
        tmp.push_back(*q);
        return DRESSI_OK;
    };
    void *d_pos = nullptr, *d_nrm = nullptr, *d_uvh = nullptr, *d_uvc = nullptr,
         *d_faces = nullptr, *d_mvp = nullptr, *d_clip = nullptr, *d_attr = nullptr,
         *g_uvh = nullptr, *g_n = nullptr, *g_p = nullptr, *inv = nullptr, *guv = nullptr,
         *mask = nullptr, *cnt = nullptr;
    if (!rc) rc = talloc(&d_pos, sizeof(float) * 3 * V);
    if (!rc) rc = talloc(&d_nrm, sizeof(float) * 3 * V);
    if (!rc) rc = talloc(&d_uvh, sizeof(float) * 4 * V);
    if (!rc) rc = talloc(&d_uvc, sizeof(float) * 4 * V);
    if (!rc) rc = talloc(&d_faces, sizeof(float) * 3 * Fn);
    if (!rc) rc = talloc(&d_mvp, sizeof(float) * 16 * N);
    if (!rc) rc = talloc(&d_clip, sizeof(float4) * V);
    if (!rc) rc = talloc(&d_attr, sizeof(float4) * V);
    if (!rc) rc = talloc(&g_uvh, sizeof(float4) * npx);
    if (!rc) rc = talloc(&g_n, sizeof(float) * 3 * npx);
    if (!rc) rc = talloc(&g_p, sizeof(float) * 3 * npx);
    if (!rc) rc = talloc(&inv, sizeof(float4) * T * N);
    if (!rc) rc = talloc(&guv, sizeof(float2) * npx * N);
    if (!rc) rc = talloc(&mask, sizeof(float) * npx * N);
    if (!rc) rc = talloc(&cnt, sizeof(uint32_t) * (T + 1));
    const auto h2d = [&](void* dst, const void* src, size_t b) -> int {
        DRESSI_TRY_HIP(hipMemcpy(dst, src, b, hipMemcpyHostToDevice));
        return DRESSI_OK;
    };
    if (!rc) rc = h2d(d_pos, pos, sizeof(float) * 3 * V);
    if (!rc) rc = h2d(d_nrm, normal, sizeof(float) * 3 * V);
    if (!rc) rc = h2d(d_uvh, uvh.data(), sizeof(float) * 4 * V);
    if (!rc) rc = h2d(d_uvc, uvc.data(), sizeof(float) * 4 * V);
    if (!rc) rc = h2d(d_faces, faces, sizeof(float) * 3 * Fn);
    if (!rc && mvps) rc = h2d(d_mvp, mvps, sizeof(float) * 16 * N);
    for (uint32_t v = 0; v < N && !rc; v++) {
        if (clips) {
            rc = h2d(d_clip, clips + (size_t)v * V * 4, sizeof(float4) * V);
            if (rc) break;
        } else {
            hipLaunchKernelGGL(k_pbr_clip, dim3(div_up(V, 256)), dim3(256), 0, s,
                               (const float*)d_pos, V, (const float*)d_mvp + 16 * v,
                               (float4*)d_clip);
        }
        // the G-buffer (BuildPbrGBuffer's Rasterize calls)
        rc = dressi_rasterize(ctx, (const float*)d_clip, V, (const float*)d_uvh, 4,
                              (const float*)d_faces, Fn, S, S, (float*)g_uvh);
        if (!rc) rc = dressi_rasterize(ctx, (const float*)d_clip, V, (const float*)d_nrm, 3,
                                       (const float*)d_faces, Fn, S, S, (float*)g_n);
        if (!rc) rc = dressi_rasterize(ctx, (const float*)d_clip, V, (const float*)d_pos, 3,
                                       (const float*)d_faces, Fn, S, S, (float*)g_p);
        // the view's inverse-UV table: Rasterize(UvAsClip(uv), ScreenAttr(clip), T)
        if (!rc) rc = dressi_screen_attr(ctx, (const float*)d_clip, V, S, S, (float*)d_attr);
        if (!rc) rc = dressi_rasterize(ctx, (const float*)d_uvc, V, (const float*)d_attr, 4,
                                       (const float*)d_faces, Fn, d.tw, d.th,
                                       (float*)inv + (size_t)v * T * 4);
        if (rc) break;
        StaticArgs a{};
        a.g_uvh = (const float4*)g_uvh;
        a.g_n = (const float*)g_n;
        a.g_p = (const float*)g_p;
        for (int j = 0; j < 12; j++) a.frame[j] = frames[v * 12 + j];
        a.light_pos[0] = light[0];
        a.light_pos[1] = light[1];
        a.light_pos[2] = light[2];
        a.S = S;
        a.st0 = (float4*)d.st0 + v * npx;
        a.st1 = (float4*)d.st1 + v * npx;
        a.st2 = (float4*)d.st2 + v * npx;
        hipLaunchKernelGGL(k_pbr_static, dim3(div_up((uint32_t)npx, 256)), dim3(256), 0, s, a);
        // raster uv and mask of the view for the gather list
        hipError_t e = hipMemcpy2DAsync((float*)guv + (size_t)v * npx * 2, 2 * sizeof(float),
                                        g_uvh, sizeof(float4), 2 * sizeof(float), npx,
                                        hipMemcpyDeviceToDevice, s);
        if (e == hipSuccess) {
            e = hipMemcpy2DAsync((float*)mask + (size_t)v * npx, sizeof(float),
                                 (const float*)g_uvh + 2, sizeof(float4), sizeof(float), npx,
                                 hipMemcpyDeviceToDevice, s);
        }
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) {
            set_error("scene set-up failed: %s", hipGetErrorString(e));
            rc = DRESSI_ERR_HIP;
        }
    }
    // the gather list
    if (!rc) {
        CsrArgs ca{};
        ca.inv = (const float4*)inv;
        ca.g_uv = (const float2*)guv;
        ca.mask = (const float*)mask;
        ca.n_views = N;
        ca.S = S;
        ca.tw = d.tw;
        ca.th = d.th;
        ca.count = (uint32_t*)cnt;
        hipLaunchKernelGGL(k_pbr_csr<0>, dim3(div_up((uint32_t)T, 256)), dim3(256), 0, s, ca);
        std::vector<uint32_t> c(T + 1, 0);
        hipError_t e = hipStreamSynchronize(s);
        if (e == hipSuccess) e = hipMemcpy(c.data(), cnt, sizeof(uint32_t) * T, hipMemcpyDeviceToHost);
        if (e != hipSuccess) {
            set_error("gather list count failed: %s", hipGetErrorString(e));
            rc = DRESSI_ERR_HIP;
        }
        std::vector<uint32_t> off(T + 1, 0);
        uint64_t acc = 0;
        for (size_t i = 0; i < T && !rc; i++) {
            off[i] = (uint32_t)acc;
            acc += c[i];
        }
        off[T] = (uint32_t)acc;
        if (!rc && acc >= (1ull << 32)) {
            set_error("gather list too long");
            rc = DRESSI_ERR_UNSUPPORTED;
        }
        uint32_t* d_off = nullptr;
        uint2* d_csr = nullptr;
        if (!rc) rc = pbr_upload(p, &d_off, off);
        if (!rc) rc = pbr_alloc(p, &d_csr, (size_t)acc);
        if (!rc) {
            ca.off = d_off;
            ca.csr = d_csr;
            hipLaunchKernelGGL(k_pbr_csr<1>, dim3(div_up((uint32_t)T, 256)), dim3(256), 0, s,
                               ca);
            hipError_t e2 = hipStreamSynchronize(s);
            if (e2 != hipSuccess) {
                set_error("gather list fill failed: %s", hipGetErrorString(e2));
                rc = DRESSI_ERR_HIP;
            }
        }
        d.csr_off = d_off;
        d.csr = d_csr;
        p->csr_len = (uint32_t)acc;
    }
    for (void* q : tmp) hipFree(q);
    tmp.clear();
    // the map-gradient gather lists (static: the directions are)
    if (!rc) rc = build_map_lists(p);
    if (rc) return rc;
    pbr_drop_graph(p);
    p->scene_set = true;
    return DRESSI_OK;
}

}  // namespace

int dressi_pbr_set_scene(dressi_pbr_plan* p, const float* pos, const float* normal,
                         const float* uv, const float* faces, const float* mvps,
                         const float* frames, const float* light) {
    DRESSI_REQUIRE(mvps, "bad arguments");
    return pbr_set_scene(p, pos, normal, uv, faces, mvps, nullptr, frames, light);
}

int dressi_pbr_set_scene_clips(dressi_pbr_plan* p, const float* pos, const float* normal,
                               const float* uv, const float* faces, const float* clips,
                               const float* frames, const float* light) {
    DRESSI_REQUIRE(clips, "bad arguments");
    return pbr_set_scene(p, pos, normal, uv, faces, nullptr, clips, frames, light);
}

int dressi_pbr_set_target(dressi_pbr_plan* p, const float* gt_albedo, const float* gt_mr,
                          const float* gt_env) {
    DRESSI_REQUIRE(p && gt_albedo && gt_mr && gt_env, "bad arguments");
    DRESSI_REQUIRE(p->scene_set, "dressi_pbr_set_scene() must be called first");
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    const size_t T = (size_t)p->d.tw * p->d.th;
    // the target pass shades with the ground-truth materials: stage them in
    // the state buffers (set_state must follow)
    if (int rc = upload3(p->d.albedo, gt_albedo, T)) return rc;
    if (int rc = upload3(p->d.mr, gt_mr, T)) return rc;
    if (int rc = render_target(p, gt_env)) return rc;
    p->target_set = true;
    p->state_set = false;
    return DRESSI_OK;
}

int dressi_pbr_set_state(dressi_pbr_plan* p, const float* albedo, const float* mr,
                         const float* env, float t) {
    DRESSI_REQUIRE(p && albedo && mr && env, "bad arguments");
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    DRESSI_TRY_HIP(hipStreamSynchronize(p->ctx->stream));
    PbrDev& d = p->d;
    const size_t T = (size_t)d.tw * d.th, E = (size_t)d.ew * d.eh;
    if (int rc = upload3(d.albedo, albedo, T)) return rc;
    if (int rc = upload3(d.mr, mr, T)) return rc;
    if (int rc = upload3(d.env, env, E)) return rc;
    for (float4* q : {d.am, d.av, d.mm, d.mv}) {
        DRESSI_TRY_HIP(hipMemset(q, 0, sizeof(float4) * T));
    }
    for (float4* q : {d.em, d.ev}) {
        DRESSI_TRY_HIP(hipMemset(q, 0, sizeof(float4) * E));
    }
    DRESSI_TRY_HIP(hipMemcpy(d.t, &t, sizeof(float), hipMemcpyHostToDevice));
    p->state_set = true;
    return DRESSI_OK;
}

int dressi_pbr_get_state(dressi_pbr_plan* p, float* albedo, float* mr, float* env, float* t) {
    DRESSI_REQUIRE(p, "bad arguments");
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    DRESSI_TRY_HIP(hipStreamSynchronize(p->ctx->stream));
    PbrDev& d = p->d;
    const size_t T = (size_t)d.tw * d.th, E = (size_t)d.ew * d.eh;
    if (albedo) {
        if (int rc = download3(albedo, d.albedo, T)) return rc;
    }
    if (mr) {
        if (int rc = download3(mr, d.mr, T)) return rc;
    }
    if (env) {
        if (int rc = download3(env, d.env, E)) return rc;
    }
    if (t) DRESSI_TRY_HIP(hipMemcpy(t, d.t, sizeof(float), hipMemcpyDeviceToHost));
    return DRESSI_OK;
}

int dressi_pbr_set_adam(dressi_pbr_plan* p, const float* m_albedo, const float* v_albedo,
                        const float* m_mr, const float* v_mr, const float* m_env,
                        const float* v_env) {
    DRESSI_REQUIRE(p && m_albedo && v_albedo && m_mr && v_mr && m_env && v_env, "bad arguments");
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    DRESSI_TRY_HIP(hipStreamSynchronize(p->ctx->stream));
    PbrDev& d = p->d;
    const size_t T = (size_t)d.tw * d.th, E = (size_t)d.ew * d.eh;
    if (int rc = upload3(d.am, m_albedo, T)) return rc;
    if (int rc = upload3(d.av, v_albedo, T)) return rc;
    if (int rc = upload3(d.mm, m_mr, T)) return rc;
    if (int rc = upload3(d.mv, v_mr, T)) return rc;
    if (int rc = upload3(d.em, m_env, E)) return rc;
    return upload3(d.ev, v_env, E);
}

int dressi_pbr_get_adam(dressi_pbr_plan* p, float* m_albedo, float* v_albedo, float* m_mr,
                        float* v_mr, float* m_env, float* v_env) {
    DRESSI_REQUIRE(p && m_albedo && v_albedo && m_mr && v_mr && m_env && v_env, "bad arguments");
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    DRESSI_TRY_HIP(hipStreamSynchronize(p->ctx->stream));
    PbrDev& d = p->d;
    const size_t T = (size_t)d.tw * d.th, E = (size_t)d.ew * d.eh;
    if (int rc = download3(m_albedo, d.am, T)) return rc;
    if (int rc = download3(v_albedo, d.av, T)) return rc;
    if (int rc = download3(m_mr, d.mm, T)) return rc;
    if (int rc = download3(v_mr, d.mv, T)) return rc;
    if (int rc = download3(m_env, d.em, E)) return rc;
    return download3(v_env, d.ev, E);
}

int dressi_pbr_step_eager(dressi_pbr_plan* p, uint32_t n_iters) {
    if (int rc = pbr_ready(p)) return rc;
    for (uint32_t i = 0; i < n_iters; i++) {
        if (int rc = pbr_enqueue(p, p->ctx->stream)) return rc;
    }
    return DRESSI_OK;
}

int dressi_pbr_step(dressi_pbr_plan* p, uint32_t n_iters) {
    if (int rc = pbr_ready(p)) return rc;
    hipStream_t s = p->ctx->stream;
    if (!p->exec || p->graph_stream != s) {
        pbr_drop_graph(p);
        hipStream_t cap_stream = nullptr, side = nullptr;
        hipEvent_t fork = nullptr, join = nullptr;
        int rc = DRESSI_OK;
        if (hipStreamCreateWithFlags(&cap_stream, hipStreamNonBlocking) != hipSuccess ||
            hipStreamCreateWithFlags(&side, hipStreamNonBlocking) != hipSuccess ||
            hipEventCreateWithFlags(&fork, hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&join, hipEventDisableTiming) != hipSuccess) {
            set_error("stream / event creation failed");
            rc = DRESSI_ERR_HIP;
        }
        const hipError_t e =
            rc ? hipSuccess : hipStreamBeginCapture(cap_stream, hipStreamCaptureModeThreadLocal);
        if (!rc && e == hipSuccess) {
            rc = pbr_enqueue_forked(p, cap_stream, side, fork, join);
            hipError_t e2 = hipStreamEndCapture(cap_stream, &p->graph);
            if (!rc && e2 != hipSuccess) {
                set_error("graph capture failed: %s", hipGetErrorString(e2));
                rc = DRESSI_ERR_HIP;
            }
        } else if (!rc) {
            set_error("hipStreamBeginCapture failed: %s", hipGetErrorString(e));
            rc = DRESSI_ERR_HIP;
        }
        if (fork) hipEventDestroy(fork);
        if (join) hipEventDestroy(join);
        if (side) hipStreamDestroy(side);
        if (cap_stream) hipStreamDestroy(cap_stream);
        if (rc) {
            pbr_drop_graph(p);
            return rc;
        }
        DRESSI_TRY_HIP(hipGraphInstantiate(&p->exec, p->graph, nullptr, nullptr, 0));
        p->graph_stream = s;
    }
    for (uint32_t i = 0; i < n_iters; i++) {
        DRESSI_TRY_HIP(hipGraphLaunch(p->exec, s));
    }
    return DRESSI_OK;
}

int dressi_pbr_buffer(dressi_pbr_plan* p, int which, void** ptr, size_t* bytes) {
    DRESSI_REQUIRE(p && ptr, "bad arguments");
    const PbrDev& d = p->d;
    const size_t npx = (size_t)d.S * d.S, N = d.n_views, T = (size_t)d.tw * d.th;
    const size_t E = (size_t)d.ew * d.eh;
    void* q = nullptr;
    size_t b = 0;
    switch (which) {
        case DRESSI_PBR_LOSS: q = d.loss; b = 4; break;
        case DRESSI_PBR_PRED: q = d.pred; b = N * npx * 16; break;
        case DRESSI_PBR_TARGET: q = d.target; b = N * npx * 16; break;
        case DRESSI_PBR_G_ALBEDO: q = d.g_tex_a; b = T * 16; break;
        case DRESSI_PBR_G_MR: q = d.g_tex_m; b = T * 16; break;
        case DRESSI_PBR_G_ENV: q = d.g_env; b = E * 16; break;
        case DRESSI_PBR_IRR: q = d.irr; b = (size_t)d.iw * d.ih * 16; break;
        case DRESSI_PBR_PREF: q = d.pref; b = (size_t)d.n_pref * 16; break;
        case DRESSI_PBR_GBUF0: q = const_cast<float4*>(d.st0); b = N * npx * 16; break;
        default: DRESSI_REQUIRE(false, "unknown buffer %d", which);
    }
    DRESSI_REQUIRE(q, "buffer %d not kept (see the DRESSI_PBR_KEEP_* flags)", which);
    *ptr = q;
    if (bytes) *bytes = b;
    return DRESSI_OK;
}

int dressi_pbr_read(dressi_pbr_plan* p, int which, void* host, size_t bytes) {
    void* q = nullptr;
    size_t b = 0;
    if (int rc = dressi_pbr_buffer(p, which, &q, &b)) return rc;
    DRESSI_REQUIRE(host && bytes == b, "buffer %d holds %zu bytes, %zu given", which, b, bytes);
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    DRESSI_TRY_HIP(hipStreamSynchronize(p->ctx->stream));
    DRESSI_TRY_HIP(hipMemcpy(host, q, b, hipMemcpyDeviceToHost));
    return DRESSI_OK;
}

int dressi_pbr_profile(dressi_pbr_plan* p, uint32_t iters, char* names, size_t name_stride,
                       float* usec, uint32_t cap, uint32_t* n) {
    if (int rc = pbr_ready(p)) return rc;
    DRESSI_REQUIRE(n, "bad arguments");
    const uint32_t reps = iters ? (iters < 256u ? iters : 256u) : 1u;
    *n = kPbrKernels;
    hipStream_t s = p->ctx->stream;
    constexpr int kEv = kPbrKernels + 1;
    std::vector<hipEvent_t> ev((size_t)reps * kEv, nullptr);
    int rc = DRESSI_OK;
    for (hipEvent_t& e : ev) {
        if (hipEventCreate(&e) != hipSuccess) {
            set_error("hipEventCreate failed");
            rc = DRESSI_ERR_HIP;
            break;
        }
    }
    for (uint32_t r = 0; r < reps && !rc; r++) {
        for (int k = 0; k < kPbrKernels && !rc; k++) {
            if (hipEventRecord(ev[(size_t)r * kEv + k], s) != hipSuccess) {
                set_error("hipEventRecord failed");
                rc = DRESSI_ERR_HIP;
                break;
            }
            rc = launch_pbr_kernel(p->d, s, k);
        }
        if (!rc && hipEventRecord(ev[(size_t)r * kEv + kPbrKernels], s) != hipSuccess) {
            set_error("hipEventRecord failed");
            rc = DRESSI_ERR_HIP;
        }
    }
    if (!rc && hipEventSynchronize(ev.back()) != hipSuccess) {
        set_error("event synchronisation failed");
        rc = DRESSI_ERR_HIP;
    }
    float ms[kPbrKernels] = {};
    for (uint32_t r = 0; r < reps && !rc; r++) {
        for (int k = 0; k < kPbrKernels; k++) {
            float t = 0.f;
            if (hipEventElapsedTime(&t, ev[(size_t)r * kEv + k], ev[(size_t)r * kEv + k + 1]) !=
                hipSuccess) {
                set_error("hipEventElapsedTime failed");
                rc = DRESSI_ERR_HIP;
                break;
            }
            ms[k] += t / reps;
        }
    }
    for (uint32_t k = 0; k < (uint32_t)kPbrKernels && k < cap && !rc; k++) {
        if (usec) usec[k] = ms[k] * 1000.f;
        if (names && name_stride > 0) {
            snprintf(names + k * name_stride, name_stride, "%s", kPbrKernelNames[k]);
        }
    }
    for (hipEvent_t e : ev) {
        if (e) hipEventDestroy(e);
    }
    if (!rc) {
        DRESSI_TRY_HIP(hipStreamSynchronize(s));
    }
    return rc;
}

}  // extern "C"
