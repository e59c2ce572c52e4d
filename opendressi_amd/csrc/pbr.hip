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
// normal, the reflection and the background ray, and the texture gather's
// inverse-UV windows -- is computed once per view at set-up; an iteration
// reads those per-pixel terms, the material taps and the maps.
//
// One iteration, 7 kernels + the pooling chain (ceil(log2) levels):
//   k_pbr_pool      env -> pooled sources of the irradiance / prefilter maps
//                   (the first level also clears the gradient accumulators)
//   k_pbr_conv_fwd  IrradianceConv + every PrefilterConv level
//   k_pbr_shade     per pixel: forward, L1 loss, backward; material
//                   gradients per pixel, map gradients scattered into
//                   64-bit fixed-point accumulators (workgroup windows in LDS)
//   k_pbr_resolve   fixed point -> float map gradients
//   k_pbr_conv_bwd  the convolutions' transposes onto the pooled sources
//   k_pbr_env_adam  pooling VJPs + background gradient, Adam on the env
//   k_pbr_tex_adam  GatherByInverseUVBilinear as a static gather list per
//                   texel, Adam on albedo and mr
//   k_pbr_loss      the loss scalar, t + 1
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <vector>

#include "dressi_hip.h"
#include "ibl_core.h"
#include "internal.h"
#include "plan.h"

namespace dressi {
namespace {

constexpr uint32_t kPbrMaxLevels = 8;
constexpr uint32_t kPbrMaxViews = 16;
constexpr uint32_t kPbrMaxPool = 12;
constexpr int kConvOuts = 16;     // outputs per convolution workgroup
constexpr int kShadeTile = 16;    // 16 x 16 pixel tile per shading workgroup
constexpr int kWin = 64;          // texels per LDS scatter window
constexpr uint32_t kIrrLevel = 0xffffffffu;
constexpr uint32_t kStripes = 32;  // copies of the irradiance / prefilter accumulators

struct PbrGroup {
    uint32_t first, count, level;  // level kIrrLevel: the irradiance map
};

struct PbrDev {
    uint32_t n_views, S, tw, th, ew, eh, levels;
    uint32_t iw, ih, isw, ish, psw, psh;
    uint32_t lw[kPbrMaxLevels], lh[kPbrMaxLevels], loff[kPbrMaxLevels], n_pref;
    const uint4* ltab;  // per level (w, h, texel offset, 0)
    float alpha[kPbrMaxLevels];
    float lr, b1, b2, eps, inv_n, irr_scale;
    int fix_k;  // fixed point: value * 2^fix_k
    uint32_t* err;  // the context's error word (kErrFixedRange)
    float light_col[3];
    // static per (view, pixel)
    const float4* st0;  // fg: (u, v, n.v, n.l); bg: (bg u, bg v, -1, 0)
    const float4* st1;  // (n.h, (1 - v.h)^5, (1 - n.v)^5, dist^2)
    const float4* st2;  // (irr u, irr v, refl u, refl v); u < 0: zero direction
    float4* target;     // mapped target (rgb)
    // map geometry
    const float4* idir;   // irradiance map texel directions (.w unused)
    const float4* isdir;  // its source (pooled env) directions + sin(theta)
    const float4* pdir;   // prefilter texel directions, all levels (.w: alpha)
    const float4* psdir;  // their source directions + sin(theta)
    const float* pnorm;   // PrefilterConvNorm of every prefilter texel
    const float2* lut;
    uint32_t lutw, luth;
    const PbrGroup* fgroups;
    uint32_t n_fgroups;
    const PbrGroup* bgroups;
    uint32_t n_bgroups;
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
    unsigned long long *acc_irr, *acc_pref, *acc_env;
    float4 *g_irr, *g_pref, *g_isrc, *g_psrc;
    float4* gyA;   // per pixel (g albedo rgb, g roughness)
    float* gyM;    // per pixel g metallic
    float* loss_part;
    float* loss;
    float4* pred;  // KEEP_PRED
    float4 *g_tex_a, *g_tex_m, *g_env;  // KEEP_GRAD
    const uint32_t* csr_off;  // per texel, into csr
    const uint2* csr;         // (global pixel, weight bits)
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

// Largest fixed-point term a scatter may add: every map-gradient term is
// bounded by inv_n before the 16-lane row pre-sum (see dressi_pbr_create), so
// a term is below 16 x 2^29 = 2^33 units; 2^34 leaves a factor of 2, and
// 2^28 such terms (2^26 pixels x 4 taps) still sum below 2^63.
constexpr double kFixLimit = 17179869184.0;  // 2^34
// Error bit: a fixed-point term exceeded kFixLimit (or was not finite) and
// was clamped; reported by dressi_ctx_synchronize.
constexpr uint32_t kErrFixedRange = 0x100u;

__device__ __forceinline__ long long to_fixed(float v, int k, uint32_t* err) {
    double s = ldexp((double)v, k);
    if (!(fabs(s) <= kFixLimit)) {
        atomicOr(err, kErrFixedRange);
        s = s != s ? 0.0 : copysign(kFixLimit, s);
    }
    return __double2ll_rn(s);
}

__device__ __forceinline__ float from_fixed(unsigned long long a, int k) {
    return (float)ldexp((double)(long long)a, -k);
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

__device__ __forceinline__ float pow5(float x) { return (float)pow((double)x, 5.0); }

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

// ---------------------------------------------------------------------------
// Iteration kernels
// ---------------------------------------------------------------------------

// One level of the pooling chain (Reduce2x2Sum * 0.25, zero padding): level
// `lvl` from level lvl - 1. The first level also clears the gradient
// accumulators of this iteration.
__global__ __launch_bounds__(256) void k_pbr_pool(PbrDev d, uint32_t lvl) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (lvl == 1 && !d.target_mode) {
        const uint32_t stride = gridDim.x * blockDim.x;
        for (uint32_t j = i; j < (d.iw * d.ih) * 3 * kStripes; j += stride) d.acc_irr[j] = 0ull;
        for (uint32_t j = i; j < d.n_pref * 3 * kStripes; j += stride) d.acc_pref[j] = 0ull;
        for (uint32_t j = i; j < (d.ew * d.eh) * 3; j += stride) d.acc_env[j] = 0ull;
    }
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

// Sum of 3 x kConvOuts per-thread partials over the 256-thread workgroup
// (wave shuffles, then the 4 waves in order); result in red[o * 3 + c].
__device__ __forceinline__ void block_reduce_outs(float (&acc)[kConvOuts][3], float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 0; o < kConvOuts; o++) {
#pragma unroll
        for (int c = 0; c < 3; c++) {
            float v = acc[o][c];
#pragma unroll
            for (int s = 32; s >= 1; s >>= 1) {
                v += __shfl_xor(v, s);
            }
            if (lane == 0) {
                red[wave * kConvOuts * 3 + o * 3 + c] = v;
            }
        }
    }
    __syncthreads();
    if (threadIdx.x < kConvOuts * 3) {
        const int j = threadIdx.x;
        red[4 * kConvOuts * 3 + j] = ((red[j] + red[kConvOuts * 3 + j]) +
                                      red[2 * kConvOuts * 3 + j]) + red[3 * kConvOuts * 3 + j];
    }
    __syncthreads();
}

// IrradianceConv and the PrefilterConv levels (f_ops.cpp:3006-3087,
// 3264-3348): a workgroup per group of <= 16 outputs of one map, the
// threads split the source texels; weights exactly as the reference's
// (ggx_conv_weight of the same float dot product), sums in another order.
__global__ __launch_bounds__(256) void k_pbr_conv_fwd(PbrDev d) {
    __shared__ float4 od[kConvOuts];
    __shared__ float red[5 * kConvOuts * 3];
    const PbrGroup gr = d.fgroups[blockIdx.x];
    const bool irr = gr.level == kIrrLevel;
    const float4* sdir = irr ? d.isdir : d.psdir;
    const float4* src = irr ? d.pool[d.irr_pool] : d.pool[d.pref_pool];
    const uint32_t n_src = irr ? d.isw * d.ish : d.psw * d.psh;
    const float alpha = irr ? 0.f : d.alpha[gr.level];
    if (threadIdx.x < kConvOuts) {
        od[threadIdx.x] = threadIdx.x < gr.count
                                  ? (irr ? d.idir : d.pdir)[gr.first + threadIdx.x]
                                  : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();
    float acc[kConvOuts][3];
#pragma unroll
    for (int o = 0; o < kConvOuts; o++) {
        acc[o][0] = acc[o][1] = acc[o][2] = 0.f;
    }
    for (uint32_t s = threadIdx.x; s < n_src; s += blockDim.x) {
        const float4 sd = sdir[s];
        const float4 e = src[s];
#pragma unroll
        for (int o = 0; o < kConvOuts; o++) {
            const float4 r = od[o];
            const float c = r.x * sd.x + r.y * sd.y + r.z * sd.z;
            if (c > 0.f) {
                const float w = (irr ? c : ggx_conv_weight(c, alpha)) * sd.w;
                acc[o][0] += e.x * w;
                acc[o][1] += e.y * w;
                acc[o][2] += e.z * w;
            }
        }
    }
    block_reduce_outs(acc, red);
    if (threadIdx.x < gr.count) {
        const float* v = red + 4 * kConvOuts * 3 + threadIdx.x * 3;
        const uint32_t o = gr.first + threadIdx.x;
        if (irr) {
            d.irr[o] = make_float4(v[0] * d.irr_scale, v[1] * d.irr_scale, v[2] * d.irr_scale, 0.f);
        } else {
            const float nt = d.pnorm[o];
            const float wn = nt > 1e-12f ? nt : 1e-12f;
            d.pref[o] = make_float4(v[0] / wn, v[1] / wn, v[2] / wn, 0.f);
        }
    }
}

// LDS scatter windows of one shading workgroup: per map (irradiance,
// prefilter levels, env) the bounding box of the tap bases of the
// contributing pixels (u unwrapped around the seam); a box of <= kWin taps
// is accumulated in LDS and flushed with one global atomic per texel and
// channel, else the lanes add to the global accumulators directly.
constexpr int kMaps = kPbrMaxLevels + 2;

struct MapTaps {
    int ix, iy;  // tap base: floor(u w - .5), floor(v h - .5)
    float w[4];  // weights in the reference's order (dy outer, dx inner)
};

__device__ __forceinline__ MapTaps map_taps(int w, int h, float u, float v) {
    const float sx = u * (float)w - 0.5f;
    const float sy = v * (float)h - 0.5f;
    MapTaps t;
    t.ix = (int)floorf(sx);
    t.iy = (int)floorf(sy);
    const float fx = sx - (float)t.ix;
    const float fy = sy - (float)t.iy;
    t.w[0] = (1.f - fx) * (1.f - fy);
    t.w[1] = fx * (1.f - fy);
    t.w[2] = (1.f - fx) * fy;
    t.w[3] = fx * fy;
    (void)w;
    (void)h;
    return t;
}

__device__ __forceinline__ uint32_t wrap_idx(int x, int y, int w, int h) {
    x = ((x % w) + w) % w;
    y = y < 0 ? 0 : (y > h - 1 ? h - 1 : y);
    return (uint32_t)(y * w + x);
}

// DPP moves within rows of 16 lanes: row_shr:S reads lane - S (lanes with
// (lane & 15) < S read 0), row_shl:S reads lane + S
template <int S>
__device__ __forceinline__ int dpp_row_shr(int v) {
    return __builtin_amdgcn_update_dpp(0, v, 0x110 + S, 0xf, 0xf, true);
}
template <int S>
__device__ __forceinline__ int dpp_row_shl(int v) {
    return __builtin_amdgcn_update_dpp(0, v, 0x100 + S, 0xf, 0xf, true);
}
template <int S>
__device__ __forceinline__ float dpp_row_shr_f(float v) {
    return __int_as_float(dpp_row_shr<S>(__float_as_int(v)));
}

// Per pixel (a 16 x 16 tile of one view per workgroup): the shading
// forward, the L1 loss and its backward (the derivation of the reference's
// autodiff of pbr_graph.cpp:47-137 through Div / Mul / Add / Max / Mix /
// Clamp / Pow / Abs, f_ops.cpp:235-537); in target mode the forward only.
// The prefilter levels with a tent weight 1 - |lod - i| >= 0 are among
// floor(lod) - 1 .. floor(lod) + 1: three register slots.
__global__ __launch_bounds__(256) void k_pbr_shade(PbrDev d) {
    __shared__ int box[kMaps][4];
    __shared__ unsigned long long win[kMaps][kWin][3];
    __shared__ float lred[4];
    const uint32_t tiles = (d.S + kShadeTile - 1) / kShadeTile;
    const uint32_t view = blockIdx.x / (tiles * tiles);
    const uint32_t tile = blockIdx.x % (tiles * tiles);
    const uint32_t x = (tile % tiles) * kShadeTile + (threadIdx.x % kShadeTile);
    const uint32_t y = (tile / tiles) * kShadeTile + (threadIdx.x / kShadeTile);
    const bool valid = x < d.S && y < d.S;
    const size_t npx = (size_t)d.S * d.S;
    const size_t p = (size_t)view * npx + (size_t)(valid ? y * d.S + x : 0);
    const int L = (int)d.levels;
    if (threadIdx.x < kMaps * 4) {
        box[threadIdx.x >> 2][threadIdx.x & 3] = (threadIdx.x & 1) ? INT_MIN : INT_MAX;
    }
    const bool train = !d.target_mode;
    // ---- forward --------------------------------------------------------
    const float4 s0 = valid ? d.st0[p] : make_float4(0.f, 0.f, -1.f, 0.f);
    const bool fg = valid && s0.z >= 0.f;
    float hdr[3] = {0.f, 0.f, 0.f};
    MapTaps t_irr{}, t_bg{}, tp[3];
    bool use_irr = false, use_bg = false, act[3] = {false, false, false};
    int li[3] = {0, 0, 0};
    float xs[3] = {0.f, 0.f, 0.f}, ws[3] = {0.f, 0.f, 0.f}, Ps[3][3];
    float a[3] = {0.f, 0.f, 0.f}, mr[3] = {0.f, 0.f, 0.f}, irr[3] = {0.f, 0.f, 0.f};
    float pref[3] = {0.f, 0.f, 0.f}, lut[2] = {0.f, 0.f};
    float ao = 0.f, rough = 0.f, metal = 0.f, lod = 0.f;
    float4 s1 = f4_zero(), s2 = f4_zero();
#pragma unroll
    for (int j = 0; j < 3; j++) {
        Ps[j][0] = Ps[j][1] = Ps[j][2] = 0.f;
        tp[j] = MapTaps{};
    }
    if (valid && !fg) {
        if (s0.x >= 0.f) {
            use_bg = true;
            t_bg = map_taps((int)d.ew, (int)d.eh, s0.x, s0.y);
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
            use_irr = true;
            t_irr = map_taps((int)d.iw, (int)d.ih, s2.x, s2.y);
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
                tp[j] = map_taps((int)lv.x, (int)lv.y, s2.z, s2.w);
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
    float lsum = 0.f;
    if (valid) {
        const float4 tg = d.target[p];
        const float tv[3] = {tg.x, tg.y, tg.z};
#pragma unroll
        for (int c = 0; c < 3; c++) {
            const float diff = tv[c] - mapped[c];
            lsum += fabsf(diff);
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
    }
    // ---- loss partial of the workgroup ------------------------------------
    {
        float v = lsum;
#pragma unroll
        for (int s = 32; s >= 1; s >>= 1) {
            v += __shfl_xor(v, s);
        }
        if ((threadIdx.x & 63) == 0) {
            lred[threadIdx.x >> 6] = v;
        }
    }
    // ---- map gradient scatter ---------------------------------------------
    // map m: 0 irradiance, 1 + i prefilter level i, L + 1 env; the
    // irradiance / prefilter accumulators are striped over kStripes copies
    // (by workgroup) so the few texels of the small maps are not one hot
    // spot. Five passes (irradiance, the three prefilter slots, env): per
    // pass, the 16 lanes of a pixel row are cut into runs of equal tap base
    // (map, ix, iy); each run's 12 weighted values are summed along the row
    // (DPP, a fixed order) and its last lane adds them to the workgroup's
    // LDS window of the map (or to the global accumulators when the window
    // would exceed kWin texels).
    const uint32_t stripe = blockIdx.x & (kStripes - 1);
    unsigned long long* acc_irr = d.acc_irr + (size_t)stripe * d.iw * d.ih * 3;
    unsigned long long* acc_pref = d.acc_pref + (size_t)stripe * d.n_pref * 3;
    const int lane16 = (int)(threadIdx.x & 15);
    const auto pass_has = [&](int ps) {
        return ps == 0 ? use_irr : (ps == 4 ? use_bg : (act[ps - 1] && ws[ps - 1] != 0.f));
    };
    const auto pass_map = [&](int ps) { return ps == 0 ? 0 : (ps == 4 ? L + 1 : 1 + li[ps - 1]); };
    const auto pass_taps = [&](int ps) -> const MapTaps& {
        return ps == 0 ? t_irr : (ps == 4 ? t_bg : tp[ps - 1]);
    };
    // run ids and run tails per pass
    int seg[5];
    bool tail[5];
#pragma unroll
    for (int ps = 0; ps < 5; ps++) {
        const bool has = pass_has(ps);
        const MapTaps& t = pass_taps(ps);
        // lanes without a contribution get a key of their own
        const int key = has ? ((pass_map(ps) << 26) | ((t.iy + 1) << 13) | (t.ix + 1))
                            : -1 - (int)threadIdx.x;
        const int left = dpp_row_shr<1>(key);
        int sg = (lane16 == 0 || left != key) ? 1 : 0;
        sg += dpp_row_shr<1>(sg);
        sg += dpp_row_shr<2>(sg);
        sg += dpp_row_shr<4>(sg);
        sg += dpp_row_shr<8>(sg);
        const int right = dpp_row_shl<1>(sg);
        seg[ps] = sg;
        tail[ps] = has && (lane16 == 15 || right != sg);
    }
    __syncthreads();  // box initialised
#pragma unroll
    for (int ps = 0; ps < 5; ps++) {
        if (tail[ps]) {
            const int m = pass_map(ps);
            const MapTaps& t = pass_taps(ps);
            atomicMin(&box[m][0], t.ix);
            atomicMax(&box[m][1], t.ix);
            atomicMin(&box[m][2], t.iy);
            atomicMax(&box[m][3], t.iy);
        }
    }
    const int n_maps = L + 2;
    for (int j = threadIdx.x; j < n_maps * kWin * 3; j += blockDim.x) {
        (&win[0][0][0])[j] = 0ull;
    }
    __syncthreads();
    const auto map_wh = [&](int m, int* w, int* h, uint32_t* off) {
        if (m == 0) {
            *w = (int)d.iw;
            *h = (int)d.ih;
            *off = 0;
        } else if (m <= L) {
            const uint4 lv = d.ltab[m - 1];
            *w = (int)lv.x;
            *h = (int)lv.y;
            *off = lv.z;
        } else {
            *w = (int)d.ew;
            *h = (int)d.eh;
            *off = 0;
        }
    };
    // window geometry: x in [box0, box1 + 1] (unwrapped), y clamped
    const auto win_ok = [&](int m, int h, int* ww, int* wy0) {
        if (box[m][0] > box[m][1]) return false;
        const int y0 = box[m][2] < 0 ? 0 : (box[m][2] > h - 1 ? h - 1 : box[m][2]);
        const int y1 = box[m][3] + 1 < 0 ? 0 : (box[m][3] + 1 > h - 1 ? h - 1 : box[m][3] + 1);
        const int w = box[m][1] - box[m][0] + 2;
        *ww = w;
        *wy0 = y0;
        return w * (y1 - y0 + 1) <= kWin;
    };
    const int k = d.fix_k;
#pragma unroll
    for (int ps = 0; ps < 5; ps++) {
        if (!__any(tail[ps])) {
            continue;
        }
        const MapTaps& t = pass_taps(ps);
        float g3[3];
        if (ps == 0) {
            g3[0] = g_irr[0];
            g3[1] = g_irr[1];
            g3[2] = g_irr[2];
        } else if (ps == 4) {
            g3[0] = gh[0];
            g3[1] = gh[1];
            g3[2] = gh[2];
        } else {
            const float wj = ws[ps - 1];
            g3[0] = gpref[0] * wj;
            g3[1] = gpref[1] * wj;
            g3[2] = gpref[2] * wj;
        }
        const bool has = pass_has(ps);
        float v[12];
#pragma unroll
        for (int q = 0; q < 4; q++) {
#pragma unroll
            for (int c = 0; c < 3; c++) {
                v[q * 3 + c] = has ? g3[c] * t.w[q] : 0.f;
            }
        }
        const int sg = seg[ps];
        // segmented inclusive scan along the row (runs are contiguous)
#pragma unroll
        for (int sh = 1; sh < 16; sh <<= 1) {
            const int osg = sh == 1 ? dpp_row_shr<1>(sg)
                                    : (sh == 2 ? dpp_row_shr<2>(sg)
                                               : (sh == 4 ? dpp_row_shr<4>(sg) : dpp_row_shr<8>(sg)));
            const bool take = lane16 >= sh && osg == sg;
#pragma unroll
            for (int e = 0; e < 12; e++) {
                const float o = sh == 1 ? dpp_row_shr_f<1>(v[e])
                                        : (sh == 2 ? dpp_row_shr_f<2>(v[e])
                                                   : (sh == 4 ? dpp_row_shr_f<4>(v[e])
                                                              : dpp_row_shr_f<8>(v[e])));
                v[e] += take ? o : 0.f;
            }
        }
        if (tail[ps]) {
            const int m = pass_map(ps);
            int w, h, ww, wy0;
            uint32_t off;
            map_wh(m, &w, &h, &off);
            const bool lds = win_ok(m, h, &ww, &wy0);
            unsigned long long* gacc =
                    m == 0 ? acc_irr : (m <= L ? acc_pref + (size_t)off * 3 : d.acc_env);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int xx = t.ix + (q & 1), yy0 = t.iy + (q >> 1);
                const int yy = yy0 < 0 ? 0 : (yy0 > h - 1 ? h - 1 : yy0);
#pragma unroll
                for (int c = 0; c < 3; c++) {
                    const long long val = to_fixed(v[q * 3 + c], k, d.err);
                    if (!val) continue;
                    if (lds) {
                        const int wi = (yy - wy0) * ww + (xx - box[m][0]);
                        atomicAdd(&win[m][wi][c], (unsigned long long)val);
                    } else {
                        atomicAdd(&gacc[(size_t)wrap_idx(xx, yy, w, h) * 3 + c],
                                  (unsigned long long)val);
                    }
                }
            }
        }
    }
    __syncthreads();
    // flush the LDS windows
    for (int j = threadIdx.x; j < n_maps * kWin; j += blockDim.x) {
        const int m = j / kWin, wi = j % kWin;
        int w, h, ww, wy0;
        uint32_t off;
        map_wh(m, &w, &h, &off);
        if (!win_ok(m, h, &ww, &wy0)) continue;
        const int xx = box[m][0] + wi % ww, yy = wy0 + wi / ww;
        if (yy > h - 1) continue;
        unsigned long long* gacc =
                m == 0 ? acc_irr : (m <= L ? acc_pref + (size_t)off * 3 : d.acc_env);
        for (int c = 0; c < 3; c++) {
            const unsigned long long val = win[m][wi][c];
            if (val) {
                atomicAdd(&gacc[(size_t)wrap_idx(xx, yy, w, h) * 3 + c], val);
            }
        }
    }
    if (threadIdx.x == 0) {
        d.loss_part[blockIdx.x] = ((lred[0] + lred[1]) + lred[2]) + lred[3];
    }
}

// fixed point -> float gradients of the irradiance and prefilter maps: the
// sum of the stripes (exact in fixed point, so in any order)
__global__ __launch_bounds__(256) void k_pbr_resolve(PbrDev d) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t ni = d.iw * d.ih;
    if (i >= ni + d.n_pref) {
        return;
    }
    const bool irr = i < ni;
    const unsigned long long* a = irr ? d.acc_irr + (size_t)i * 3
                                      : d.acc_pref + (size_t)(i - ni) * 3;
    const size_t stride = (size_t)(irr ? ni : d.n_pref) * 3;
    unsigned long long s0 = 0, s1 = 0, s2 = 0;
    for (uint32_t st = 0; st < kStripes; st++) {
        s0 += a[st * stride + 0];
        s1 += a[st * stride + 1];
        s2 += a[st * stride + 2];
    }
    const float4 g = make_float4(from_fixed(s0, d.fix_k), from_fixed(s1, d.fix_k),
                                 from_fixed(s2, d.fix_k), 0.f);
    if (irr) {
        d.g_irr[i] = g;
    } else {
        d.g_pref[i - ni] = g;
    }
}

// The convolutions' transposes (IrradianceConvBwd f_ops.cpp:2970-3004,
// PrefilterConvBwd :3207-3262, every level onto the one pooled source): a
// workgroup per group of <= 16 source texels, the threads split the map
// texels.
__global__ __launch_bounds__(256) void k_pbr_conv_bwd(PbrDev d) {
    __shared__ float4 sd_s[kConvOuts];
    __shared__ float red[5 * kConvOuts * 3];
    const PbrGroup gr = d.bgroups[blockIdx.x];
    const bool irr = gr.level == kIrrLevel;
    const float4* sdir = irr ? d.isdir : d.psdir;
    if (threadIdx.x < kConvOuts) {
        sd_s[threadIdx.x] = threadIdx.x < gr.count ? sdir[gr.first + threadIdx.x]
                                                   : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();
    float acc[kConvOuts][3];
#pragma unroll
    for (int o = 0; o < kConvOuts; o++) {
        acc[o][0] = acc[o][1] = acc[o][2] = 0.f;
    }
    const uint32_t n_t = irr ? d.iw * d.ih : d.n_pref;
    const float4* tdir = irr ? d.idir : d.pdir;
    const float4* tg = irr ? d.g_irr : d.g_pref;
    // the next texel's direction, gradient and norm are loaded before the
    // current one is used (the loop is bound by these loads' latency)
    float4 r_n = make_float4(0.f, 0.f, 0.f, 0.f), g_n = r_n;
    float nt_n = 1.f;
    if (threadIdx.x < n_t) {
        r_n = tdir[threadIdx.x];
        g_n = tg[threadIdx.x];
        nt_n = irr ? 1.f : d.pnorm[threadIdx.x];
    }
    for (uint32_t t = threadIdx.x; t < n_t; t += blockDim.x) {
        const float4 r = r_n;
        const float4 g = g_n;
        const float nt = nt_n;
        const uint32_t tn = t + blockDim.x;
        if (tn < n_t) {
            r_n = tdir[tn];
            g_n = tg[tn];
            nt_n = irr ? 1.f : d.pnorm[tn];
        }
        if (g.x == 0.f && g.y == 0.f && g.z == 0.f) {
            continue;
        }
        float inv = 1.f;
        if (!irr) {
            inv = nt > 1e-12f ? nt : 1e-12f;
        }
#pragma unroll
        for (int o = 0; o < kConvOuts; o++) {
            const float4 s = sd_s[o];
            const float c = r.x * s.x + r.y * s.y + r.z * s.z;
            if (c > 0.f) {
                const float w = irr ? c * s.w : ggx_conv_weight(c, r.w) / inv;
                acc[o][0] += g.x * w;
                acc[o][1] += g.y * w;
                acc[o][2] += g.z * w;
            }
        }
    }
    block_reduce_outs(acc, red);
    if (threadIdx.x < gr.count) {
        const float* v = red + 4 * kConvOuts * 3 + threadIdx.x * 3;
        const uint32_t o = gr.first + threadIdx.x;
        if (irr) {
            d.g_isrc[o] = make_float4(v[0] * d.irr_scale, v[1] * d.irr_scale,
                                      v[2] * d.irr_scale, 0.f);
        } else {
            const float st = sd_s[threadIdx.x].w;
            d.g_psrc[o] = make_float4(v[0] * st, v[1] * st, v[2] * st, 0.f);
        }
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

// Per env texel: the background gradient, the pooling chains' VJPs
// (UpsampleNearest2x of gy * 0.25 per level, f_ops.cpp:958-994) of the
// irradiance and prefilter sources, their sum, Adam (env >= 0).
__global__ __launch_bounds__(256) void k_pbr_env_adam(PbrDev d) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= d.ew * d.eh) {
        return;
    }
    const uint32_t x = i % d.ew, y = i / d.ew;
    const unsigned long long* a = d.acc_env + (size_t)i * 3;
    float g[3] = {from_fixed(a[0], d.fix_k), from_fixed(a[1], d.fix_k), from_fixed(a[2], d.fix_k)};
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

// Per texel: the static gather list (GatherByInverseUVBilinear over every
// view) of the per-pixel material gradients, Adam on albedo and mr.
__global__ __launch_bounds__(256) void k_pbr_tex_adam(PbrDev d) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= d.tw * d.th) {
        return;
    }
    float ga[3] = {0.f, 0.f, 0.f}, gr = 0.f, gm = 0.f;
    const uint32_t e0 = d.csr_off[i], e1 = d.csr_off[i + 1];
    for (uint32_t e = e0; e < e1; e++) {
        const uint2 en = d.csr[e];
        const float w = __uint_as_float(en.y);
        const float4 g = d.gyA[en.x];
        ga[0] += g.x * w;
        ga[1] += g.y * w;
        ga[2] += g.z * w;
        gr += g.w * w;
        gm += d.gyM[en.x] * w;
    }
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

// The loss scalar (the workgroups' partial |diff| sums * 1 / (W H 3)) and
// the step counter.
__global__ __launch_bounds__(256) void k_pbr_loss(PbrDev d, uint32_t n_part) {
    __shared__ float red[4];
    // 8 independent loads in flight per thread (a single workgroup would
    // otherwise wait one memory latency per partial)
    float acc8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (uint32_t j0 = threadIdx.x; j0 < n_part; j0 += 8 * blockDim.x) {
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const uint32_t j = j0 + (uint32_t)u * blockDim.x;
            acc8[u] += j < n_part ? d.loss_part[j] : 0.f;
        }
    }
    float v = ((acc8[0] + acc8[1]) + (acc8[2] + acc8[3])) + ((acc8[4] + acc8[5]) + (acc8[6] + acc8[7]));
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) {
        v += __shfl_xor(v, s);
    }
    if ((threadIdx.x & 63) == 0) {
        red[threadIdx.x >> 6] = v;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        d.loss[0] = (((red[0] + red[1]) + red[2]) + red[3]) * d.inv_n;
        *d.t = *d.t + 1.f;
    }
}

// Kernel list of one iteration (the pooling chain counts as one entry)
constexpr int kPbrKernels = 8;
const char* const kPbrKernelNames[kPbrKernels] = {
        "k_pbr_pool", "k_pbr_conv_fwd", "k_pbr_shade", "k_pbr_resolve",
        "k_pbr_conv_bwd", "k_pbr_env_adam", "k_pbr_tex_adam", "k_pbr_loss"};

uint32_t shade_blocks(const PbrDev& d) {
    const uint32_t tiles = (d.S + kShadeTile - 1) / kShadeTile;
    return tiles * tiles * d.n_views;
}

int launch_pbr_kernel(const PbrDev& d, hipStream_t s, int k) {
    switch (k) {
        case 0:
            for (uint32_t l = 1; l <= d.n_pool; l++) {
                const uint32_t n = d.pw[l] * d.ph[l];
                const uint32_t blocks = std::max(div_up(n, 256), l == 1 ? 512u : 1u);
                hipLaunchKernelGGL(k_pbr_pool, dim3(blocks), dim3(256), 0, s, d, l);
                DRESSI_CHECK_LAUNCH();
            }
            if (d.n_pool == 0) {
                // no pooling level: clear the accumulators with a level-1
                // launch that pools nothing
                PbrDev z = d;
                z.pw[1] = 0;
                z.ph[1] = 0;
                hipLaunchKernelGGL(k_pbr_pool, dim3(512), dim3(256), 0, s, z, 1u);
                DRESSI_CHECK_LAUNCH();
            }
            return DRESSI_OK;
        case 1:
            hipLaunchKernelGGL(k_pbr_conv_fwd, dim3(d.n_fgroups), dim3(256), 0, s, d);
            break;
        case 2:
            hipLaunchKernelGGL(k_pbr_shade, dim3(shade_blocks(d)), dim3(256), 0, s, d);
            break;
        case 3:
            hipLaunchKernelGGL(k_pbr_resolve, dim3(div_up(d.iw * d.ih + d.n_pref, 256)),
                               dim3(256), 0, s, d);
            break;
        case 4:
            hipLaunchKernelGGL(k_pbr_conv_bwd, dim3(d.n_bgroups), dim3(256), 0, s, d);
            break;
        case 5:
            hipLaunchKernelGGL(k_pbr_env_adam, dim3(div_up(d.ew * d.eh, 256)), dim3(256), 0, s,
                               d);
            break;
        case 6:
            hipLaunchKernelGGL(k_pbr_tex_adam, dim3(div_up(d.tw * d.th, 256)), dim3(256), 0, s,
                               d);
            break;
        default:
            hipLaunchKernelGGL(k_pbr_loss, dim3(1), dim3(256), 0, s, d, shade_blocks(d));
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
    std::vector<PbrGroup> fgroups, bgroups;
    bool scene_set = false, target_set = false, state_set = false;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    hipStream_t graph_stream = nullptr;
    uint32_t csr_len = 0;
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
// Adam runs on `side` beside the environment's chain (resolve, transposed
// convolutions, env Adam): the two read and write disjoint buffers (both
// only read t), and both join before the loss kernel advances t.
int pbr_enqueue_forked(dressi_pbr_plan* p, hipStream_t s, hipStream_t side, hipEvent_t fork,
                       hipEvent_t join) {
    for (int k = 0; k <= 2; k++) {  // pool, conv_fwd, shade
        if (int rc = launch_pbr_kernel(p->d, s, k)) return rc;
    }
    DRESSI_TRY_HIP(hipEventRecord(fork, s));
    DRESSI_TRY_HIP(hipStreamWaitEvent(side, fork, 0));
    if (int rc = launch_pbr_kernel(p->d, side, 6)) return rc;  // tex_adam
    DRESSI_TRY_HIP(hipEventRecord(join, side));
    for (int k = 3; k <= 5; k++) {  // resolve, conv_bwd, env_adam
        if (int rc = launch_pbr_kernel(p->d, s, k)) return rc;
    }
    DRESSI_TRY_HIP(hipStreamWaitEvent(s, join, 0));
    return launch_pbr_kernel(p->d, s, 7);  // loss, t + 1
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

// Output groups of <= kConvOuts texels, never spanning two maps
void make_groups(std::vector<PbrGroup>& out, uint32_t first, uint32_t count, uint32_t level) {
    for (uint32_t o = 0; o < count; o += kConvOuts) {
        out.push_back(PbrGroup{first + o, std::min<uint32_t>(kConvOuts, count - o), level});
    }
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
    // accumulators of the target pass: throw-away
    if (!rc) rc = talloc(&q, sizeof(unsigned long long) * 3 * t.iw * t.ih);
    t.acc_irr = (unsigned long long*)q;
    if (!rc) rc = talloc(&q, sizeof(unsigned long long) * 3 * t.n_pref);
    t.acc_pref = (unsigned long long*)q;
    if (!rc) rc = talloc(&q, sizeof(unsigned long long) * 3 * ne);
    t.acc_env = (unsigned long long*)q;
    t.target_mode = 1;
    hipStream_t s = p->ctx->stream;
    if (!rc) rc = launch_pbr_kernel(t, s, 0);
    if (!rc) rc = launch_pbr_kernel(t, s, 1);
    if (!rc) rc = launch_pbr_kernel(t, s, 2);
    hipError_t e = hipStreamSynchronize(s);
    for (void* b : tmp) hipFree(b);
    if (!rc && e != hipSuccess) {
        set_error("target render failed: %s", hipGetErrorString(e));
        rc = DRESSI_ERR_HIP;
    }
    return rc;
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
    // <= 2^26 pixels: the fixed-point map-gradient sums (kFixLimit) cannot wrap
    DRESSI_REQUIRE((uint64_t)desc->n_views * desc->width * desc->height <= (1ull << 26),
                   "too many pixels (views x width x height must be <= 2^26)");
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
    // |d loss / d hdr| <= inv_n (L1 on the Reinhard-mapped image of
    // non-negative radiance: d ldr / d hdr = 1 / (1 + hdr)^2 <= 1) and every
    // scattered term is that times a coefficient in [0, 1] (material terms
    // and split-sum factors in [0, 1], bilinear weights): with 2^28 units per
    // inv_n a term stays below 2^29 units, a 16-lane pre-sum below 2^33, and
    // to_fixed flags and clamps anything beyond 2^34 (kFixLimit)
    d.fix_k = 28 - ilogbf(d.inv_n);
    d.err = ctx->d_err;
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
    if (!rc) rc = pbr_alloc(p, &d.g_isrc, (size_t)d.isw * d.ish);
    if (!rc) rc = pbr_alloc(p, &d.g_psrc, (size_t)d.psw * d.psh);
    if (!rc) rc = pbr_alloc(p, &d.acc_irr, (size_t)d.iw * d.ih * 3 * kStripes);
    if (!rc) rc = pbr_alloc(p, &d.acc_pref, (size_t)d.n_pref * 3 * kStripes);
    if (!rc) rc = pbr_alloc(p, &d.acc_env, E * 3);
    if (!rc) rc = pbr_alloc(p, &d.gyA, N * npx);
    if (!rc) rc = pbr_alloc(p, &d.gyM, N * npx);
    if (!rc) rc = pbr_alloc(p, &d.loss_part, shade_blocks(d));
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
    // direction tables (the reference's float bits, see ibl_core.h)
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
        d.idir = a;
        d.isdir = b;
        d.pdir = c;
        d.psdir = e;
    }
    // conv groups
    if (!rc) {
        make_groups(p->fgroups, 0, d.iw * d.ih, kIrrLevel);
        for (uint32_t i = 0; i < d.levels; i++) {
            make_groups(p->fgroups, d.loff[i], d.lw[i] * d.lh[i], i);
        }
        make_groups(p->bgroups, 0, d.isw * d.ish, kIrrLevel);
        make_groups(p->bgroups, 0, d.psw * d.psh, 0);
        PbrGroup *fg = nullptr, *bg = nullptr;
        rc = pbr_upload(p, &fg, p->fgroups);
        if (!rc) rc = pbr_upload(p, &bg, p->bgroups);
        d.fgroups = fg;
        d.n_fgroups = (uint32_t)p->fgroups.size();
        d.bgroups = bg;
        d.n_bgroups = (uint32_t)p->bgroups.size();
    }
    // static maps: prefilter normalisers and the BRDF LUT, through the
    // per-op entry points on the plan's context
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
        if (!rc) {
            hipError_t e = hipStreamSynchronize(ctx->stream);
            if (e != hipSuccess) {
                set_error("static IBL maps failed: %s", hipGetErrorString(e));
                rc = DRESSI_ERR_HIP;
            }
        }
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
    delete p;
    return DRESSI_OK;
}

int dressi_pbr_set_scene(dressi_pbr_plan* p, const float* pos, const float* normal,
                         const float* uv, const float* faces, const float* mvps,
                         const float* frames, const float* light) {
    DRESSI_REQUIRE(p && pos && normal && uv && faces && mvps && frames && light, "bad arguments");
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
    if (!rc) rc = h2d(d_mvp, mvps, sizeof(float) * 16 * N);
    for (uint32_t v = 0; v < N && !rc; v++) {
        hipLaunchKernelGGL(k_pbr_clip, dim3(div_up(V, 256)), dim3(256), 0, s,
                           (const float*)d_pos, V, (const float*)d_mvp + 16 * v,
                           (float4*)d_clip);
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
    if (rc) return rc;
    pbr_drop_graph(p);
    p->scene_set = true;
    return DRESSI_OK;
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
