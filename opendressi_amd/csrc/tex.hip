// tex.hip -- the texture path (C3): TextureBilinear and its inverse-UV
// backward (GatherByInverseUVBilinear) as per-op entry points, ScreenAttr on
// the device, the UV-sphere generator, and the fused texture-fit plan
// (src/core/f_ops.cpp:2650-2780, src/core/ibl_math.h:91-115,
// src/core/mesh_utils.cpp:180-203, examples/texture_optimization/run.cpp:
// 112-145).
#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "plan.h"

namespace dressi {
namespace {

// BilerpClamp (src/core/ibl_math.h:91-115): 4-tap bilinear at uv * size -
// 0.5, both axes clamped to the edge; `data` is {w,h} x n (n <= 4).
__device__ __forceinline__ void bilerp_clamp_n(const float* data, int w, int h, uint32_t n,
                                               float u, float v, float out[4]) {
    const float sx = u * (float)w - 0.5f;
    const float sy = v * (float)h - 0.5f;
    const int ix = (int)floorf(sx);
    const int iy = (int)floorf(sy);
    const float fx = sx - (float)ix;
    const float fy = sy - (float)iy;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        out[c] = 0.f;
    }
#pragma unroll
    for (int dy = 0; dy <= 1; dy++) {
#pragma unroll
        for (int dx = 0; dx <= 1; dx++) {
            const int x = min(max(ix + dx, 0), w - 1);
            const int y = min(max(iy + dy, 0), h - 1);
            const float wgt = (dx == 0 ? 1.f - fx : fx) * (dy == 0 ? 1.f - fy : fy);
            const float* p = data + ((size_t)y * w + (size_t)x) * n;
            for (uint32_t c = 0; c < n; c++) {
                out[c] += wgt * p[c];
            }
        }
    }
}

// The same for an RGBA texture (one 16-byte load per tap).
__device__ __forceinline__ float4 bilerp_clamp4(const float4* tex, int w, int h, float u, float v) {
    const float sx = u * (float)w - 0.5f;
    const float sy = v * (float)h - 0.5f;
    const int ix = (int)floorf(sx);
    const int iy = (int)floorf(sy);
    const float fx = sx - (float)ix;
    const float fy = sy - (float)iy;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int dy = 0; dy <= 1; dy++) {
#pragma unroll
        for (int dx = 0; dx <= 1; dx++) {
            const int x = min(max(ix + dx, 0), w - 1);
            const int y = min(max(iy + dy, 0), h - 1);
            const float wgt = (dx == 0 ? 1.f - fx : fx) * (dy == 0 ? 1.f - fy : fy);
            const float4 p = tex[(size_t)y * w + x];
            o.x += wgt * p.x;
            o.y += wgt * p.y;
            o.z += wgt * p.z;
            o.w += wgt * p.w;
        }
    }
    return o;
}

// Tent weight of screen pixel uv `suv` on texel (tx, ty)
// (f_ops.cpp:2712-2718): max(0, 1 - |s - t|) per axis at s = uv * size - 0.5.
__device__ __forceinline__ float tent_weight(float2 suv, int tw, int th, int tx, int ty) {
    const float stx = suv.x * (float)tw - 0.5f;
    const float sty = suv.y * (float)th - 0.5f;
    const float a = 1.f - fabsf(stx - (float)tx);
    const float b = 1.f - fabsf(sty - (float)ty);
    return (a > 0.f ? a : 0.f) * (b > 0.f ? b : 0.f);
}

// ---------------------------------------------------------------------------
// Per-op kernels (reference layouts)
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void k_texture_bilinear_op(const float* tex, int tw, int th,
                                                             uint32_t n_comp, const float2* uv,
                                                             size_t n_px, float* out) {
    const size_t p = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= n_px) {
        return;
    }
    const float2 q = uv[p];
    float o[4];
    bilerp_clamp_n(tex, tw, th, n_comp, q.x, q.y, o);
    for (uint32_t c = 0; c < n_comp; c++) {
        out[p * n_comp + c] = o[c];
    }
}

// GatherByInverseUVBilinear (f_ops.cpp:2665-2731), one thread per texel.
__global__ __launch_bounds__(256) void k_gather_bilinear_op(const float* gy, uint32_t n_comp,
                                                            int sw, int sh, const float4* inv_uv,
                                                            int tw, int th, const float2* uv,
                                                            float* out) {
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= tw * th) {
        return;
    }
    const int ty = q / tw, tx = q - ty * tw;
    float4 iv = inv_uv[q];
    for (int ny = -4; ny <= 4 && iv.z < 0.5f; ny++) {
        for (int nx = -4; nx <= 4; nx++) {
            const int px = tx + nx, py = ty + ny;
            if (px < 0 || py < 0 || px >= tw || py >= th) {
                continue;
            }
            iv = inv_uv[(size_t)py * tw + px];
            if (iv.z > 0.5f) {
                break;
            }
        }
    }
    float o[4] = {0.f, 0.f, 0.f, 0.f};
    if (iv.z > 0.5f) {
        const int scx = (int)iv.x, scy = (int)iv.y;
        for (int dy = -3; dy <= 3; dy++) {
            for (int dx = -3; dx <= 3; dx++) {
                const int spx = scx + dx, spy = scy + dy;
                if (spx < 0 || spy < 0 || spx >= sw || spy >= sh) {
                    continue;
                }
                const size_t sp = (size_t)spy * sw + spx;
                const float w = tent_weight(uv[sp], tw, th, tx, ty);
                if (w > 0.f) {
                    for (uint32_t c = 0; c < n_comp; c++) {
                        o[c] += gy[sp * n_comp + c] * w;
                    }
                }
            }
        }
    }
    for (uint32_t c = 0; c < n_comp; c++) {
        out[(size_t)q * n_comp + c] = o[c];
    }
}

// Anchor of texel (tx, ty) in the inverse-UV table: its own entry when
// covered (.z > 0.5), else the first covered entry of the +-4 neighbourhood
// in row order (f_ops.cpp:2665-2690; the GLSL of GatherByInverseUV,
// src/codegen/glsl_codegen.cpp:664-685, uses the same search).
__device__ __forceinline__ float4 inv_uv_anchor(const float4* inv_uv, int tw, int th, int tx,
                                                int ty) {
    float4 iv = inv_uv[(size_t)ty * tw + tx];
    for (int ny = -4; ny <= 4 && iv.z < 0.5f; ny++) {
        for (int nx = -4; nx <= 4; nx++) {
            const int px = tx + nx, py = ty + ny;
            if (px < 0 || py < 0 || px >= tw || py >= th) {
                continue;
            }
            iv = inv_uv[(size_t)py * tw + px];
            if (iv.z > 0.5f) {
                break;
            }
        }
    }
    return iv;
}

// F::Texture forward (src/core/f_ops.cpp:2605-2639): the GLSL texture()
// read of a nearest, clamp-to-edge sampler (src/vk/executor.cpp:192-202):
// texel (clamp(floor(u tw), 0, tw - 1), clamp(floor(v th), 0, th - 1)).
__global__ __launch_bounds__(256) void k_texture_nearest_op(const float* tex, int tw, int th,
                                                            uint32_t n_comp, const float2* uv,
                                                            size_t n_px, float* out) {
    const size_t p = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= n_px) {
        return;
    }
    const float2 q = uv[p];
    const float fx = floorf(q.x * (float)tw), fy = floorf(q.y * (float)th);
    // NaN compares false: it takes texel 0, as a clamp of NaN would
    const int ix = fx >= (float)(tw - 1) ? tw - 1 : (fx > 0.f ? (int)fx : 0);
    const int iy = fy >= (float)(th - 1) ? th - 1 : (fy > 0.f ? (int)fy : 0);
    const float* t = tex + ((size_t)iy * tw + ix) * n_comp;
    for (uint32_t c = 0; c < n_comp; c++) {
        out[p * n_comp + c] = t[c];
    }
}

// GatherByInverseUV, F::Texture's backward w.r.t. the texture (its GLSL,
// src/codegen/glsl_codegen.cpp:657-703): per texel the anchor's screen
// pixel (truncated), then the first pixel of the 7 x 7 window around it
// (row order) whose uv truncates to this texel; the texel takes that
// pixel's gradient (zero when none).
__global__ __launch_bounds__(256) void k_gather_nearest_op(const float* gy, uint32_t n_comp,
                                                           int sw, int sh, const float4* inv_uv,
                                                           int tw, int th, const float2* uv,
                                                           float* out) {
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= tw * th) {
        return;
    }
    const int ty = q / tw, tx = q - ty * tw;
    const float4 iv = inv_uv_anchor(inv_uv, tw, th, tx, ty);
    float o[4] = {0.f, 0.f, 0.f, 0.f};
    if (iv.z > 0.5f) {
        const int scx = (int)iv.x, scy = (int)iv.y;
        bool found = false;
        for (int dy = -3; dy <= 3 && !found; dy++) {
            for (int dx = -3; dx <= 3; dx++) {
                const int spx = scx + dx, spy = scy + dy;
                if (spx < 0 || spy < 0 || spx >= sw || spy >= sh) {
                    continue;
                }
                const size_t sp = (size_t)spy * sw + spx;
                const float2 su = uv[sp];
                if ((int)(su.x * (float)tw) == tx && (int)(su.y * (float)th) == ty) {
                    for (uint32_t c = 0; c < n_comp; c++) {
                        o[c] = gy[sp * n_comp + c];
                    }
                    found = true;
                    break;
                }
            }
        }
    }
    for (uint32_t c = 0; c < n_comp; c++) {
        out[(size_t)q * n_comp + c] = o[c];
    }
}

// ScreenAttr (src/core/mesh_utils.cpp:191-203).
__global__ __launch_bounds__(256) void k_screen_attr_op(const float4* clip, uint32_t n, float W,
                                                        float H, float4* out) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) {
        return;
    }
    const float4 c = clip[i];
    const float ndc_x = c.x / c.w;
    const float ndc_y = c.y / c.w;
    out[i] = make_float4((ndc_x * 0.5f + 0.5f) * W, (ndc_y * 0.5f + 0.5f) * H, 1.f, 0.f);
}

// ---------------------------------------------------------------------------
// The fused texture-fit plan
// ---------------------------------------------------------------------------

struct TexDev {
    HsrDev r;               // screen raster: g (S x S, N views), n_verts, faces, clip
                            // [N][V], arecs [N][F], bins, ids [N][S][S]
    int tw, th;
    uint32_t n_sets;
    float inv_px, lr, b1, b2, eps;
    const float* pos;       // [V][3]
    const float2* uv;       // [V]
    const float* mvps;      // [n_sets][N][16]
    float2* sattr;          // [N][V] ScreenAttr x, y
    const float4* texel;    // [T]: the inverse-UV anchor's UV-raster record: barycentrics
                            // l0, l1, l2 and bits(face + 1), zero when no anchor
    const float4* gt;       // [T] target texture
    float4* tex;            // [T]
    float4* m;
    float4* v;
    float* t;
    float* t_next;          // t + 1, written by k_tex_clip for k_tex_bwd_adam
    float2* suv;            // [N][S][S] g_uv
    float4* gs;             // [N][S][S] d loss / d TextureBilinear(tex) output
    uint32_t* key;          // [N][S][S] floor(uv * T - 0.5) + 1 as x | y << 16 (clamped)
    float4* loss;           // [S][S]
    float4* pred;           // [N][S][S] or null
    float4* target;         // [N][S][S] or null
    float4* grad;           // [T] or null
    const float2* bc_tab;
    uint32_t bc_len;
    uint32_t ext_clip;      // clip and sattr come from dressi_tex_set_clips
};

// Per (view, vertex): clip = MVP * (pos, 1) with the cameras of set
// t mod n_sets (TransformToClip, examples/common/asset_utils.cpp:768-782),
// and its ScreenAttr x / y.
__global__ __launch_bounds__(256) void k_tex_clip(TexDev d) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t nv = d.r.n_verts;
    if (i >= d.r.g.n_views * nv) {
        return;
    }
    if (i == 0) {
        // the backward never reads t itself, so its first thread may store
        // t + 1 without racing the others
        *d.t_next = *d.t + 1.f;
    }
    if (d.ext_clip) {
        return;  // the caller's clip and ScreenAttr images
    }
    const uint32_t view = i / nv;
    const uint32_t vtx = i - view * nv;
    const uint32_t set = (uint32_t)(*d.t) % d.n_sets;
    const float* m = d.mvps + ((size_t)set * d.r.g.n_views + view) * 16;
    const float4 c = mvp_transform(m, d.pos[vtx * 3 + 0], d.pos[vtx * 3 + 1], d.pos[vtx * 3 + 2]);
    d.r.clip[i] = c;
    const float ndc_x = c.x / c.w;
    const float ndc_y = c.y / c.w;
    d.sattr[i] = make_float2((ndc_x * 0.5f + 0.5f) * (float)d.r.g.width,
                             (ndc_y * 0.5f + 0.5f) * (float)d.r.g.height);
}

// The inverse-UV anchor of every texel (view-independent, so computed once):
// the texel's own UV-raster record when covered, else that of the first
// covered texel of the +-4 neighbourhood in row order
// (GatherByInverseUVBilinear's dilation, f_ops.cpp:2679-2697), else zero.
__global__ __launch_bounds__(256) void k_tex_anchor(const float4* own, int tw, int th,
                                                    float4* anchor) {
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= tw * th) {
        return;
    }
    const int ty = q / tw, tx = q - ty * tw;
    float4 rec = own[q];
    bool cov = __float_as_uint(rec.w) != 0u;
    for (int ny = -4; ny <= 4 && !cov; ny++) {
        for (int nx = -4; nx <= 4; nx++) {
            const int px = tx + nx, py = ty + ny;
            if (px < 0 || py < 0 || px >= tw || py >= th) {
                continue;
            }
            rec = own[(size_t)py * tw + px];
            if (__float_as_uint(rec.w) != 0u) {
                cov = true;
                break;
            }
        }
    }
    anchor[q] = cov ? rec : make_float4(0.f, 0.f, 0.f, __uint_as_float(0u));
}

// Rasterize of the UV layout (UvAsClip: w = 1, so the perspective-correct
// weights are the barycentrics): per texel the winner's barycentrics and
// face + 1 (0 = uncovered).
__global__ __launch_bounds__(256) void k_tex_texels(HsrDev u, float4* texel) {
    const uint32_t q = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t w = u.g.width;
    if (q >= w * u.g.height) {
        return;
    }
    const uint32_t id = u.ids[q];
    float4 out = make_float4(0.f, 0.f, 0.f, __uint_as_float(0u));
    if (id) {
        const AaRec& r = u.arecs[id - 1];
        const uint32_t py = q / w, px = q - py * w;
        float l0, l1, l2;
        barycentric((float)px + 0.5f, (float)py + 0.5f, r.x[0], r.y[0], r.x[1], r.y[1], r.x[2],
                    r.y[2], r.inv_area, &l0, &l1, &l2);
        out = make_float4(l0, l1, l2, __uint_as_float(id));
    }
    texel[q] = out;
}

// One view's inverse-UV entry of a covered texel (Rasterize of ScreenAttr
// over the UV layout, cpu_raster.cpp:209-222 with inv_w = 1):
// (sum_k l_k a_k) / (l0 + l1 + l2) for the screen x and y.
__device__ __forceinline__ float2 tex_inv_uv(const TexDev& d, uint32_t view, float4 rec) {
    const uint32_t f = __float_as_uint(rec.w) - 1u;
    const float2* sa = d.sattr + (size_t)view * d.r.n_verts;
    const float2 a0 = sa[d.r.faces[f * 3 + 0]];
    const float2 a1 = sa[d.r.faces[f * 3 + 1]];
    const float2 a2 = sa[d.r.faces[f * 3 + 2]];
    const float l0 = rec.x * 1.f, l1 = rec.y * 1.f, l2 = rec.z * 1.f;
    const float denom = l0 + l1 + l2;
    float nx = 0.f, ny = 0.f;
    nx += l0 * a0.x;
    nx += l1 * a1.x;
    nx += l2 * a2.x;
    ny += l0 * a0.y;
    ny += l1 * a1.y;
    ny += l2 * a2.y;
    return make_float2(nx / denom, ny / denom);
}

// Forward of every view for 64 pixels of a row (one wave per view): the
// screen raster's winner gives g_uv and g_mask (perspective-correct,
// cpu_raster.cpp:209-222), both textures are sampled, and the loss image
// (SumPixelWise over the views, through LDS) plus d loss / d sample are
// written. Also clears the bin counters (the raster has consumed them).
template <int NV>
__global__ __launch_bounds__(64 * NV) void k_tex_fwd(TexDev d) {
    __shared__ float4 lv[NV][64];
    const uint32_t view = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    {
        const uint32_t nthr = gridDim.x * gridDim.y * blockDim.x;
        const uint32_t gid = (blockIdx.y * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x;
        for (uint32_t b = gid; b < d.r.bins.n_bins; b += nthr) {
            d.r.bins.counts[b] = 0;
        }
    }
    const uint32_t w = d.r.g.width, h = d.r.g.height;
    const uint32_t x = blockIdx.x * 64 + (uint32_t)lane;
    const uint32_t y = blockIdx.y;
    const bool on = x < w;
    const size_t npx = (size_t)w * h;
    const size_t o = (size_t)y * w + x;
    float4 l = make_float4(0.f, 0.f, 0.f, 0.f);
    if (on) {
        const size_t vo = view * npx + o;
        const uint32_t id = d.r.ids[vo];
        float u = 0.f, v = 0.f, mask = 0.f;
        if (id) {
            const uint32_t f = id - 1;
            const size_t vf = (size_t)view * d.r.g.n_faces + f;
            const AaRec& rec = d.r.arecs[vf];
            // the face's 1 / w and uv corners, beside its record (AA setup)
            const float4 t0 = d.r.tface[vf * 3], t1 = d.r.tface[vf * 3 + 1],
                         t2 = d.r.tface[vf * 3 + 2];
            float l0, l1, l2;
            barycentric((float)x + 0.5f, (float)y + 0.5f, rec.x[0], rec.y[0], rec.x[1], rec.y[1],
                        rec.x[2], rec.y[2], rec.inv_area, &l0, &l1, &l2);
            const float lw0 = l0 * t0.x;
            const float lw1 = l1 * t0.y;
            const float lw2 = l2 * t0.z;
            const float denom = lw0 + lw1 + lw2;
            const float2 a0 = make_float2(t1.x, t1.y), a1 = make_float2(t1.z, t1.w),
                         a2 = make_float2(t2.x, t2.y);
            float nu = 0.f, nvv = 0.f, nm = 0.f;
            nu += lw0 * a0.x;
            nu += lw1 * a1.x;
            nu += lw2 * a2.x;
            nvv += lw0 * a0.y;
            nvv += lw1 * a1.y;
            nvv += lw2 * a2.y;
            nm += lw0 * 1.f;
            nm += lw1 * 1.f;
            nm += lw2 * 1.f;
            u = nu / denom;
            v = nvv / denom;
            mask = nm / denom;
        }
        const float4 st = bilerp_clamp4(d.gt, d.tw, d.th, u, v);
        const float4 sp = bilerp_clamp4(d.tex, d.tw, d.th, u, v);
        const float sti[4] = {st.x, st.y, st.z, st.w};
        const float spi[4] = {sp.x, sp.y, sp.z, sp.w};
        const float kw[4] = {d.inv_px, d.inv_px, d.inv_px, 0.f};
        float li[4], gi[4], ti[4], pi[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            ti[k] = mask * sti[k];
            pi[k] = mask * spi[k];
            const float diff = ti[k] - pi[k];
            li[k] = diff * diff * kw[k];
            // image loss seeded with 1: d diff = (0 + c diff) + c diff,
            // d pred = -d diff, d sample = d pred * g_mask
            const float cd = kw[k] * diff;
            float gd = 0.f;
            gd += cd;
            gd += cd;
            gi[k] = -gd * mask;
        }
        d.suv[vo] = make_float2(u, v);
        d.gs[vo] = make_float4(gi[0], gi[1], gi[2], gi[3]);
        // the texels this pixel's tent can weigh: floor(s) + {0, 1} at
        // s = uv * T - 0.5 (exactly the backward's s); NaN and far values
        // clamp to keys no texel matches (or to one whose exact weight is 0)
        const float kx = fminf(fmaxf(floorf(u * (float)d.tw - 0.5f) + 1.f, 0.f), 65535.f);
        const float ky = fminf(fmaxf(floorf(v * (float)d.th - 0.5f) + 1.f, 0.f), 65535.f);
        d.key[vo] = (uint32_t)kx | ((uint32_t)ky << 16);
        if (d.pred) {
            d.pred[vo] = make_float4(pi[0], pi[1], pi[2], pi[3]);
            d.target[vo] = make_float4(ti[0], ti[1], ti[2], ti[3]);
        }
        l = make_float4(li[0], li[1], li[2], li[3]);
    }
    lv[view][lane] = l;
    __syncthreads();
    if (view == 0 && on) {
        float in[NV][4];
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const float4 q = lv[k][lane];
            in[k][0] = q.x;
            in[k][1] = q.y;
            in[k][2] = q.z;
            in[k][3] = q.w;
        }
        float out[4];
        Tree<NV, 4>::run(in, out);
        d.loss[o] = make_float4(out[0], out[1], out[2], out[3]);
    }
}

constexpr int kTexStage = 1024;  // tent keys of one view staged in LDS per wave

// Per texel (one wave per 8 x 8 texel block): GatherByInverseUVBilinear of
// every view -- the anchor from the UV raster and that view's ScreenAttr
// (the +-4 dilation for uncovered texels), the 7 x 7 window in row order.
// A window pixel can weigh the texel only when its tent key names it (every
// pixel whose exact weight can be > 0 does): the keys of the union of the
// wave's windows are staged in LDS when they fit, and each staged pixel sets
// its window bit in the masks of the (at most four) texels of the block its
// key names whose window holds it (else each texel scans its window); the
// candidates' g_uv / gradient are then loaded four at a time and the weights
// added in window order. The views' contributions are summed
// newest first through the <= 4-ary tree, then Adam on the
// RGBA texel at step t + 1 (t_next, published by k_tex_clip); the first
// thread stores t + 1.
template <int NV>
__global__ __launch_bounds__(64) void k_tex_bwd_adam(TexDev d) {
    __shared__ uint32_t lk[kTexStage];
    __shared__ int lsx[64], lsy[64];              // the texels' window centres (INT_MIN: none)
    __shared__ unsigned long long lcm[64];        // the texels' candidate window bits
    const int lane = (int)threadIdx.x;
    const int tw = d.tw, th = d.th;
    const int sw = (int)d.r.g.width, sh = (int)d.r.g.height;
    const size_t npx = (size_t)sw * sh;
    const int bxn = (tw + 7) / 8;
    const int tx = (int)(blockIdx.x % (uint32_t)bxn) * 8 + (lane & 7);
    const int ty = (int)(blockIdx.x / (uint32_t)bxn) * 8 + (lane >> 3);
    const bool valid = tx < tw && ty < th;
    const uint32_t q = valid ? (uint32_t)(ty * tw + tx) : 0u;
    const float t_new = *d.t_next;
    // the anchor texel's UV-raster record (own or dilated, precomputed) and
    // its face's corners
    const float4 rec = valid ? d.texel[q] : make_float4(0.f, 0.f, 0.f, 0.f);
    const bool cov = __float_as_uint(rec.w) != 0u;
    int32_t c0 = 0, c1 = 0, c2 = 0;
    if (cov) {
        const uint32_t f = __float_as_uint(rec.w) - 1u;
        c0 = d.r.faces[f * 3 + 0];
        c1 = d.r.faces[f * 3 + 1];
        c2 = d.r.faces[f * 3 + 2];
    }
    float cin[NV][4];  // the views' contributions (constant indices: registers)
#pragma unroll 1
    for (int view = 0; view < NV; view++) {
        int scx = 0, scy = 0;
        bool act = false;
        if (cov) {
            // the view's inverse-UV entry: (sum_k l_k a_k) / (l0 + l1 + l2)
            const float2* sa = d.sattr + (size_t)view * d.r.n_verts;
            const float2 a0 = sa[c0], a1 = sa[c1], a2 = sa[c2];
            const float denom = rec.x + rec.y + rec.z;
            float nx = 0.f, ny = 0.f;
            nx += rec.x * a0.x;
            nx += rec.y * a1.x;
            nx += rec.z * a2.x;
            ny += rec.x * a0.y;
            ny += rec.y * a1.y;
            ny += rec.z * a2.y;
            scx = (int)(nx / denom);
            scy = (int)(ny / denom);
            act = scx + 3 >= 0 && scx - 3 < sw && scy + 3 >= 0 && scy - 3 < sh;
        }
        // the wave's union of windows, clipped to the screen
        int x0 = act ? max(scx - 3, 0) : 0x7fffffff;
        int y0 = act ? max(scy - 3, 0) : 0x7fffffff;
        int x1 = act ? min(scx + 3, sw - 1) : -1;
        int y1 = act ? min(scy + 3, sh - 1) : -1;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            x0 = min(x0, __shfl_xor(x0, o));
            y0 = min(y0, __shfl_xor(y0, o));
            x1 = max(x1, __shfl_xor(x1, o));
            y1 = max(y1, __shfl_xor(y1, o));
        }
        const int bw = x1 - x0 + 1, bh = y1 - y0 + 1;
        const bool staged = x0 <= x1 && bw * bh <= kTexStage;
        const uint32_t* keys = d.key + (size_t)view * npx;
        if (staged) {
            for (int i = lane; i < bw * bh; i += 64) {
                const int ry = i / bw;
                lk[i] = keys[(size_t)(y0 + ry) * sw + (x0 + i - ry * bw)];
            }
            __syncthreads();
        }
        // candidate window positions (bit (dy + 3) * 7 + dx + 3)
        uint64_t cm = 0;
        if (staged) {
            lsx[lane] = act ? scx : INT_MIN;
            lsy[lane] = scy;
            lcm[lane] = 0ull;
            __syncthreads();
            const int bx0 = (int)(blockIdx.x % (uint32_t)bxn) * 8;
            const int by0 = (int)(blockIdx.x / (uint32_t)bxn) * 8;
            for (int i = lane; i < bw * bh; i += 64) {
                const int ry = i / bw;
                const int px = x0 + i - ry * bw, py = y0 + ry;
                const uint32_t k = lk[i];
                const int kx = (int)(k & 0xffffu), ky = (int)(k >> 16);
#pragma unroll
                for (int dy = 0; dy < 2; dy++) {
#pragma unroll
                    for (int dx = 0; dx < 2; dx++) {
                        // texel (kx - 1 + dx, ky - 1 + dy): tx + 1 - kx in {0, 1}
                        const int lx = kx - 1 + dx - bx0, ly = ky - 1 + dy - by0;
                        if (lx < 0 || lx >= 8 || ly < 0 || ly >= 8) {
                            continue;
                        }
                        const int t = ly * 8 + lx;
                        const int cx = lsx[t];
                        if (cx == INT_MIN) {
                            continue;
                        }
                        const int wx = px - cx + 3, wy = py - lsy[t] + 3;
                        if (wx >= 0 && wx < 7 && wy >= 0 && wy < 7) {
                            atomicOr(&lcm[t], 1ull << (wy * 7 + wx));
                        }
                    }
                }
            }
            __syncthreads();
            cm = act ? (uint64_t)lcm[lane] : 0ull;
        } else if (act) {
#pragma unroll
            for (int r = 0; r < 7; r++) {
                const int spy = scy + r - 3;
                if (spy < 0 || spy >= sh) {
                    continue;
                }
#pragma unroll
                for (int i = 0; i < 7; i++) {
                    const int spx = scx + i - 3;
                    if (spx < 0 || spx >= sw) {
                        continue;
                    }
                    const uint32_t k = staged ? lk[(spy - y0) * bw + (spx - x0)]
                                              : keys[(size_t)spy * sw + spx];
                    const uint32_t kx = k & 0xffffu, ky = k >> 16;
                    if ((uint32_t)(tx + 1 - (int)kx) <= 1u && (uint32_t)(ty + 1 - (int)ky) <= 1u) {
                        cm |= 1ull << (r * 7 + i);
                    }
                }
            }
        }
        float o4[4] = {0.f, 0.f, 0.f, 0.f};
        const float2* suv = d.suv + (size_t)view * npx;
        const float4* gs = d.gs + (size_t)view * npx;
        while (cm) {
            // up to four candidates: their loads in flight together, then
            // the exact weights added in window order
            size_t sp[4];
            bool on[4];
            float2 u4[4];
            float4 g4[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                on[c] = cm != 0;
                const int kb = on[c] ? __builtin_ctzll(cm) : 0;
                cm &= on[c] ? cm - 1 : cm;
                const int r = kb / 7, i = kb - r * 7;
                sp[c] = on[c] ? (size_t)(scy + r - 3) * sw + (size_t)(scx + i - 3) : 0;
                u4[c] = on[c] ? suv[sp[c]] : make_float2(0.f, 0.f);
                g4[c] = on[c] ? gs[sp[c]] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int c = 0; c < 4; c++) {
                if (on[c]) {
                    const float wgt = tent_weight(u4[c], tw, th, tx, ty);
                    if (wgt > 0.f) {
                        o4[0] += g4[c].x * wgt;
                        o4[1] += g4[c].y * wgt;
                        o4[2] += g4[c].z * wgt;
                        o4[3] += g4[c].w * wgt;
                    }
                }
            }
        }
#pragma unroll
        for (int k = 0; k < NV; k++) {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                cin[k][c] = k == view ? o4[c] : cin[k][c];
            }
        }
        if (staged) {
            __syncthreads();  // the next view restages lk
        }
    }
    if (valid) {
        // the views' contributions, newest first
        float in[NV][4];
#pragma unroll
        for (int vi = 0; vi < NV; vi++) {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                in[vi][c] = cin[NV - 1 - vi][c];
            }
        }
        float g[4];
        Tree<NV, 4>::run(in, g);
        if (d.grad) {
            d.grad[q] = make_float4(g[0], g[1], g[2], g[3]);
        }
        float bc1, bc2;
        if (t_new >= 1.f && t_new <= (float)d.bc_len && t_new == floorf(t_new)) {
            const float2 bc = d.bc_tab[(uint32_t)t_new - 1];
            bc1 = bc.x;
            bc2 = bc.y;
        } else {
            bc1 = 1.f - powf(d.b1, t_new);
            bc2 = 1.f - powf(d.b2, t_new);
        }
        const float cb1 = 1.f - d.b1, cb2 = 1.f - d.b2;
        const float4 p4 = d.tex[q], m4 = d.m[q], v4 = d.v[q];
        float pi[4] = {p4.x, p4.y, p4.z, p4.w};
        float mi[4] = {m4.x, m4.y, m4.z, m4.w};
        float vi4[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float m_new = mi[c] * d.b1 + g[c] * cb1;
            const float v_new = vi4[c] * d.b2 + g[c] * g[c] * cb2;
            const float step = (m_new / bc1) / (sqrtf(v_new / bc2) + d.eps) * d.lr;
            pi[c] = pi[c] - step;
            mi[c] = m_new;
            vi4[c] = v_new;
        }
        d.tex[q] = make_float4(pi[0], pi[1], pi[2], pi[3]);
        d.m[q] = make_float4(mi[0], mi[1], mi[2], mi[3]);
        d.v[q] = make_float4(vi4[0], vi4[1], vi4[2], vi4[3]);
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        *d.t = t_new;
    }
}

constexpr int kTexKernels = 5;
const char* const kTexKernelNames[kTexKernels] = {"k_tex_clip", "k_aa_setup", "k_aa_raster",
                                                  "k_tex_fwd", "k_tex_bwd_adam"};

int launch_tex_kernel(const TexDev& d, hipStream_t s, int k) {
    const RasterGeom& g = d.r.g;
    switch (k) {
        case 0:
            hipLaunchKernelGGL(k_tex_clip, dim3(div_up(g.n_views * d.r.n_verts, 256)), dim3(256),
                               0, s, d);
            break;
        case 1:
            return launch_aa_setup(d.r, s);
        case 2:
            return launch_aa_raster(d.r, s);
        default: {
            const dim3 grid = k == 3 ? dim3(div_up(g.width, 64), g.height)
                                     : dim3(div_up((uint32_t)d.tw, 8) * div_up((uint32_t)d.th, 8));
            switch (g.n_views) {
#define DRESSI_NV(N)                                                                      \
    case N:                                                                               \
        if (k == 3) {                                                                     \
            hipLaunchKernelGGL(k_tex_fwd<N>, grid, dim3(64 * N), 0, s, d);                \
        } else {                                                                          \
            hipLaunchKernelGGL(k_tex_bwd_adam<N>, grid, dim3(64), 0, s, d);               \
        }                                                                                 \
        break;
                DRESSI_NV(1) DRESSI_NV(2) DRESSI_NV(3) DRESSI_NV(4)
                DRESSI_NV(5) DRESSI_NV(6) DRESSI_NV(7) DRESSI_NV(8)
#undef DRESSI_NV
                default:
                    set_error("n_views %u unsupported", g.n_views);
                    return DRESSI_ERR_UNSUPPORTED;
            }
            break;
        }
    }
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

}  // namespace
}  // namespace dressi

using namespace dressi;

struct dressi_tex_plan {
    dressi_ctx* ctx = nullptr;
    dressi_tex_desc desc{};
    TexDev d{};
    std::vector<void*> allocs;
    void* bin_mem = nullptr;
    size_t bin_bytes = 0;
    bool mesh_set = false, cams_set = false, target_set = false, clips_set = false;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    hipStream_t graph_stream = nullptr;
};

namespace {

template <typename T>
int tex_alloc(dressi_tex_plan* p, T** out, size_t count) {
    void* ptr = nullptr;
    DRESSI_TRY_HIP(hipMalloc(&ptr, sizeof(T) * (count ? count : 1)));
    p->allocs.push_back(ptr);
    *out = (T*)ptr;
    return DRESSI_OK;
}

void tex_drop_graph(dressi_tex_plan* p) {
    if (p->exec) {
        hipGraphExecDestroy(p->exec);
        p->exec = nullptr;
    }
    if (p->graph) {
        hipGraphDestroy(p->graph);
        p->graph = nullptr;
    }
}

int tex_ready(dressi_tex_plan* p) {
    DRESSI_REQUIRE(p, "NULL plan");
    DRESSI_REQUIRE(p->mesh_set, "dressi_tex_set_mesh() must be called before stepping");
    if (p->d.ext_clip) {
        DRESSI_REQUIRE(p->clips_set, "dressi_tex_set_clips() must be called before stepping");
    } else {
        DRESSI_REQUIRE(p->cams_set, "dressi_tex_set_cameras() must be called before stepping");
    }
    DRESSI_REQUIRE(p->target_set, "dressi_tex_set_target() must be called before stepping");
    return DRESSI_OK;
}

int tex_enqueue(dressi_tex_plan* p, hipStream_t s) {
    for (int k = 0; k < kTexKernels; k++) {
        if (int rc = launch_tex_kernel(p->d, s, k)) return rc;
    }
    return DRESSI_OK;
}

}  // namespace

extern "C" {

int dressi_texture_bilinear(dressi_ctx* ctx, const float* tex, uint32_t tw, uint32_t th,
                            uint32_t n_comp, const float* uv, uint32_t uw, uint32_t uh,
                            float* out) {
    DRESSI_REQUIRE(ctx && tex && uv && out, "bad arguments");
    DRESSI_REQUIRE(n_comp >= 1 && n_comp <= 4, "n_comp must be 1..4");
    DRESSI_REQUIRE(tw > 0 && th > 0 && tw <= 65536 && th <= 65536, "bad texture size");
    const size_t n = (size_t)uw * uh;
    if (!n) return DRESSI_OK;
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    hipLaunchKernelGGL(k_texture_bilinear_op, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0,
                       ctx->stream, tex, (int)tw, (int)th, n_comp, (const float2*)uv, n, out);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int dressi_texture_bilinear_bwd(dressi_ctx* ctx, const float* gy, uint32_t n_comp, uint32_t sw,
                                uint32_t sh, const float* inv_uv, uint32_t tw, uint32_t th,
                                const float* uv, float* out) {
    DRESSI_REQUIRE(ctx && gy && inv_uv && uv && out, "bad arguments");
    DRESSI_REQUIRE(n_comp >= 1 && n_comp <= 4, "n_comp must be 1..4");
    DRESSI_REQUIRE((uint64_t)tw * th < (1ull << 31) && (uint64_t)sw * sh < (1ull << 40),
                   "size too large");
    if (!tw || !th) return DRESSI_OK;
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    hipLaunchKernelGGL(k_gather_bilinear_op, dim3(div_up(tw * th, 256)), dim3(256), 0,
                       ctx->stream, gy, n_comp, (int)sw, (int)sh, (const float4*)inv_uv, (int)tw,
                       (int)th, (const float2*)uv, out);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int dressi_texture_nearest(dressi_ctx* ctx, const float* tex, uint32_t tw, uint32_t th,
                           uint32_t n_comp, const float* uv, uint32_t uw, uint32_t uh,
                           float* out) {
    DRESSI_REQUIRE(ctx && tex && uv && out, "bad arguments");
    DRESSI_REQUIRE(n_comp >= 1 && n_comp <= 4, "n_comp must be 1..4");
    DRESSI_REQUIRE(tw > 0 && th > 0 && tw <= 65536 && th <= 65536, "bad texture size");
    const size_t n = (size_t)uw * uh;
    if (!n) return DRESSI_OK;
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    hipLaunchKernelGGL(k_texture_nearest_op, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0,
                       ctx->stream, tex, (int)tw, (int)th, n_comp, (const float2*)uv, n, out);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int dressi_texture_nearest_bwd(dressi_ctx* ctx, const float* gy, uint32_t n_comp, uint32_t sw,
                               uint32_t sh, const float* inv_uv, uint32_t tw, uint32_t th,
                               const float* uv, float* out) {
    DRESSI_REQUIRE(ctx && gy && inv_uv && uv && out, "bad arguments");
    DRESSI_REQUIRE(n_comp >= 1 && n_comp <= 4, "n_comp must be 1..4");
    DRESSI_REQUIRE((uint64_t)tw * th < (1ull << 31) && (uint64_t)sw * sh < (1ull << 40),
                   "size too large");
    if (!tw || !th) return DRESSI_OK;
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    hipLaunchKernelGGL(k_gather_nearest_op, dim3(div_up(tw * th, 256)), dim3(256), 0,
                       ctx->stream, gy, n_comp, (int)sw, (int)sh, (const float4*)inv_uv, (int)tw,
                       (int)th, (const float2*)uv, out);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int dressi_screen_attr(dressi_ctx* ctx, const float* clip, uint32_t n_verts, uint32_t width,
                       uint32_t height, float* out) {
    DRESSI_REQUIRE(ctx && clip && out, "bad arguments");
    if (!n_verts) return DRESSI_OK;
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    hipLaunchKernelGGL(k_screen_attr_op, dim3(div_up(n_verts, 256)), dim3(256), 0, ctx->stream,
                       (const float4*)clip, n_verts, (float)width, (float)height, (float4*)out);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int dressi_uv_sphere(uint32_t stacks, uint32_t slices, uint32_t* n_verts, uint32_t* n_faces,
                     float* pos, float* uv, float* faces) {
    DRESSI_REQUIRE(n_verts && n_faces, "bad arguments");
    stacks = stacks < 2u ? 2u : stacks;
    slices = slices < 3u ? 3u : slices;
    DRESSI_REQUIRE((uint64_t)(stacks + 1) * (slices + 1) < (1ull << 24), "sphere too large");
    const uint32_t cols = slices + 1;
    *n_verts = cols * (stacks + 1);
    *n_faces = 2 * stacks * slices - 2 * slices;
    if (!pos || !uv || !faces) {
        return DRESSI_OK;
    }
    const float pi = 3.14159265358979323846f;
    for (uint32_t i = 0; i <= stacks; i++) {
        const float theta = pi * (float)i / (float)stacks;
        const float st = std::sin(theta), ct = std::cos(theta);
        for (uint32_t j = 0; j <= slices; j++) {
            const float phi = 2.f * pi * (float)j / (float)slices;
            const uint32_t v = i * cols + j;
            pos[v * 3 + 0] = st * std::cos(phi);
            pos[v * 3 + 1] = ct;
            pos[v * 3 + 2] = st * std::sin(phi);
            uv[v * 2 + 0] = (float)j / (float)slices;
            uv[v * 2 + 1] = (float)i / (float)stacks;
        }
    }
    uint32_t f = 0;
    for (uint32_t i = 0; i < stacks; i++) {
        for (uint32_t j = 0; j < slices; j++) {
            const uint32_t tl = i * cols + j, tr = tl + 1, bl = tl + cols, br = bl + 1;
            if (i != stacks - 1) {
                faces[f * 3 + 0] = (float)tl;
                faces[f * 3 + 1] = (float)br;
                faces[f * 3 + 2] = (float)bl;
                f++;
            }
            if (i != 0) {
                faces[f * 3 + 0] = (float)tl;
                faces[f * 3 + 1] = (float)tr;
                faces[f * 3 + 2] = (float)br;
                f++;
            }
        }
    }
    return DRESSI_OK;
}

void dressi_uv_as_clip(const float* uv, uint32_t n_verts, float* clip) {
    for (uint32_t i = 0; i < n_verts; i++) {
        clip[i * 4 + 0] = uv[i * 2 + 0] * 2.f - 1.f;
        clip[i * 4 + 1] = uv[i * 2 + 1] * 2.f - 1.f;
        clip[i * 4 + 2] = 0.5f;
        clip[i * 4 + 3] = 1.f;
    }
}

int dressi_tex_create(dressi_ctx* ctx, const dressi_tex_desc* desc, dressi_tex_plan** out) {
    DRESSI_REQUIRE(ctx && desc && out, "bad arguments");
    DRESSI_REQUIRE(desc->n_verts > 0 && desc->n_faces > 0, "empty mesh");
    DRESSI_REQUIRE(desc->n_views >= 1 && desc->n_views <= kMaxViews,
                   "n_views must be in [1, %u]", kMaxViews);
    DRESSI_REQUIRE(desc->width > 0 && desc->height > 0 && desc->tex_w > 0 && desc->tex_h > 0,
                   "empty screen or texture");
    DRESSI_REQUIRE(desc->width <= 16384 && desc->height <= 16384 && desc->tex_w <= 16384 &&
                           desc->tex_h <= 16384,
                   "screen and texture sides must be <= 16384");
    DRESSI_REQUIRE(desc->n_sets >= 1, "n_sets must be >= 1");
    DRESSI_REQUIRE((uint64_t)desc->n_views * desc->n_faces < (1ull << 31), "too many faces");
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    dressi_tex_plan* p = new dressi_tex_plan();
    p->ctx = ctx;
    p->desc = *desc;
    TexDev& d = p->d;
    HsrDev& r = d.r;
    r.g = make_geom(desc->width, desc->height, desc->n_views, desc->n_faces);
    r.n_verts = desc->n_verts;
    r.technique = 1;
    d.tw = (int)desc->tex_w;
    d.th = (int)desc->tex_h;
    d.n_sets = desc->n_sets;
    d.inv_px = 1.f / (float)(desc->width * desc->height);
    d.lr = desc->lr;
    d.b1 = desc->beta1;
    d.b2 = desc->beta2;
    d.eps = desc->eps;
    d.ext_clip = (desc->flags & DRESSI_TEX_EXTERNAL_CLIP) ? 1u : 0u;
    const size_t V = desc->n_verts, F = desc->n_faces, N = desc->n_views;
    const size_t npx = (size_t)desc->width * desc->height;
    const size_t T = (size_t)desc->tex_w * desc->tex_h;
    int rc = DRESSI_OK;
    float* pos = nullptr;
    float2* uv = nullptr;
    float* mvps = nullptr;
    float4* texel = nullptr;
    float4* gt = nullptr;
    rc = rc ? rc : tex_alloc(p, &pos, V * 3);
    rc = rc ? rc : tex_alloc(p, &uv, V);
    rc = rc ? rc : tex_alloc(p, &mvps, (size_t)desc->n_sets * N * 16);
    rc = rc ? rc : tex_alloc(p, &d.sattr, N * V);
    rc = rc ? rc : tex_alloc(p, &texel, T);
    rc = rc ? rc : tex_alloc(p, &gt, T);
    rc = rc ? rc : tex_alloc(p, &d.tex, T);
    rc = rc ? rc : tex_alloc(p, &d.m, T);
    rc = rc ? rc : tex_alloc(p, &d.v, T);
    rc = rc ? rc : tex_alloc(p, &d.t, 1);
    rc = rc ? rc : tex_alloc(p, &d.t_next, 1);
    rc = rc ? rc : tex_alloc(p, &d.suv, N * npx);
    rc = rc ? rc : tex_alloc(p, &d.gs, N * npx);
    rc = rc ? rc : tex_alloc(p, &d.key, N * npx);
    rc = rc ? rc : tex_alloc(p, &d.loss, npx);
    rc = rc ? rc : tex_alloc(p, &r.clip, N * V);
    rc = rc ? rc : tex_alloc(p, &r.arecs, std::max(N * F, F));
    rc = rc ? rc : tex_alloc(p, &r.tface, (size_t)N * F * 3);
    rc = rc ? rc : tex_alloc(p, &r.ids, std::max(N * npx, T));
    if (!rc && (desc->flags & DRESSI_TEX_KEEP_IMAGES)) {
        rc = tex_alloc(p, &d.pred, N * npx);
        rc = rc ? rc : tex_alloc(p, &d.target, N * npx);
    }
    if (!rc && (desc->flags & DRESSI_TEX_KEEP_GRAD)) rc = tex_alloc(p, &d.grad, T);
    d.pos = pos;
    d.uv = uv;
    r.tf_uv = uv;
    d.mvps = mvps;
    d.texel = texel;
    d.gt = gt;
    float2* bc = nullptr;
    if (!rc) rc = tex_alloc(p, &bc, kBiasTableLen);
    if (!rc) {
        std::vector<float2> tab(kBiasTableLen);
        for (uint32_t i = 0; i < kBiasTableLen; i++) {
            const float tn = (float)(i + 1);
            tab[i] = make_float2(1.f - powf(desc->beta1, tn), 1.f - powf(desc->beta2, tn));
        }
        hipError_t e = hipMemcpy(bc, tab.data(), sizeof(float2) * kBiasTableLen,
                                 hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            set_error("bias table upload failed: %s", hipGetErrorString(e));
            rc = DRESSI_ERR_HIP;
        }
        d.bc_tab = bc;
        d.bc_len = kBiasTableLen;
    }
    if (!rc) {
        // bins: the screen rasters' N x tiles, or the UV raster's tiles
        const RasterGeom ug = make_geom(desc->tex_w, desc->tex_h, 1, desc->n_faces);
        const uint32_t n_bins = std::max(r.g.n_tiles * r.g.n_views, ug.n_tiles);
        p->bin_bytes = fixed_bin_bytes(n_bins, kSoftBinCap);
        uint32_t* bm = nullptr;
        rc = tex_alloc(p, &bm, p->bin_bytes / sizeof(uint32_t) + 1);
        if (!rc) {
            p->bin_mem = bm;
            fixed_bin_carve(bm, r.g.n_tiles * r.g.n_views, kSoftBinCap, &r.bins);
        }
    }
    if (!rc) {
        hipError_t e = hipMemsetAsync(p->bin_mem, 0, p->bin_bytes, ctx->stream);
        if (e == hipSuccess) e = hipMemsetAsync(d.t, 0, sizeof(float), ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) {
            set_error("plan init failed: %s", hipGetErrorString(e));
            rc = DRESSI_ERR_HIP;
        }
    }
    if (rc) {
        dressi_tex_destroy(p);
        return rc;
    }
    *out = p;
    return DRESSI_OK;
}

int dressi_tex_destroy(dressi_tex_plan* p) {
    if (!p) {
        return DRESSI_OK;
    }
    hipSetDevice(p->ctx->device);
    hipStreamSynchronize(p->ctx->stream);
    tex_drop_graph(p);
    for (void* a : p->allocs) {
        hipFree(a);
    }
    delete p;
    return DRESSI_OK;
}

int dressi_tex_set_mesh(dressi_tex_plan* p, const float* pos, const float* uv,
                        const float* faces) {
    DRESSI_REQUIRE(p && pos && uv && faces, "bad arguments");
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    const uint32_t V = p->desc.n_verts, F = p->desc.n_faces;
    std::vector<int32_t> fi((size_t)F * 3);
    for (size_t i = 0; i < fi.size(); i++) {
        const float x = faces[i];
        DRESSI_REQUIRE(x >= 0.f && x < (float)V, "face index out of range at %zu", i);
        fi[i] = (int32_t)(uint32_t)(int64_t)(x + 0.5f);
    }
    hipStream_t s = p->ctx->stream;
    TexDev& d = p->d;
    if (!p->mesh_set) {
        int32_t* df = nullptr;
        if (int rc = tex_alloc(p, &df, fi.size())) return rc;
        d.r.faces = df;
    }
    std::vector<float> uvc((size_t)V * 4);
    dressi_uv_as_clip(uv, V, uvc.data());
    DRESSI_TRY_HIP(hipMemcpyAsync((void*)d.r.faces, fi.data(), fi.size() * 4,
                                  hipMemcpyHostToDevice, s));
    DRESSI_TRY_HIP(hipMemcpyAsync((void*)d.pos, pos, (size_t)V * 12, hipMemcpyHostToDevice, s));
    DRESSI_TRY_HIP(hipMemcpyAsync((void*)d.uv, uv, (size_t)V * 8, hipMemcpyHostToDevice, s));
    // the UV-space raster (static): UvAsClip positions in the clip buffer,
    // one "view" of T x T, the bins carved for its tiles
    HsrDev u = d.r;
    u.tface = nullptr;  // the attribute corners are the screen raster's
    u.g = make_geom(p->desc.tex_w, p->desc.tex_h, 1, F);
    fixed_bin_carve(p->bin_mem, u.g.n_tiles, kSoftBinCap, &u.bins);
    DRESSI_TRY_HIP(hipMemcpyAsync(u.clip, uvc.data(), uvc.size() * 4, hipMemcpyHostToDevice, s));
    DRESSI_TRY_HIP(hipMemsetAsync(p->bin_mem, 0, p->bin_bytes, s));
    if (int rc = launch_aa_setup(u, s)) return rc;
    if (int rc = launch_aa_raster(u, s)) return rc;
    // own records into the screen-gradient buffer (free until the first
    // iteration), then the anchors
    const uint32_t T = p->desc.tex_w * p->desc.tex_h;
    DRESSI_REQUIRE((size_t)T <= (size_t)p->desc.n_views * p->desc.width * p->desc.height,
                   "texture larger than the screen-gradient scratch");
    float4* own = d.gs;
    hipLaunchKernelGGL(k_tex_texels, dim3(div_up(T, 256)), dim3(256), 0, s, u, own);
    DRESSI_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_tex_anchor, dim3(div_up(T, 256)), dim3(256), 0, s, (const float4*)own,
                       (int)p->desc.tex_w, (int)p->desc.tex_h, (float4*)d.texel);
    DRESSI_CHECK_LAUNCH();
    DRESSI_TRY_HIP(hipMemsetAsync(p->bin_mem, 0, p->bin_bytes, s));
    DRESSI_TRY_HIP(hipStreamSynchronize(s));
    p->mesh_set = true;
    return DRESSI_OK;
}

int dressi_tex_set_cameras(dressi_tex_plan* p, const float* mvps) {
    DRESSI_REQUIRE(p && mvps, "bad arguments");
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    const size_t n = (size_t)p->desc.n_sets * p->desc.n_views * 16;
    DRESSI_TRY_HIP(hipMemcpyAsync((void*)p->d.mvps, mvps, n * 4, hipMemcpyHostToDevice,
                                  p->ctx->stream));
    DRESSI_TRY_HIP(hipStreamSynchronize(p->ctx->stream));
    p->cams_set = true;
    return DRESSI_OK;
}

int dressi_tex_set_clips(dressi_tex_plan* p, const float* clips, const float* attrs) {
    DRESSI_REQUIRE(p && clips && attrs, "bad arguments");
    DRESSI_REQUIRE(p->d.ext_clip, "the plan was not created with DRESSI_TEX_EXTERNAL_CLIP");
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    const size_t nv = (size_t)p->desc.n_views * p->desc.n_verts;
    std::vector<float2> xy(nv);
    for (size_t i = 0; i < nv; i++) {
        DRESSI_REQUIRE(attrs[i * 4 + 2] == 1.f && attrs[i * 4 + 3] == 0.f,
                       "attribute %zu is not a ScreenAttr (z = 1, w = 0)", i);
        xy[i] = make_float2(attrs[i * 4], attrs[i * 4 + 1]);
    }
    hipStream_t s = p->ctx->stream;
    DRESSI_TRY_HIP(hipMemcpyAsync((void*)p->d.r.clip, clips, nv * sizeof(float4),
                                  hipMemcpyHostToDevice, s));
    DRESSI_TRY_HIP(hipMemcpyAsync((void*)p->d.sattr, xy.data(), nv * sizeof(float2),
                                  hipMemcpyHostToDevice, s));
    DRESSI_TRY_HIP(hipStreamSynchronize(s));
    p->clips_set = true;
    return DRESSI_OK;
}

int dressi_tex_set_target(dressi_tex_plan* p, const float* gt_tex) {
    DRESSI_REQUIRE(p && gt_tex, "bad arguments");
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    const size_t T = (size_t)p->desc.tex_w * p->desc.tex_h;
    DRESSI_TRY_HIP(hipMemcpyAsync((void*)p->d.gt, gt_tex, T * 16, hipMemcpyHostToDevice,
                                  p->ctx->stream));
    DRESSI_TRY_HIP(hipStreamSynchronize(p->ctx->stream));
    p->target_set = true;
    return DRESSI_OK;
}

int dressi_tex_set_state(dressi_tex_plan* p, const float* tex, const float* m, const float* v,
                         float t) {
    DRESSI_REQUIRE(p && tex, "bad arguments");
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    hipStream_t s = p->ctx->stream;
    const size_t bytes = (size_t)p->desc.tex_w * p->desc.tex_h * 16;
    DRESSI_TRY_HIP(hipMemcpyAsync(p->d.tex, tex, bytes, hipMemcpyHostToDevice, s));
    if (m) {
        DRESSI_TRY_HIP(hipMemcpyAsync(p->d.m, m, bytes, hipMemcpyHostToDevice, s));
    } else {
        DRESSI_TRY_HIP(hipMemsetAsync(p->d.m, 0, bytes, s));
    }
    if (v) {
        DRESSI_TRY_HIP(hipMemcpyAsync(p->d.v, v, bytes, hipMemcpyHostToDevice, s));
    } else {
        DRESSI_TRY_HIP(hipMemsetAsync(p->d.v, 0, bytes, s));
    }
    DRESSI_TRY_HIP(hipMemcpyAsync(p->d.t, &t, sizeof(float), hipMemcpyHostToDevice, s));
    DRESSI_TRY_HIP(hipStreamSynchronize(s));
    return DRESSI_OK;
}

int dressi_tex_get_state(dressi_tex_plan* p, float* tex, float* m, float* v, float* t) {
    DRESSI_REQUIRE(p, "bad arguments");
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    hipStream_t s = p->ctx->stream;
    const size_t bytes = (size_t)p->desc.tex_w * p->desc.tex_h * 16;
    DRESSI_TRY_HIP(hipStreamSynchronize(s));
    if (tex) DRESSI_TRY_HIP(hipMemcpy(tex, p->d.tex, bytes, hipMemcpyDeviceToHost));
    if (m) DRESSI_TRY_HIP(hipMemcpy(m, p->d.m, bytes, hipMemcpyDeviceToHost));
    if (v) DRESSI_TRY_HIP(hipMemcpy(v, p->d.v, bytes, hipMemcpyDeviceToHost));
    if (t) DRESSI_TRY_HIP(hipMemcpy(t, p->d.t, sizeof(float), hipMemcpyDeviceToHost));
    return DRESSI_OK;
}

int dressi_tex_step_eager(dressi_tex_plan* p, uint32_t n_iters) {
    if (int rc = tex_ready(p)) return rc;
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    for (uint32_t i = 0; i < n_iters; i++) {
        if (int rc = tex_enqueue(p, p->ctx->stream)) return rc;
    }
    return DRESSI_OK;
}

int dressi_tex_step(dressi_tex_plan* p, uint32_t n_iters) {
    if (int rc = tex_ready(p)) return rc;
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    hipStream_t s = p->ctx->stream;
    if (!p->exec || p->graph_stream != s) {
        tex_drop_graph(p);
        hipStream_t cap_stream = nullptr;
        DRESSI_TRY_HIP(hipStreamCreateWithFlags(&cap_stream, hipStreamNonBlocking));
        hipError_t e = hipStreamBeginCapture(cap_stream, hipStreamCaptureModeThreadLocal);
        int rc = DRESSI_OK;
        if (e == hipSuccess) {
            rc = tex_enqueue(p, cap_stream);
            hipError_t e2 = hipStreamEndCapture(cap_stream, &p->graph);
            if (!rc && e2 != hipSuccess) {
                set_error("graph capture failed: %s", hipGetErrorString(e2));
                rc = DRESSI_ERR_HIP;
            }
        } else {
            set_error("hipStreamBeginCapture failed: %s", hipGetErrorString(e));
            rc = DRESSI_ERR_HIP;
        }
        hipStreamDestroy(cap_stream);
        if (rc) {
            tex_drop_graph(p);
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

int dressi_tex_buffer(dressi_tex_plan* p, int which, void** ptr, size_t* bytes) {
    DRESSI_REQUIRE(p && ptr, "bad arguments");
    const size_t npx = (size_t)p->desc.width * p->desc.height;
    const size_t N = p->desc.n_views;
    const size_t T = (size_t)p->desc.tex_w * p->desc.tex_h;
    void* q = nullptr;
    size_t b = 0;
    switch (which) {
        case DRESSI_TEX_LOSS: q = p->d.loss; b = npx * 16; break;
        case DRESSI_TEX_PRED: q = p->d.pred; b = N * npx * 16; break;
        case DRESSI_TEX_TARGET: q = p->d.target; b = N * npx * 16; break;
        case DRESSI_TEX_FACE_ID: q = p->d.r.ids; b = N * npx * 4; break;
        case DRESSI_TEX_GRAD: q = p->d.grad; b = T * 16; break;
        case DRESSI_TEX_TEX: q = p->d.tex; b = T * 16; break;
        case DRESSI_TEX_UV: q = p->d.suv; b = N * npx * 8; break;
        default: DRESSI_REQUIRE(false, "unknown buffer %d", which);
    }
    DRESSI_REQUIRE(q, "buffer %d not kept (see the DRESSI_TEX_KEEP_* flags)", which);
    *ptr = q;
    if (bytes) *bytes = b;
    return DRESSI_OK;
}

int dressi_tex_read(dressi_tex_plan* p, int which, void* host, size_t bytes) {
    void* q = nullptr;
    size_t b = 0;
    if (int rc = dressi_tex_buffer(p, which, &q, &b)) return rc;
    DRESSI_REQUIRE(host && bytes == b, "buffer %d holds %zu bytes, %zu given", which, b, bytes);
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    DRESSI_TRY_HIP(hipStreamSynchronize(p->ctx->stream));
    DRESSI_TRY_HIP(hipMemcpy(host, q, b, hipMemcpyDeviceToHost));
    return DRESSI_OK;
}

int dressi_tex_profile(dressi_tex_plan* p, uint32_t iters, char* names, size_t name_stride,
                       float* usec, uint32_t cap, uint32_t* n) {
    if (int rc = tex_ready(p)) return rc;
    DRESSI_REQUIRE(n, "bad arguments");
    // in place: `iters` eager iterations with a HIP event before each kernel
    // and after the last
    const uint32_t reps = iters ? (iters < 256u ? iters : 256u) : 1u;
    *n = kTexKernels;
    hipStream_t s = p->ctx->stream;
    constexpr int kEv = kTexKernels + 1;
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
        for (int k = 0; k < kTexKernels && !rc; k++) {
            if (hipEventRecord(ev[(size_t)r * kEv + k], s) != hipSuccess) {
                set_error("hipEventRecord failed");
                rc = DRESSI_ERR_HIP;
                break;
            }
            rc = launch_tex_kernel(p->d, s, k);
        }
        if (!rc && hipEventRecord(ev[(size_t)r * kEv + kTexKernels], s) != hipSuccess) {
            set_error("hipEventRecord failed");
            rc = DRESSI_ERR_HIP;
        }
    }
    if (!rc && hipEventSynchronize(ev.back()) != hipSuccess) {
        set_error("event synchronisation failed");
        rc = DRESSI_ERR_HIP;
    }
    float ms[kTexKernels] = {};
    for (uint32_t r = 0; r < reps && !rc; r++) {
        for (int k = 0; k < kTexKernels; k++) {
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
    for (uint32_t k = 0; k < (uint32_t)kTexKernels && k < cap && !rc; k++) {
        if (usec) usec[k] = ms[k] * 1000.f;
        if (names && name_stride > 0) {
            snprintf(names + k * name_stride, name_stride, "%s", kTexKernelNames[k]);
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
