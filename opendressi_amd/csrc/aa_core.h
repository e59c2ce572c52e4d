// aa_core.h -- device side of the screen-space antialiasing (Dr.Hair-style
// AA of the reference, src/core/cpu_raster.cpp:371-454 and
// src/core/f_ops.cpp:2213-2579): the 8-neighbour pair evaluation and the
// per-pair vertex gradient, shared by the per-op kernels and the fused
// silhouette plan.
#pragma once

#include "internal.h"

namespace dressi {

// f_ops.cpp:2213-2214 (kAaOffs)
__device__ __constant__ const int kAaOffX[8] = {-1, 0, 1, -1, 1, -1, 0, 1};
__device__ __constant__ const int kAaOffY[8] = {-1, -1, -1, 0, 0, 1, 1, 1};

// Per (view, face) record of the fused hard raster (RasterizeCore,
// cpu_raster.cpp:42-94): screen corners, 1 / area, coverage margin for the
// block cull (as the soft raster's), inclusive pixel bbox (bx0 > bx1: no
// fragment), NDC z and a depth below every z the face can produce at a
// covered pixel. 16 words; words 0-7 and 8-11 are 16-byte loads of the cull.
struct alignas(16) AaRec {
    float x[3], y[3];
    float inv_area;
    float margin;  // < 0: no cull bound
    int bx0, by0, bx1, by1;
    float z[3];
    float zcull;  // >= 0
};
static_assert(sizeof(AaRec) == 64, "AaRec layout");

// cpu_raster.h:67-74 (AaPair)
struct AaPair {
    float r;
    uint32_t ia, ib;  // vertex ids of the chosen edge
    float qa[2], qb[2];
    float es, len;
};

// EvalAaPair for ids its / itn (face + 1, 0 = background) of pixel s and its
// neighbour n. `tri(f, vi, qx, qy)` gives face f's vertex ids and screen
// corners (ProjectClipToScreen) and returns false where the reference skips
// the owner (a bad index or a corner with |w| <= 1e-6 or w < 0).
template <typename Tri>
__device__ __forceinline__ bool eval_aa_pair(uint32_t its, uint32_t itn, int sx, int sy, int nx,
                                             int ny, uint32_t n_faces, Tri&& tri, AaPair* out) {
    if (its == itn) {
        return false;
    }
    const float ps0 = (float)sx + 0.5f, ps1 = (float)sy + 0.5f;
    const float pn0 = (float)nx + 0.5f, pn1 = (float)ny + 0.5f;
    for (int o = 0; o < 2; o++) {
        const uint32_t owner = o == 0 ? itn : its;
        if (owner == 0) {
            continue;
        }
        const uint32_t f = owner - 1;
        if (f >= n_faces) {
            continue;
        }
        uint32_t vi[3];
        float qx[3], qy[3];
        if (!tri(f, vi, qx, qy)) {
            continue;
        }
        int best_j = -1;
        float best_t = 0.f;
        for (int j = 0; j < 3; j++) {
            const int j1 = (j + 1) % 3;
            const float es = (qx[j1] - qx[j]) * (ps1 - qy[j]) - (qy[j1] - qy[j]) * (ps0 - qx[j]);
            const float en = (qx[j1] - qx[j]) * (pn1 - qy[j]) - (qy[j1] - qy[j]) * (pn0 - qx[j]);
            if (es * en >= 0.f) {
                continue;
            }
            const float t = es / (es - en);
            if (best_j < 0 || (o == 0 ? t > best_t : t < best_t)) {
                best_t = t;
                best_j = j;
            }
        }
        if (best_j < 0) {
            continue;
        }
        const int j1 = (best_j + 1) % 3;
        const float ex = qx[j1] - qx[best_j];
        const float ey = qy[j1] - qy[best_j];
        const float len = sqrtf(ex * ex + ey * ey);
        if (len < 1e-6f) {
            continue;
        }
        const float es = ex * (ps1 - qy[best_j]) - ey * (ps0 - qx[best_j]);
        out->r = smin(fabsf(es) / len, 1.f);
        out->ia = vi[best_j];
        out->ib = vi[j1];
        out->qa[0] = qx[best_j];
        out->qa[1] = qy[best_j];
        out->qb[0] = qx[j1];
        out->qb[1] = qy[j1];
        out->es = es;
        out->len = len;
        return true;
    }
    return false;
}

// Owner triangles from clip positions (per-op layouts): vertex ids from the
// float faces (int64(v + 0.5f)), projected with ProjectClipToScreen.
struct TriFromClip {
    const float* faces;
    const float4* clip;
    uint32_t n_verts;
    float W, H;
    __device__ bool operator()(uint32_t f, uint32_t vi[3], float qx[3], float qy[3]) const {
        for (int k = 0; k < 3; k++) {
            vi[k] = (uint32_t)(int64_t)(faces[(size_t)f * 3 + k] + 0.5f);
            if (vi[k] >= n_verts) {
                return false;
            }
            const float4 c = clip[vi[k]];
            if (!clip_w_valid(c.w)) {
                return false;
            }
            const ScreenVert v = project_to_screen(c.x, c.y, c.z, c.w, W, H);
            qx[k] = v.x;
            qy[k] = v.y;
        }
        return true;
    }
};

// d r / d q_a and d r / d q_b of an active pair at pixel (x, y)
// (f_ops.cpp:2358-2371).
__device__ __forceinline__ void aa_pair_dq(const AaPair& pr, int x, int y, float dqa[2],
                                           float dqb[2]) {
    const float ps0 = (float)x + 0.5f, ps1 = (float)y + 0.5f;
    const float sgn = pr.es >= 0.f ? 1.f : -1.f;
    const float inv_l = 1.f / pr.len;
    const float l3 = fabsf(pr.es) * inv_l * inv_l * inv_l;
    const float ex = pr.qb[0] - pr.qa[0];
    const float ey = pr.qb[1] - pr.qa[1];
    dqa[0] = sgn * inv_l * (pr.qb[1] - ps1) + l3 * ex;
    dqa[1] = sgn * inv_l * (ps0 - pr.qb[0]) + l3 * ey;
    dqb[0] = sgn * inv_l * (ps1 - pr.qa[1]) - l3 * ex;
    dqb[1] = sgn * inv_l * (pr.qa[0] - ps0) - l3 * ey;
}

// Adds the clip-space gradient of one endpoint (f_ops.cpp:2372-2384):
// x: gqx 0.5 W / w, y: gqy 0.5 H / w, w: -(gqx 0.5 W cx + gqy 0.5 H cy) / w^2.
__device__ __forceinline__ void aa_add_endpoint(float gr, const float dq[2], float4 c, float W,
                                                float H, float4* dst) {
    const float gqx = gr * dq[0];
    const float gqy = gr * dq[1];
    dst->x += gqx * 0.5f * W / c.w;
    dst->y += gqy * 0.5f * H / c.w;
    dst->w += -(gqx * 0.5f * W * c.x + gqy * 0.5f * H * c.y) / (c.w * c.w);
}

// The sample pixel of AntiAliasBwdVtx (f_ops.cpp:2431-2450): edge smp % 3 of
// the face's screen triangle s3 (computed with c.xy / c.w), u = hash salt 2,
// offset (hash salt 3 * 2 - 1) * 2 px along the edge normal. False when the
// edge is degenerate.
__device__ __forceinline__ bool aa_sample_px(const float s3x[3], const float s3y[3], uint32_t f,
                                             uint32_t smp, uint32_t seed_u, int* x, int* y) {
    const int e = (int)(smp % 3);
    const int e1 = (e + 1) % 3;
    const float ex = s3x[e1] - s3x[e];
    const float ey = s3y[e1] - s3y[e];
    const float len = sqrtf(ex * ex + ey * ey);
    if (len < 1e-6f) {
        return false;
    }
    const float u = hash_to_unit(f, smp, seed_u, 2);
    const float o = (hash_to_unit(f, smp, seed_u, 3) * 2.f - 1.f) * 2.f;
    *x = (int)floorf(s3x[e] + u * ex - o * (ey / len));
    *y = (int)floorf(s3y[e] + u * ey + o * (ex / len));
    return true;
}

// Screen triangle of a face for the vertex backward (c.xy / c.w form); false
// when a corner has w <= 1e-6.
__device__ __forceinline__ bool aa_face_screen(const float4 c[3], float W, float H, float s3x[3],
                                               float s3y[3]) {
    for (int k = 0; k < 3; k++) {
        if (c[k].w <= 1e-6f) {
            return false;
        }
        s3x[k] = (c[k].x / c[k].w * 0.5f + 0.5f) * W;
        s3y[k] = (c[k].y / c[k].w * 0.5f + 0.5f) * H;
    }
    return true;
}

}  // namespace dressi
