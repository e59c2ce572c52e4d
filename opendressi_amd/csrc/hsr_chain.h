// hsr_chain.h -- the silhouette example's per-pixel image-space chain and its
// reverse-mode derivative, evaluated in registers.
//
// Forward (examples/silhouette_optimization/run.cpp:253-300, 320-342,
// 382-393) at a pixel covered by face f, from the face's three corner clips
// c_k (LookupFaces -> FaceFetch):
//   s_k   = ((c_k.xy / (c_k.w + 1 - mask)) * 0.5 + 0.5) * (W, H)
//   d_e   = |pc - (a + clamp(((pc-a).e) / (e.e + 1e-12), 0, 1) e)| (+1e-12 inside sqrt)
//   dist  = (2 * inside - 1) * min(min(d01, d12), d20)
//   D     = mask * sigmoid(dist * 7 / r)
//   pred  = max(cov * step(0, dist_raster), 1 - 1 * (1 - D))
//   loss  = (target - pred)^2 / (W * H)
// The backward applies each op's derivative in the order the reference's
// BuildBackward composes them (src/core/build_backward.cpp:62-149): gradient
// contributions of a variable are summed in descending node-creation order,
// which for the example's expressions (g++ evaluates call arguments right to
// left) is listed at each sum below. Every op is replayed with the same
// float operations and the sigmoid's exp is libc_expf, so the results are
// bit-identical to the reference evaluator's.
#pragma once

#include "dressi_math.h"

namespace dressi {

struct EdgeFw {
    float e[2], pa[2], num, den, q, t, dd[2], d;
};

__device__ __forceinline__ void edge_fw(float ax, float ay, float bx, float by, float pcx,
                                        float pcy, EdgeFw& r) {
    r.e[0] = bx - ax;
    r.e[1] = by - ay;
    r.pa[0] = pcx - ax;
    r.pa[1] = pcy - ay;
    r.num = r.pa[0] * r.e[0] + r.pa[1] * r.e[1];
    const float ee = r.e[0] * r.e[0] + r.e[1] * r.e[1];
    r.den = ee + 1e-12f;
    r.q = r.num / r.den;
    r.t = smin(smax(r.q, 0.f), 1.f);
    const float ate0 = ax + r.t * r.e[0];
    const float ate1 = ay + r.t * r.e[1];
    r.dd[0] = pcx - ate0;
    r.dd[1] = pcy - ate1;
    const float dd2 = r.dd[0] * r.dd[0] + r.dd[1] * r.dd[1];
    r.d = sqrtf(dd2 + 1e-12f);
}

// Edge backward: ga[0..2] = contributions to `a` in the order
// Add(a, t e), Sub(pc, a), Sub(b, a); gb = Sub(b, a)'s contribution to `b`.
__device__ __forceinline__ void edge_bw(const EdgeFw& r, float g_d, float ga[3][2],
                                        float gb[2]) {
    const float g_s = g_d * (0.5f / r.d);
    float g_ate[2];
#pragma unroll
    for (int c = 0; c < 2; c++) {
        const float A = g_s * r.dd[c];
        g_ate[c] = -(A + A);  // Dot(dd,dd) twice, then Sub(pc, ate)
    }
    const float g_t = g_ate[0] * r.e[0] + g_ate[1] * r.e[1];  // CompSum(g_te * e)
    const float g_q = g_t * (step_f(0.f, r.q) * step_f(r.q, 1.f));
    const float g_num = g_q / r.den;
    const float g_ee = -((g_q * r.num) / (r.den * r.den));
#pragma unroll
    for (int c = 0; c < 2; c++) {
        // e: Mul(t, e), Dot(pa, e), Dot(e, e) x2
        float acc = 0.f;
        acc += g_ate[c] * r.t;
        acc += g_num * r.pa[c];
        const float ce = g_ee * r.e[c];
        acc += ce;
        acc += ce;
        ga[0][c] = g_ate[c];
        ga[1][c] = -(g_num * r.e[c]);
        ga[2][c] = -acc;
        gb[c] = acc;
    }
}

struct PixelFw {
    float w[3], s[3][2];
    EdgeFw ed[3];  // (s0,s1), (s1,s2), (s2,s0)
    float m01, dmin, inside, sig, soft_sil, hard, pred;
};

// The chain's screen corners of a face: s_k = ((c_k.xy / (c_k.w + 1 - mask))
// * 0.5 + 0.5) * (W, H) with mask = 1 (the face covers the pixel).
__device__ __forceinline__ void chain_screen(const float4 c[3], float W, float H,
                                             float s[3][2]) {
#pragma unroll
    for (int k = 0; k < 3; k++) {
        const float w = c[k].w + 0.f;
        s[k][0] = ((c[k].x / w) * 0.5f + 0.5f) * W;
        s[k][1] = ((c[k].y / w) * 0.5f + 0.5f) * H;
    }
}

// Forward of the chain from the screen corners st.s at pixel centre
// (pcx, pcy); `mask` / `cov` are 1 on covered pixels, `dist_c` is the
// rasterizer's signed distance channel.
__device__ __forceinline__ void pixel_fw_screen(float mask, float dist_c, float cov, float pcx,
                                                float pcy, float sigma_scale, PixelFw& st) {
    edge_fw(st.s[0][0], st.s[0][1], st.s[1][0], st.s[1][1], pcx, pcy, st.ed[0]);
    edge_fw(st.s[1][0], st.s[1][1], st.s[2][0], st.s[2][1], pcx, pcy, st.ed[1]);
    edge_fw(st.s[2][0], st.s[2][1], st.s[0][0], st.s[0][1], pcx, pcy, st.ed[2]);
    st.m01 = smin(st.ed[0].d, st.ed[1].d);
    st.dmin = smin(st.m01, st.ed[2].d);
    float sp = 1.f, sn = 1.f;
#pragma unroll
    for (int k = 0; k < 3; k++) {
        const int k1 = (k + 1) % 3;
        const float ex = st.s[k1][0] - st.s[k][0];
        const float ey = st.s[k1][1] - st.s[k][1];
        const float cr = ex * (pcy - st.s[k][1]) - ey * (pcx - st.s[k][0]);
        sp = k == 0 ? step_f(0.f, cr) : sp * step_f(0.f, cr);
        sn = k == 0 ? step_f(0.f, -cr) : sn * step_f(0.f, -cr);
    }
    st.inside = smin(sp + sn, 1.f);
    const float dist = (st.inside * 2.f - 1.f) * st.dmin;
    st.sig = 1.f / (1.f + libc_expf(-(dist * sigma_scale)));
    const float D = mask * st.sig;
    st.soft_sil = 1.f - 1.f * (1.f - D);
    st.hard = cov * step_f(0.f, dist_c);
    st.pred = smax(st.hard, st.soft_sil);
}

// Forward of the chain at pixel centre (pcx, pcy) from the three fetched
// corner clips.
__device__ __forceinline__ void pixel_fw(const float4 c[3], float mask, float dist_c, float cov,
                                         float pcx, float pcy, float W, float H,
                                         float sigma_scale, PixelFw& st) {
    const float om = 1.f - mask;
#pragma unroll
    for (int k = 0; k < 3; k++) {
        st.w[k] = c[k].w + om;
        st.s[k][0] = ((c[k].x / st.w[k]) * 0.5f + 0.5f) * W;
        st.s[k][1] = ((c[k].y / st.w[k]) * 0.5f + 0.5f) * H;
    }
    pixel_fw_screen(mask, dist_c, cov, pcx, pcy, sigma_scale, st);
}

// Gradient of (target - pred)^2 * inv_px w.r.t. the three fetched corner
// clips (x, y, z = 0, w).
__device__ __forceinline__ void pixel_bw(const PixelFw& st, const float4 c[3], float mask,
                                         float target, float inv_px, float W, float H,
                                         float sigma_scale, float4 g[3]) {
    const float cd = inv_px * (target - st.pred);
    const float g_pred = -(cd + cd);
    const float g_soft = g_pred * (1.f - step_f(st.soft_sil, st.hard));
    const float g_D = -((-g_soft) * 1.f);
    const float g_sig = g_D * mask;
    const float g_z = g_sig * (st.sig * (1.f - st.sig));
    const float g_dmin = (g_z * sigma_scale) * (st.inside * 2.f - 1.f);
    const float mk1 = step_f(st.m01, st.ed[2].d);
    const float g_m01 = g_dmin * mk1;
    const float g_d20 = g_dmin * (1.f - mk1);
    const float mk2 = step_f(st.ed[0].d, st.ed[1].d);
    const float g_d01 = g_m01 * mk2;
    const float g_d12 = g_m01 * (1.f - mk2);
    float ga01[3][2], gb01[2], ga12[3][2], gb12[2], ga20[3][2], gb20[2];
    edge_bw(st.ed[0], g_d01, ga01, gb01);
    edge_bw(st.ed[1], g_d12, ga12, gb12);
    edge_bw(st.ed[2], g_d20, ga20, gb20);
    // s_k sums: edge_dist nodes were created (s2,s0), (s1,s2), (s0,s1), so
    // (s0,s1)'s consumers come first in each 4-term sum.
    float gs[3][2];
#pragma unroll
    for (int q = 0; q < 2; q++) {
        float a0 = 0.f;
        a0 += ga01[0][q];
        a0 += ga01[1][q];
        a0 += ga01[2][q];
        a0 += gb20[q];
        gs[0][q] = a0;
        float a1 = 0.f;
        a1 += gb01[q];
        a1 += ga12[0][q];
        a1 += ga12[1][q];
        a1 += ga12[2][q];
        gs[1][q] = a1;
        float a2 = 0.f;
        a2 += gb12[q];
        a2 += ga20[0][q];
        a2 += ga20[1][q];
        a2 += ga20[2][q];
        gs[2][q] = a2;
    }
#pragma unroll
    for (int k = 0; k < 3; k++) {
        const float g_xw = (gs[k][0] * W) * 0.5f;
        const float g_yw = (gs[k][1] * H) * 0.5f;
        const float wk = st.w[k];
        const float gw_x = -((g_xw * c[k].x) / (wk * wk));
        const float gw_y = -((g_yw * c[k].y) / (wk * wk));
        g[k] = make_float4(g_xw / wk, g_yw / wk, 0.f, gw_y + gw_x);
    }
}

}  // namespace dressi
