// dressi_math.h -- screen-space arithmetic shared by the HIP kernels.
//
// Every function reproduces the reference CPU kernel's float expression
// order exactly (the library is compiled with -ffp-contract=off and IEEE
// division/sqrt), so coverage, face ids and depth decisions are bit-identical
// to the reference. References are to the reference checkout.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dressi {

#define DRESSI_HD __host__ __device__ __forceinline__

constexpr float kWEps = 1e-6f;     // src/core/cpu_raster.cpp:21
constexpr float kDistEps = 1e-6f;  // src/core/cpu_raster.cpp:22

// std::min / std::max semantics (the reference's CPU kernels)
DRESSI_HD float smin(float a, float b) { return (b < a) ? b : a; }
DRESSI_HD float smax(float a, float b) { return (a < b) ? b : a; }
// F::Step(edge, x) (src/core/f_ops.cpp:530-537)
DRESSI_HD float step_f(float edge, float x) { return x < edge ? 0.f : 1.f; }
// uint32_t(int64_t(v + 0.5f)): the reference's float-id decode
DRESSI_HD uint32_t fid_u(float v) { return (uint32_t)(int64_t)(v + 0.5f); }

struct ScreenVert {
    float x, y, z, inv_w;
};

// cpu_raster.cpp:19-27 (ProjectToScreen)
DRESSI_HD ScreenVert project_to_screen(float cx, float cy, float cz, float cw,
                                       float w, float h) {
    const float inv_w = 1.f / cw;
    ScreenVert v;
    v.x = (cx * inv_w * 0.5f + 0.5f) * w;
    v.y = (cy * inv_w * 0.5f + 0.5f) * h;
    v.z = cz * inv_w;
    v.inv_w = inv_w;
    return v;
}

// cpu_raster.cpp:227-239 (ProjectClipToScreen) validity
DRESSI_HD bool clip_w_valid(float cw) { return !(fabsf(cw) <= kWEps || cw < 0.f); }

// cpu_raster.cpp:88-94: inclusive pixel bbox of a screen triangle
DRESSI_HD void pixel_bbox(float x0f, float x1f, float x2f, float y0f, float y1f,
                          float y2f, int w, int h, int* bx0, int* by0, int* bx1,
                          int* by1) {
    const float min_x = smin(smin(x0f, x1f), x2f);
    const float max_x = smax(smax(x0f, x1f), x2f);
    const float min_y = smin(smin(y0f, y1f), y2f);
    const float max_y = smax(smax(y0f, y1f), y2f);
    int a = (int)floorf(min_x - 0.5f);
    *bx0 = a > 0 ? a : 0;
    a = (int)ceilf(max_x - 0.5f);
    *bx1 = a < w - 1 ? a : w - 1;
    a = (int)floorf(min_y - 0.5f);
    *by0 = a > 0 ? a : 0;
    a = (int)ceilf(max_y - 0.5f);
    *by1 = a < h - 1 ? a : h - 1;
}

// cpu_raster.cpp:177-193 (ScreenBarycentric) split into its per-triangle
// part (area, 1/area) and per-pixel part; the values are identical to the
// one-call form.
DRESSI_HD float tri_area(float x0, float y0, float x1, float y1, float x2, float y2) {
    return (x1 - x0) * (y2 - y0) - (y1 - y0) * (x2 - x0);
}
DRESSI_HD void barycentric(float px, float py, float x0, float y0, float x1,
                           float y1, float x2, float y2, float inv_area,
                           float* l0, float* l1, float* l2) {
    *l0 = ((x1 - px) * (y2 - py) - (y1 - py) * (x2 - px)) * inv_area;
    *l1 = ((x2 - px) * (y0 - py) - (y2 - py) * (x0 - px)) * inv_area;
    *l2 = 1.f - *l0 - *l1;
}

// Per-triangle constants of SignedDistToTri (cpu_raster.cpp:114-151): edge
// k = (s[k], s[(k+1)%3]), e = b - a, len2 = |e|^2.
struct HardTri {
    float ax[3], ay[3], ex[3], ey[3], len2[3];
};

DRESSI_HD void hard_tri_init(HardTri* t, const float sx[3], const float sy[3]) {
    for (int k = 0; k < 3; k++) {
        const int k1 = (k + 1) % 3;
        t->ax[k] = sx[k];
        t->ay[k] = sy[k];
        t->ex[k] = sx[k1] - sx[k];
        t->ey[k] = sy[k1] - sy[k];
        t->len2[k] = t->ex[k] * t->ex[k] + t->ey[k] * t->ey[k];
    }
}

// cpu_raster.cpp:114-151 (SignedDistToTri): >= 0 inside (winding-agnostic)
DRESSI_HD float signed_dist(float px, float py, const float ax[3], const float ay[3],
                            const float ex[3], const float ey[3], const float len2[3]) {
    float best_d2 = -1.f;
    int n_pos = 0, n_neg = 0;
#pragma unroll
    for (int k = 0; k < 3; k++) {
        float t = 0.f;
        if (len2[k] > kDistEps * kDistEps) {
            t = ((px - ax[k]) * ex[k] + (py - ay[k]) * ey[k]) / len2[k];
            t = smin(smax(t, 0.f), 1.f);
        }
        const float qx = ax[k] + t * ex[k];
        const float qy = ay[k] + t * ey[k];
        const float dx = px - qx;
        const float dy = py - qy;
        const float d2 = dx * dx + dy * dy;
        if (best_d2 < 0.f || d2 < best_d2) {
            best_d2 = d2;
        }
        const float cr = ex[k] * (py - ay[k]) - ey[k] * (px - ax[k]);
        n_pos += (cr >= 0.f);
        n_neg += (cr <= 0.f);
    }
    const float sgn = (n_pos == 3 || n_neg == 3) ? 1.f : -1.f;
    return sgn * sqrtf(smax(best_d2, 0.f));
}

// cpu_raster.cpp:329-333: the Eq.3 depth shift
DRESSI_HD float eq3_depth(float dist, float hard_z, float radius) {
    return dist >= 0.f ? 0.5f * smin(smax(hard_z, 0.f), 1.f)
                       : 0.5f + 0.5f * smin(-dist / radius, 1.f);
}

// Sort key: depth (sign bit cleared so -0 == +0), then the larger face
// index -- the reference's LessOrEqual test in face order keeps the later
// face on ties (cpu_raster.cpp:101-104, 342-345).
DRESSI_HD uint64_t depth_key(float depth, uint32_t f) {
    union {
        float f;
        uint32_t u;
    } b;
    b.f = depth;
    return ((uint64_t)(b.u & 0x7fffffffu) << 32) | (uint64_t)(0xffffffffu - f);
}
constexpr uint64_t kEmptyKey = ~0ull;
DRESSI_HD uint32_t key_face(uint64_t key) { return 0xffffffffu - (uint32_t)(key & 0xffffffffu); }

// src/core/f_ops.cpp:1473-1487 (WangHash, HashToUnit)
DRESSI_HD uint32_t wang_hash(uint32_t x) {
    x = (x ^ 61u) ^ (x >> 16);
    x *= 9u;
    x ^= x >> 4;
    x *= 0x27d4eb2du;
    x ^= x >> 15;
    return x;
}
DRESSI_HD float hash_to_unit(uint32_t f, uint32_t s, uint32_t seed, uint32_t salt) {
    const uint32_t hh = wang_hash(f * 9781u ^ s * 6151u ^ seed * 26699u ^ salt * 42589u);
    return (float)(hh & 0xFFFFFFu) / 16777216.f;
}

// expf with the exact results of the host C library the reference evaluator
// calls (glibc's single-precision exp: Szabolcs Nagy's table-driven method,
// ARM optimized-routines math/expf.c): x * 32/ln2 = k + r, 2^(k/32) from a
// 32-entry table, 2^(r/32) by a cubic, all in double; the range reduction
// uses fused multiply-adds as the x86-64 FMA build of that routine does.
// The table holds asuint64(2^(i/32)) - (i << 47) (the correctly rounded
// doubles of 2^(i/32)); the cubic is that routine's published minimax fit.
// Checked against the host expf on every non-NaN float (identical).
__host__ __device__ __forceinline__ float libc_expf(float x) {
    constexpr uint64_t kTab[32] = {
            0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full,
            0x3fef9301d0125b51ull, 0x3fef72b83c7d517bull, 0x3fef54873168b9aaull,
            0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, 0x3fef06fe0a31b715ull,
            0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
            0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull,
            0x3feea47eb03a5585ull, 0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull,
            0x3feea11473eb0187ull, 0x3feea589994cce13ull, 0x3feeace5422aa0dbull,
            0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
            0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull,
            0x3fef3720dcef9069ull, 0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full,
            0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};
    constexpr double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / 32;
    constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32;
    constexpr double kShift = 0x1.8p+52;
    union {
        float f;
        uint32_t u;
    } xb;
    xb.f = x;
    const uint32_t abstop = (xb.u >> 20) & 0x7ff;
    if (abstop >= 0x42b) {  // |x| >= 88, inf, nan
        if (xb.u == 0xff800000u) {
            return 0.f;
        }
        if (abstop >= 0x7f8) {
            return x + x;
        }
        if (x > 0x1.62e42ep6f) {
            return __builtin_huge_valf();
        }
        if (x < -0x1.9fe368p6f) {
            return 0.f;
        }
    }
    const double xd = (double)x;
    union {
        double d;
        uint64_t u;
    } kb, sb;
    kb.d = fma(kInvLn2N, xd, kShift);
    const uint64_t ki = kb.u;
    const double kd = kb.d - kShift;
    const double r = fma(kInvLn2N, xd, -kd);
    sb.u = kTab[ki % 32] + (ki << 47);
    const double z = fma(kC0, r, kC1);
    const double r2 = r * r;
    double y = fma(kC2, r, 1.0);
    y = fma(z, r2, y);
    return (float)(y * sb.d);
}

// Clip transform, column-major MVP: acc = sum_k m[k*4+row] * p[k] with p[3]
// = 1 (examples/common/asset_utils.cpp:768-782; the graph form
// TransformToClipVar evaluates the same float sequence).
DRESSI_HD float4 mvp_transform(const float* m, float x, float y, float z) {
    float r[4];
#pragma unroll
    for (int row = 0; row < 4; row++) {
        float acc = 0.f;
        acc += m[0 * 4 + row] * x;
        acc += m[1 * 4 + row] * y;
        acc += m[2 * 4 + row] * z;
        acc += m[3 * 4 + row] * 1.f;
        r[row] = acc;
    }
    return make_float4(r[0], r[1], r[2], r[3]);
}

}  // namespace dressi
