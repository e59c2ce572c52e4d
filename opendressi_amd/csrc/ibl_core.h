// ibl_core.h -- device and host helpers of the split-sum IBL path: the
// equirect mapping, bilinear taps, the GGX convolution weight and the
// Hammersley / GGX sample tables (src/core/ibl_math.h).
//
// Texel-centre directions and the sample angles are built on the host with
// the C library's sinf / cosf, exactly as the reference's CPU code evaluates
// them: the roughness-0 prefilter kernel turns a one-ulp change of a
// direction into a ~1e-2 change of its peak weight, so these tables must be
// the reference's bits. Per-pixel directions (normals, reflections, view
// rays) are mapped to uv on the device with atan2f / acosf that return what
// the host C library returns (libm_f32.h).
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <vector>

#include "libm_f32.h"

namespace dressi {

constexpr float kIblPi = 3.14159265358979323846f;
constexpr float kIblTwoPi = 6.28318530717958647692f;
constexpr float kIblInvPi = 0.31830988618379067154f;
constexpr float kIblInvTwoPi = 0.15915494309189533577f;

// Texel-centre direction + sin(theta) of an equirect {w,h} map, row major:
// DirFromEquirectUv((x + .5) / w, (y + .5) / h) (ibl_math.h:48-54); .w is
// sin(v pi), the area term of the convolutions (f_ops.cpp:2983-2984).
inline std::vector<float4> host_equirect_dirs(uint32_t w, uint32_t h) {
    std::vector<float4> out((size_t)w * h);
    for (uint32_t y = 0; y < h; y++) {
        const float v = ((float)y + 0.5f) / (float)h;
        const float theta = v * kIblPi;
        const float st = sinf(theta);
        const float ct = cosf(theta);
        for (uint32_t x = 0; x < w; x++) {
            const float u = ((float)x + 0.5f) / (float)w;
            const float phi = (u - 0.5f) * kIblTwoPi;
            out[(size_t)y * w + x] = make_float4(st * cosf(phi), ct, st * sinf(phi), st);
        }
    }
    return out;
}

// Van der Corput radical inverse (ibl_math.h:119-128)
__host__ __device__ inline float radical_inverse(uint32_t bits) {
    bits = (bits << 16u) | (bits >> 16u);
    bits = ((bits & 0x55555555u) << 1u) | ((bits & 0xAAAAAAAAu) >> 1u);
    bits = ((bits & 0x33333333u) << 2u) | ((bits & 0xCCCCCCCCu) >> 2u);
    bits = ((bits & 0x0F0F0F0Fu) << 4u) | ((bits & 0xF0F0F0F0u) >> 4u);
    bits = ((bits & 0x00FF00FFu) << 8u) | ((bits & 0xFF00FF00u) >> 8u);
    return (float)bits * 2.3283064365386963e-10f;
}

// Per Hammersley sample i of n: (cos phi, sin phi, xi1) with phi = 2 pi i / n
// (ibl_math.h:130-141)
inline std::vector<float4> host_hammersley(uint32_t n) {
    std::vector<float4> out(n);
    for (uint32_t i = 0; i < n; i++) {
        const float xi0 = (float)i / (float)n;
        const float phi = kIblTwoPi * xi0;
        out[i] = make_float4(cosf(phi), sinf(phi), radical_inverse(i), 0.f);
    }
    return out;
}

struct V3f {
    float x, y, z;
};

__device__ __forceinline__ V3f mk3(float x, float y, float z) { return V3f{x, y, z}; }
__device__ __forceinline__ float dot3(V3f a, V3f b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
__device__ __forceinline__ V3f cross3(V3f a, V3f b) {
    return V3f{a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x};
}
__device__ __forceinline__ V3f normalize3(V3f v) {
    const float len = sqrtf(dot3(v, v));
    return V3f{v.x / len, v.y / len, v.z / len};
}

// EquirectUvFromDir (ibl_math.h:41-46) for a unit direction
__device__ __forceinline__ void equirect_uv(V3f d, float* u, float* v) {
    const float y = d.y < -1.f ? -1.f : (d.y > 1.f ? 1.f : d.y);
    *u = libm::atan2f(d.z, d.x) * kIblInvTwoPi + 0.5f;
    *v = libm::acosf(y) * kIblInvPi;
}

// EquirectSample's direction handling (f_ops.cpp:2946-2958): false for a
// zero-length direction (sample 0), else the uv of the normalised direction
__device__ __forceinline__ bool dir_to_equirect(V3f d, float* u, float* v) {
    const float dlen = sqrtf(dot3(d, d));
    if (dlen < 1e-8f) {
        return false;
    }
    equirect_uv(V3f{d.x / dlen, d.y / dlen, d.z / dlen}, u, v);
    return true;
}

// One bilinear tap set: texel indices and weights in the reference's tap
// order (dy outer, dx inner), u wrapping, v clamped (BilerpWrap,
// ibl_math.h:58-89) or both clamped (BilerpClamp, :92-115).
struct Taps {
    int idx[4];
    float w[4];
};

__device__ __forceinline__ Taps taps_wrap(int w, int h, float u, float v) {
    const float sx = u * (float)w - 0.5f;
    const float sy = v * (float)h - 0.5f;
    const int ix = (int)floorf(sx);
    const int iy = (int)floorf(sy);
    const float fx = sx - (float)ix;
    const float fy = sy - (float)iy;
    Taps t;
#pragma unroll
    for (int dy = 0; dy <= 1; dy++) {
#pragma unroll
        for (int dx = 0; dx <= 1; dx++) {
            int x = ix + dx;
            if (x < 0) x += w;
            if (x >= w) x -= w;
            int y = iy + dy;
            y = y < 0 ? 0 : (y > h - 1 ? h - 1 : y);
            t.idx[dy * 2 + dx] = y * w + x;
            t.w[dy * 2 + dx] = (dx == 0 ? 1.f - fx : fx) * (dy == 0 ? 1.f - fy : fy);
        }
    }
    return t;
}

__device__ __forceinline__ Taps taps_clamp(int w, int h, float u, float v) {
    const float sx = u * (float)w - 0.5f;
    const float sy = v * (float)h - 0.5f;
    const int ix = (int)floorf(sx);
    const int iy = (int)floorf(sy);
    const float fx = sx - (float)ix;
    const float fy = sy - (float)iy;
    Taps t;
#pragma unroll
    for (int dy = 0; dy <= 1; dy++) {
#pragma unroll
        for (int dx = 0; dx <= 1; dx++) {
            int x = ix + dx;
            x = x < 0 ? 0 : (x > w - 1 ? w - 1 : x);
            int y = iy + dy;
            y = y < 0 ? 0 : (y > h - 1 ? h - 1 : y);
            t.idx[dy * 2 + dx] = y * w + x;
            t.w[dy * 2 + dx] = (dx == 0 ? 1.f - fx : fx) * (dy == 0 ? 1.f - fy : fy);
        }
    }
    return t;
}

// out[c] = sum over taps in order of w * data[idx * n + c], from 0
__device__ __forceinline__ void taps_fetch(const Taps& t, const float* data, uint32_t n,
                                           float* out) {
    for (uint32_t c = 0; c < n; c++) {
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            acc += t.w[k] * data[(size_t)t.idx[k] * n + c];
        }
        out[c] = acc;
    }
}

// GgxConvWeight (ibl_math.h:162-170)
__device__ __forceinline__ float ggx_conv_weight(float c, float alpha) {
    if (c <= 0.f) {
        return 0.f;
    }
    const float ch2 = (1.f + c) * 0.5f;
    const float a2 = alpha * alpha;
    const float d = ch2 * (a2 - 1.f) + 1.f;
    return a2 / (kIblPi * d * d) * c;
}

// Schlick-GGX G1 (ibl_math.h:153-156)
__device__ __forceinline__ float g1_ibl(float n_dot_x, float k) {
    return n_dot_x / (n_dot_x * (1.f - k) + k);
}

// ImportanceSampleGGX (ibl_math.h:134-150) from a sample-table entry
// (cos phi, sin phi, xi1)
__device__ __forceinline__ V3f importance_sample_ggx(float4 smp, float roughness, V3f n) {
    const float a = roughness * roughness;
    const float xi1 = smp.z;
    const float ct = sqrtf((1.f - xi1) / (1.f + (a * a - 1.f) * xi1));
    const float st0 = 1.f - ct * ct;
    const float st = sqrtf(st0 > 0.f ? st0 : 0.f);
    const V3f h_t = V3f{smp.x * st, smp.y * st, ct};
    const V3f up = fabsf(n.z) < 0.999f ? V3f{0.f, 0.f, 1.f} : V3f{1.f, 0.f, 0.f};
    const V3f tx = normalize3(cross3(up, n));
    const V3f ty = cross3(n, tx);
    return normalize3(V3f{tx.x * h_t.x + ty.x * h_t.y + n.x * h_t.z,
                          tx.y * h_t.x + ty.y * h_t.y + n.y * h_t.z,
                          tx.z * h_t.x + ty.z * h_t.y + n.z * h_t.z});
}

}  // namespace dressi
