// libm_f32.h -- single-precision atan, atan2 and acos that return, for every
// argument, what the host C library returns (glibc 2.35 on x86-64, whose
// float versions are the fdlibm ones).
//
// The reference evaluates its equirect mapping (src/core/ibl_math.h:41-47,
// EquirectUvFromDir) with std::atan2(float, float) and std::acos(float),
// i.e. the C library's atan2f / acosf, which are not correctly rounded: a
// correctly rounded device version differs from them by one ulp on a few
// percent of inputs, and one ulp of a direction's uv moves a bilinear tap
// weight. These functions restate the published algorithm of those C library
// routines -- Sun Microsystems' fdlibm 5.3 s_atan.c / e_atan2.c / e_acos.c in
// their single-precision form (argument reduction against atan(0.5), atan(1),
// atan(1.5) and infinity with hi/lo splits and an 11-term odd/even polynomial
// for atan; the quadrant rules of atan2; the rational approximation
// R(z) = P(z) / Q(z) of (asin(x) - x) / x^3 with the sqrt-based reflection
// and the split of sqrt(z) into a 12-bit head and a correction for acos).
// The coefficients are fdlibm's, given by their bit patterns.
//
// Checked against the host library: acosf on every float in [-1, 1], atanf
// and atan2f on random and structured arguments (tests/test_abi.py builds
// and runs the check on the CPU; tests/test_gpu_pbr.py runs the device
// versions against the host's outputs).
//
// Every operation is one IEEE single-precision rounding: the library is
// built with -ffp-contract=off and correctly rounded division and sqrt.
#ifndef DRESSI_LIBM_F32_H
#define DRESSI_LIBM_F32_H

#include <hip/hip_runtime.h>

#include <cstdint>

#include "libm_pow5_table.h"

namespace dressi {
namespace libm {

__host__ __device__ inline uint32_t fbits(float x) { return __builtin_bit_cast(uint32_t, x); }
__host__ __device__ inline float bitsf(uint32_t u) { return __builtin_bit_cast(float, u); }

// atan(x): |x| reduced to [0, 7/16) directly or around 0.5, 1, 1.5 and
// infinity (atan(t) = atan(c) + atan((t - c) / (1 + c t))), then the
// polynomial x - x (s1 + s2) in z = x^2 split into odd and even parts.
__host__ __device__ inline float atanf(float x) {
    const uint32_t hx = fbits(x);
    const uint32_t ix = hx & 0x7fffffffu;
    if (ix >= 0x4c000000u) {  // |x| >= 2^25 (or NaN): atan(x) rounds to pi / 2
        if (ix > 0x7f800000u) {
            return x + x;
        }
        const float r = bitsf(0x3fc90fdau) + bitsf(0x33a22168u);
        return (hx >> 31) ? -r : r;
    }
    int id;
    if (ix < 0x3ee00000u) {  // |x| < 0.4375
        if (ix < 0x31000000u) {  // |x| < 2^-29: atan(x) rounds to x
            return x;
        }
        id = -1;
    } else {
        x = x < 0.f ? -x : x;
        if (ix < 0x3f980000u) {      // |x| < 1.1875
            if (ix < 0x3f300000u) {  // 7/16 <= |x| < 11/16
                id = 0;
                x = (2.f * x - 1.f) / (2.f + x);
            } else {  // 11/16 <= |x| < 19/16
                id = 1;
                x = (x - 1.f) / (x + 1.f);
            }
        } else {
            if (ix < 0x401c0000u) {  // |x| < 2.4375
                id = 2;
                x = (x - 1.5f) / (1.f + 1.5f * x);
            } else {  // 2.4375 <= |x| < 2^25
                id = 3;
                x = -1.f / x;
            }
        }
    }
    const float a0 = bitsf(0x3eaaaaabu), a1 = bitsf(0xbe4ccccdu), a2 = bitsf(0x3e124925u),
                a3 = bitsf(0xbde38e38u), a4 = bitsf(0x3dba2e6eu), a5 = bitsf(0xbd9d8795u),
                a6 = bitsf(0x3d886b35u), a7 = bitsf(0xbd6ef16bu), a8 = bitsf(0x3d4bda59u),
                a9 = bitsf(0xbd15a221u), a10 = bitsf(0x3c8569d7u);
    const float z = x * x;
    const float w = z * z;
    const float s1 = z * (a0 + w * (a2 + w * (a4 + w * (a6 + w * (a8 + w * a10)))));
    const float s2 = w * (a1 + w * (a3 + w * (a5 + w * (a7 + w * a9))));
    if (id < 0) {
        return x - x * (s1 + s2);
    }
    // atan(c) split into a head and a tail for c = 0.5, 1, 1.5, infinity
    const uint32_t hi_bits[4] = {0x3eed6338u, 0x3f490fdau, 0x3f7b985eu, 0x3fc90fdau};
    const uint32_t lo_bits[4] = {0x31ac3769u, 0x33222168u, 0x33140fb4u, 0x33a22168u};
    const float r = bitsf(hi_bits[id]) - ((x * (s1 + s2) - bitsf(lo_bits[id])) - x);
    return (hx >> 31) ? -r : r;
}

// atan2(y, x): the quadrant rules around atan(|y / x|), with pi split into a
// float head and tail.
__host__ __device__ inline float atan2f(float y, float x) {
    const float pi_o_4 = bitsf(0x3f490fdbu), pi_o_2 = bitsf(0x3fc90fdbu);
    const float pi = bitsf(0x40490fdbu), pi_lo = bitsf(0xb3bbbd2eu);
    const uint32_t hx = fbits(x), hy = fbits(y);
    const uint32_t ix = hx & 0x7fffffffu, iy = hy & 0x7fffffffu;
    if (ix > 0x7f800000u || iy > 0x7f800000u) {  // NaN
        return x + y;
    }
    if (hx == 0x3f800000u) {  // x = 1
        return atanf(y);
    }
    const int m = (int)((hy >> 31) & 1u) | (int)((hx >> 30) & 2u);  // 2 sign(x) + sign(y)
    if (iy == 0) {
        switch (m) {
            case 0:
            case 1:
                return y;
            case 2:
                return pi;
            default:
                return -pi;
        }
    }
    if (ix == 0) {
        return (hy >> 31) ? -pi_o_2 : pi_o_2;
    }
    if (ix == 0x7f800000u) {
        if (iy == 0x7f800000u) {
            switch (m) {
                case 0:
                    return pi_o_4;
                case 1:
                    return -pi_o_4;
                case 2:
                    return 3.f * pi_o_4;
                default:
                    return -3.f * pi_o_4;
            }
        }
        switch (m) {
            case 0:
                return 0.f;
            case 1:
                return -0.f;
            case 2:
                return pi;
            default:
                return -pi;
        }
    }
    if (iy == 0x7f800000u) {
        return (hy >> 31) ? -pi_o_2 : pi_o_2;
    }
    const int k = ((int)iy - (int)ix) >> 23;
    float z;
    if (k > 26) {  // |y / x| > 2^26
        z = pi_o_2 + 0.5f * pi_lo;
    } else if ((hx >> 31) && k < -26) {  // |y| / x < -2^26
        z = 0.f;
    } else {
        z = atanf(bitsf(fbits(y / x) & 0x7fffffffu));
    }
    switch (m) {
        case 0:
            return z;
        case 1:
            return -z;
        case 2:
            return pi - (z - pi_lo);
        default:
            return (z - pi_lo) - pi;
    }
}

// acos(x): |x| < 0.5 from pi/2 - (x + x R(x^2)); otherwise through
// z = (1 - |x|) / 2 and s = sqrt(z): x > 0 as 2 (s + s R(z)) with s split into
// a 12-bit head df and the correction c = (z - df^2) / (s + df); x < 0 as
// pi - 2 (s + s R(z)).
__host__ __device__ inline float acosf(float x) {
    const float pi = bitsf(0x40490fdau), pio2_hi = bitsf(0x3fc90fdau),
                pio2_lo = bitsf(0x33a22168u);
    const float pS0 = bitsf(0x3e2aaaabu), pS1 = bitsf(0xbea6b090u), pS2 = bitsf(0x3e4e0aa8u),
                pS3 = bitsf(0xbd241146u), pS4 = bitsf(0x3a4f7f04u), pS5 = bitsf(0x3811ef08u);
    const float qS1 = bitsf(0xc019d139u), qS2 = bitsf(0x4001572du), qS3 = bitsf(0xbf303361u),
                qS4 = bitsf(0x3d9dc62eu);
    const uint32_t hx = fbits(x);
    const uint32_t ix = hx & 0x7fffffffu;
    if (ix == 0x3f800000u) {  // |x| = 1
        return (hx >> 31) ? pi + 2.f * pio2_lo : 0.f;
    }
    if (ix > 0x3f800000u) {  // |x| > 1 or NaN
        return (x - x) / (x - x);
    }
    if (ix < 0x3f000000u) {  // |x| < 0.5
        if (ix <= 0x23000000u) {  // |x| <= 2^-57
            return pio2_hi + pio2_lo;
        }
        const float z = x * x;
        const float p = z * (pS0 + z * (pS1 + z * (pS2 + z * (pS3 + z * (pS4 + z * pS5)))));
        const float q = 1.f + z * (qS1 + z * (qS2 + z * (qS3 + z * qS4)));
        const float r = p / q;
        return pio2_hi - (x - (pio2_lo - x * r));
    }
    if (hx >> 31) {  // x <= -0.5
        const float z = (1.f + x) * 0.5f;
        const float p = z * (pS0 + z * (pS1 + z * (pS2 + z * (pS3 + z * (pS4 + z * pS5)))));
        const float q = 1.f + z * (qS1 + z * (qS2 + z * (qS3 + z * qS4)));
        const float s = __builtin_sqrtf(z);
        const float r = p / q;
        const float w = r * s - pio2_lo;
        return pi - 2.f * (s + w);
    }
    // x >= 0.5
    const float z = (1.f - x) * 0.5f;
    const float s = __builtin_sqrtf(z);
    const float df = bitsf(fbits(s) & 0xfffff000u);
    const float c = (z - df * df) / (s + df);
    const float p = z * (pS0 + z * (pS1 + z * (pS2 + z * (pS3 + z * (pS4 + z * pS5)))));
    const float q = 1.f + z * (qS1 + z * (qS2 + z * (qS3 + z * qS4)));
    const float r = p / q;
    const float w = r * s + c;
    return 2.f * (df + w);
}

namespace detail {

// a * b as a 128-bit (hi, lo) pair
__host__ __device__ inline void mul_64x64(uint64_t a, uint64_t b, uint64_t* hi, uint64_t* lo) {
    const uint64_t a0 = a & 0xffffffffu, a1 = a >> 32, b0 = b & 0xffffffffu, b1 = b >> 32;
    const uint64_t p00 = a0 * b0, p01 = a0 * b1, p10 = a1 * b0, p11 = a1 * b1;
    const uint64_t mid = (p00 >> 32) + (p01 & 0xffffffffu) + (p10 & 0xffffffffu);
    *lo = (p00 & 0xffffffffu) | (mid << 32);
    *hi = p11 + (p01 >> 32) + (p10 >> 32) + (mid >> 32);
}

}  // namespace detail

// powf(x, 5.0f) as the host C library returns it, for x = 0 and x in
// [2^-25, 1] (the Schlick factors (1 - cos)^5 of the PBR shading and its BRDF
// LUT; cosines of at most 1 in float give 0 or at least 2^-24). The C library
// evaluates exp2(5 log2 x) in double and rounds once; here x^5 is formed
// exactly (the 24-bit mantissa's 120-bit fifth power), rounded to nearest
// even, and moved by one ulp where the library's result is the other
// neighbour (kPow5Miss, generated from the library's outputs on every float
// of the domain). Below 2^-25 the correctly rounded x^5 is returned.
__host__ __device__ inline float pow5f(float x) {
    const uint32_t u = fbits(x);
    if ((u & 0x7fffffffu) == 0) {
        return x;
    }
    if (u >= 0x3f800000u || u < 0x33000000u) {
        // x = 1 (exact) and arguments outside the table's domain
        const double d = (double)x;
        return (float)(d * d * d * d * d);
    }
    const int e = (int)((u >> 23) & 0xffu);
    const uint64_t m = (u & 0x7fffffu) | 0x800000u;
    uint64_t hi, lo;
    detail::mul_64x64(m * m, m * m, &hi, &lo);  // m^4 < 2^96
    uint64_t h1, l1;
    detail::mul_64x64(lo, m, &h1, &l1);
    hi = hi * m + h1;  // m^5 = hi:l1 < 2^120
    lo = l1;
    // msb of m^5 is bit 115 + c, c in 0..4; keep 24 bits
    const int msb = 64 + (63 - __builtin_clzll(hi));
    const int sh = msb - 23;  // > 64
    uint64_t q = hi >> (sh - 64);
    const uint64_t rem_hi = hi & ((1ull << (sh - 64)) - 1ull);
    const uint64_t half_hi = 1ull << (sh - 65);
    if (rem_hi > half_hi || (rem_hi == half_hi && (lo != 0 || (q & 1)))) {
        q++;
    }
    // q in [2^23, 2^24]; x^5 = q * 2^(sh + 5 (e - 150))
    const int ex = sh + 5 * (e - 150) + 23;  // exponent of q's leading bit when q < 2^24
    uint32_t r;
    if (q == (1ull << 24)) {
        r = (uint32_t)(ex + 1 + 127) << 23;
    } else {
        r = ((uint32_t)(ex + 127) << 23) | (uint32_t)(q & 0x7fffffu);
    }
    // binary search of the miss table for this mantissa
    const uint32_t key = (u & 0x7fffffu) << 1;
    uint32_t lo_i = 0, hi_i = kPow5MissCount;
    while (lo_i < hi_i) {
        const uint32_t mid = (lo_i + hi_i) >> 1;
        if (kPow5Miss[mid][0] < key) {
            lo_i = mid + 1;
        } else {
            hi_i = mid;
        }
    }
    const uint32_t bit = 1u << (e - 102);
    for (uint32_t i = lo_i; i < kPow5MissCount && (kPow5Miss[i][0] >> 1) == (key >> 1); i++) {
        if (kPow5Miss[i][1] & bit) {
            r = (kPow5Miss[i][0] & 1u) ? r + 1u : r - 1u;
        }
    }
    return bitsf(r);
}

}  // namespace libm
}  // namespace dressi

#endif  // DRESSI_LIBM_F32_H
