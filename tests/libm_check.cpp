// libm_check.cpp -- the library's single-precision atanf / atan2f / acosf /
// pow5f (opendressi_amd/csrc/libm_f32.h, compiled here for the host) against
// the host C library, bit for bit:
//   acosf   every 3rd float of [-1, 1] (all of them with stride 1)
//   atanf   every 7th finite float (all of them with stride 1)
//   atan2f  random pairs of unit-vector components, random bit patterns,
//           and quotients around the 2^26 cut-offs
//   pow5f   every float of [2^-25, 1] with stride 3, every mantissa of its
//           miss table in every binade, and 0
//   libm_check [stride]      prints the mismatch counts, exits 1 on any
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>

#include "../opendressi_amd/csrc/libm_f32.h"

namespace {

float bf(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

uint32_t fb(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

uint64_t g_bad = 0;

void check(const char* what, float want, float got, float a, float b = 0.f) {
    if (fb(want) != fb(got)) {
        if (g_bad < 8) {
            printf("%s(%a, %a): C library %a, libm_f32 %a\n", what, a, b, want, got);
        }
        g_bad++;
    }
}

}  // namespace

int main(int argc, char** argv) {
    const uint64_t stride = argc > 1 ? strtoull(argv[1], nullptr, 10) : 1;
    uint64_t n = 0;
    for (uint64_t u = 0; u <= 0xffffffffull; u += stride * 3) {
        const float x = bf((uint32_t)u);
        if (std::fabs(x) <= 1.f) {
            check("acosf", ::acosf(x), dressi::libm::acosf(x), x);
            n++;
        }
    }
    for (float x : {1.f, -1.f, 0.5f, -0.5f, 0.f, -0.f}) {
        check("acosf", ::acosf(x), dressi::libm::acosf(x), x);
    }
    printf("acosf: %llu arguments\n", (unsigned long long)n);
    n = 0;
    for (uint64_t u = 0; u <= 0xffffffffull; u += stride * 7) {
        const float x = bf((uint32_t)u);
        if (!std::isnan(x)) {
            check("atanf", ::atanf(x), dressi::libm::atanf(x), x);
            n++;
        }
    }
    printf("atanf: %llu arguments\n", (unsigned long long)n);
    std::mt19937_64 rng(12345);
    std::uniform_real_distribution<float> unit(-1.f, 1.f);
    std::normal_distribution<float> gauss(0.f, 1.f);
    n = 0;
    for (uint64_t i = 0; i < 30000000ull / stride; i++) {
        float y, x;
        switch (i % 4) {
            case 0: {  // the (z, x) components of a normalised direction
                const float a = gauss(rng), b = gauss(rng), c = gauss(rng);
                const float len = std::sqrt(a * a + b * b + c * c);
                y = c / len;
                x = a / len;
                break;
            }
            case 1:
                y = unit(rng);
                x = unit(rng);
                break;
            case 2:
                y = bf((uint32_t)rng());
                x = bf((uint32_t)rng());
                break;
            default: {  // |y / x| near 2^+-26
                x = unit(rng);
                const int k = (int)(rng() % 9) + 22;
                y = std::ldexp(unit(rng), (rng() & 1) ? k : -k) * (x == 0.f ? 1.f : x);
                break;
            }
        }
        if (std::isnan(x) || std::isnan(y)) {
            continue;
        }
        check("atan2f", ::atan2f(y, x), dressi::libm::atan2f(y, x), y, x);
        n++;
    }
    const float sp[] = {0.f, -0.f, 1.f, -1.f, INFINITY, -INFINITY, 1e-30f, -1e-30f};
    for (float y : sp) {
        for (float x : sp) {
            check("atan2f", ::atan2f(y, x), dressi::libm::atan2f(y, x), y, x);
        }
    }
    printf("atan2f: %llu argument pairs\n", (unsigned long long)n);
    n = 0;
    for (uint64_t u = 0x33000000u; u <= 0x3f800000u; u += stride * 3) {
        const float x = bf((uint32_t)u);
        check("pow5f", ::powf(x, 5.f), dressi::libm::pow5f(x), x);
        n++;
    }
    for (uint32_t i = 0; i < dressi::libm::kPow5MissCount; i++) {
        const uint32_t m = dressi::libm::kPow5Miss[i][0] >> 1;
        for (uint32_t e = 102; e <= 126; e++) {
            const float x = bf((e << 23) | m);
            check("pow5f", ::powf(x, 5.f), dressi::libm::pow5f(x), x);
            n++;
        }
    }
    check("pow5f", ::powf(0.f, 5.f), dressi::libm::pow5f(0.f), 0.f);
    printf("pow5f: %llu arguments\n", (unsigned long long)n);
    printf("mismatches: %llu\n", (unsigned long long)g_bad);
    return g_bad ? 1 : 0;
}
