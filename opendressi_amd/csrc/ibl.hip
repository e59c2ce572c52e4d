// ibl.hip -- the split-sum IBL ops as per-op entry points (reference
// layouts): EquirectSample and its map VJP, AvgPool2x2 and its VJP,
// IrradianceConv / PrefilterConv and their transposes, PrefilterEnv and
// BrdfIntegrationLut (src/core/f_ops.cpp:2785-3415, src/core/ibl_math.h).
//
// The dense convolutions run one thread per output texel over the source
// texels in the reference's loop order, so with the reference's direction
// tables (ibl_core.h) their sums are the reference's bit for bit. The map
// VJP of EquirectSample scatters in 64-bit fixed point (exact, so the
// result does not depend on the order of the atomics).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <vector>

#include "dressi_hip.h"
#include "ibl_core.h"
#include "internal.h"

namespace dressi {
namespace {

// ---------------------------------------------------------------------------
// EquirectSample
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void k_eq_sample(const float* map, int mw, int mh, uint32_t n,
                                                   const float* dir, size_t npx, float* out) {
    const size_t p = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= npx) {
        return;
    }
    float u, v;
    float res[4] = {0.f, 0.f, 0.f, 0.f};
    if (dir_to_equirect(mk3(dir[p * 3 + 0], dir[p * 3 + 1], dir[p * 3 + 2]), &u, &v)) {
        taps_fetch(taps_wrap(mw, mh, u, v), map, n, res);
    }
    for (uint32_t c = 0; c < n; c++) {
        out[p * n + c] = res[c];
    }
}

// max |gy| as float bits (non-negative floats order like their bits)
__global__ __launch_bounds__(256) void k_max_abs(const float* x, size_t count, uint32_t* out) {
    uint32_t m = 0;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (size_t)gridDim.x * blockDim.x) {
        const uint32_t b = __float_as_uint(fabsf(x[i]));
        m = b > m && b < 0x7f800000u ? b : m;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const uint32_t other = (uint32_t)__shfl_xor((int)m, o);
        m = other > m ? other : m;
    }
    if ((threadIdx.x & 63) == 0) {
        atomicMax(out, m);
    }
}

// Fixed-point exponent for sums bounded by max|x| * count: every partial
// sum stays below 2^62 in magnitude.
__device__ __forceinline__ int fixed_exponent(uint32_t max_bits, double count) {
    const double bound = (double)__uint_as_float(max_bits) * count;
    if (!(bound > 0.0)) {
        return 0;
    }
    int e;
    frexp(bound, &e);  // bound < 2^e
    return 62 - e;
}

// Map VJP of EquirectSample (EquirectSampleBwd, f_ops.cpp:2823-2919): each
// pixel's gy * tap weight (the reference's float product) added to its four
// texels in fixed point at 2^k.
__global__ __launch_bounds__(256) void k_eq_scatter(const float* gy, uint32_t n, const float* dir,
                                                    size_t npx, int mw, int mh,
                                                    const uint32_t* max_bits,
                                                    unsigned long long* acc) {
    const size_t p = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= npx) {
        return;
    }
    float u, v;
    if (!dir_to_equirect(mk3(dir[p * 3 + 0], dir[p * 3 + 1], dir[p * 3 + 2]), &u, &v)) {
        return;
    }
    const int k = fixed_exponent(*max_bits, (double)npx);
    const Taps t = taps_wrap(mw, mh, u, v);
    for (uint32_t c = 0; c < n; c++) {
        const float g = gy[p * n + c];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float prod = g * t.w[j];
            const long long q = __double2ll_rn(ldexp((double)prod, k));
            if (q) {
                atomicAdd(&acc[(size_t)t.idx[j] * n + c], (unsigned long long)q);
            }
        }
    }
}

__global__ __launch_bounds__(256) void k_fixed_resolve(const unsigned long long* acc,
                                                       size_t count, const uint32_t* max_bits,
                                                       double npx, float* out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) {
        return;
    }
    const int k = fixed_exponent(*max_bits, npx);
    out[i] = (float)ldexp((double)(long long)acc[i], -k);
}

// ---------------------------------------------------------------------------
// AvgPool2x2 (Reduce2x2Sum * 0.25, f_ops.cpp:996-1033, 3411-3415)
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void k_pool_fwd(const float* x, int w, int h, uint32_t n,
                                                  int ow, int oh, float* out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= ow * oh) {
        return;
    }
    const int ox = i % ow, oy = i / ow;
    for (uint32_t c = 0; c < n; c++) {
        float acc = 0.f;
        for (int dy = 0; dy < 2; dy++) {
            for (int dx = 0; dx < 2; dx++) {
                const int px = 2 * ox + dx, py = 2 * oy + dy;
                if (px < w && py < h) {
                    acc += x[((size_t)py * w + px) * n + c];
                }
            }
        }
        out[(size_t)i * n + c] = acc * 0.25f;
    }
}

// VJP: UpsampleNearest2x(gy * 0.25) (f_ops.cpp:958-994)
__global__ __launch_bounds__(256) void k_pool_bwd(const float* gy, int w, int h, uint32_t n,
                                                  int ow, float* out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= w * h) {
        return;
    }
    const int px = i % w, py = i / w;
    for (uint32_t c = 0; c < n; c++) {
        out[(size_t)i * n + c] = gy[((size_t)(py / 2) * ow + px / 2) * n + c] * 0.25f;
    }
}

// ---------------------------------------------------------------------------
// Dense equirect convolutions
// ---------------------------------------------------------------------------

enum ConvMode : int {
    kIrrFwd = 0,   // out(t) = scale * sum_s e(s) max(N_t . d_s, 0) sin_s
    kIrrBwd = 1,   // out(s) = scale * sum_t gy(t) max(N_t . d_s, 0) sin_s
    kPrefNorm = 2, // out(t) = sum_s ggx(r_t . d_s) sin_s
    kPrefFwd = 3,  // out(t) = sum_s e(s) ggx(r_t . d_s) sin_s / max(W_t, 1e-12)
    kPrefBwd = 4,  // out(s) = sin_s sum_t gy(t) ggx(r_t . d_s) / max(W_t, 1e-12)
};

// One thread per output texel, the other side in the reference's loop order
// (f_ops.cpp:2970-3087, 3166-3348). `odir` are the output-map directions,
// `sdir` the source (env) directions; `in` is the env (forward modes) or the
// output-map gradient (backward modes), n <= 4 channels.
template <int MODE>
__global__ __launch_bounds__(64) void k_eq_conv(const float4* odir, uint32_t n_o,
                                                const float4* sdir, uint32_t n_s,
                                                const float* in, const float* norm, uint32_t n,
                                                float alpha, float scale, float* out) {
    constexpr bool kBwd = MODE == kIrrBwd || MODE == kPrefBwd;
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t n_i = kBwd ? n_s : n_o;
    const uint32_t n_j = kBwd ? n_o : n_s;
    if (i >= n_i) {
        return;
    }
    const float4 me = kBwd ? sdir[i] : odir[i];
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t j = 0; j < n_j; j++) {
        const float4 ot = kBwd ? odir[j] : me;
        const float4 sd = kBwd ? me : sdir[j];
        const float dt = ot.x * sd.x + ot.y * sd.y + ot.z * sd.z;
        float w;
        if (MODE == kIrrFwd || MODE == kIrrBwd) {
            w = (dt > 0.f ? dt : 0.f) * sd.w;
        } else if (MODE == kPrefNorm || MODE == kPrefFwd) {
            w = ggx_conv_weight(dt, alpha) * sd.w;
        } else {
            const float w0 = ggx_conv_weight(dt, alpha);
            if (w0 <= 0.f) {
                continue;
            }
            const float nt = norm[j];
            w = w0 / (nt > 1e-12f ? nt : 1e-12f);
        }
        if (MODE == kPrefNorm) {
            acc[0] += w;
        } else {
            const float* src = in + (size_t)j * n;
            for (uint32_t c = 0; c < n; c++) {
                acc[c] += src[c] * w;
            }
        }
    }
    if (MODE == kPrefNorm) {
        out[i] = acc[0];
        return;
    }
    for (uint32_t c = 0; c < n; c++) {
        float r = acc[c];
        if (MODE == kIrrFwd || MODE == kIrrBwd) {
            r *= scale;
        } else if (MODE == kPrefFwd) {
            const float nt = norm[i];
            r /= (nt > 1e-12f ? nt : 1e-12f);
        } else {
            r *= me.w;
        }
        out[(size_t)i * n + c] = r;
    }
}

// PrefilterEnv (f_ops.cpp:3089-3157): per output texel, n_samples GGX
// importance samples (Hammersley table), NoL-weighted bilinear taps.
__global__ __launch_bounds__(64) void k_prefilter_env(const float4* odir, uint32_t n_o,
                                                      const float* env, int sw, int sh,
                                                      uint32_t n, const float4* smp,
                                                      uint32_t n_samples, float roughness,
                                                      float* out) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_o) {
        return;
    }
    const float4 o = odir[i];
    const V3f N = mk3(o.x, o.y, o.z);
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    float wsum = 0.f;
    for (uint32_t s = 0; s < n_samples; s++) {
        const V3f h = importance_sample_ggx(smp[s], roughness, N);
        const float ndh2 = 2.f * dot3(N, h);
        const V3f l = normalize3(mk3(ndh2 * h.x - N.x, ndh2 * h.y - N.y, ndh2 * h.z - N.z));
        const float nol = dot3(N, l);
        if (nol > 0.f) {
            float u, v, tap[4];
            equirect_uv(l, &u, &v);
            taps_fetch(taps_wrap(sw, sh, u, v), env, n, tap);
            for (uint32_t c = 0; c < n; c++) {
                acc[c] += tap[c] * nol;
            }
            wsum += nol;
        }
    }
    const float wden = wsum > 1e-4f ? wsum : 1e-4f;
    for (uint32_t c = 0; c < n; c++) {
        out[(size_t)i * n + c] = acc[c] / wden;
    }
}

// BrdfIntegrationLut (f_ops.cpp:3350-3409)
__global__ __launch_bounds__(64) void k_brdf_lut(int w, int h, const float4* smp,
                                                 uint32_t n_samples, float2* out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= w * h) {
        return;
    }
    const int ox = i % w, oy = i / w;
    const float rough = ((float)oy + 0.5f) / (float)h;
    const float k = rough * rough / 2.f;
    const float ndv = ((float)ox + 0.5f) / (float)w;
    const float s0 = 1.f - ndv * ndv;
    const V3f V = mk3(sqrtf(s0 > 0.f ? s0 : 0.f), 0.f, ndv);
    float a = 0.f, b = 0.f;
    for (uint32_t s = 0; s < n_samples; s++) {
        const V3f hv = importance_sample_ggx(smp[s], rough, mk3(0.f, 0.f, 1.f));
        const float vdh2 = 2.f * dot3(V, hv);
        const V3f l = normalize3(mk3(vdh2 * hv.x - V.x, vdh2 * hv.y - V.y, vdh2 * hv.z - V.z));
        const float nol = l.z > 0.f ? l.z : 0.f;
        const float noh = hv.z > 0.f ? hv.z : 0.f;
        const float vd = dot3(V, hv);
        const float voh = vd > 0.f ? vd : 0.f;
        if (nol > 0.f) {
            const float g = g1_ibl(ndv, k) * g1_ibl(nol, k);
            const float nd = noh * ndv;
            const float gv = g * voh / (nd > 1e-8f ? nd : 1e-8f);
            const float fc = libm::pow5f(1.f - voh);
            a += (1.f - fc) * gv;
            b += fc * gv;
        }
    }
    out[i] = make_float2(a / (float)n_samples, b / (float)n_samples);
}

// host table -> context workspace `slot` (synchronous: the table is a
// temporary)
int upload(dressi_ctx* ctx, int slot, const std::vector<float4>& v, const float4** out) {
    void* p = nullptr;
    if (int rc = ctx_workspace(ctx, slot, v.size() * sizeof(float4), &p)) return rc;
    DRESSI_TRY_HIP(hipMemcpyAsync(p, v.data(), v.size() * sizeof(float4), hipMemcpyHostToDevice,
                                  ctx->stream));
    DRESSI_TRY_HIP(hipStreamSynchronize(ctx->stream));
    *out = (const float4*)p;
    return DRESSI_OK;
}

template <int MODE>
int run_conv(dressi_ctx* ctx, const float* in, uint32_t sw, uint32_t sh, uint32_t n,
             uint32_t ow, uint32_t oh, float alpha, const float* norm, float* out) {
    const float4 *od = nullptr, *sd = nullptr;
    if (int rc = upload(ctx, 10, host_equirect_dirs(ow, oh), &od)) return rc;
    if (int rc = upload(ctx, 11, host_equirect_dirs(sw, sh), &sd)) return rc;
    constexpr bool kBwd = MODE == kIrrBwd || MODE == kPrefBwd;
    const uint32_t n_i = kBwd ? sw * sh : ow * oh;
    const float scale = kIblTwoPi / ((float)sw * (float)sh);
    hipLaunchKernelGGL(k_eq_conv<MODE>, dim3(div_up(n_i, 64)), dim3(64), 0, ctx->stream, od,
                       ow * oh, sd, sw * sh, in, norm, n, alpha, scale, out);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int check_map(uint32_t w, uint32_t h, uint32_t n) {
    DRESSI_REQUIRE(n >= 1 && n <= 4, "n_comp must be 1..4");
    DRESSI_REQUIRE(w > 0 && h > 0 && (uint64_t)w * h < (1ull << 28), "bad map size %ux%u", w, h);
    return DRESSI_OK;
}

}  // namespace
}  // namespace dressi

using namespace dressi;

extern "C" {

int dressi_equirect_sample(dressi_ctx* ctx, const float* map, uint32_t mw, uint32_t mh,
                           uint32_t n_comp, const float* dir, uint32_t dw, uint32_t dh,
                           float* out) {
    DRESSI_REQUIRE(ctx && map && dir && out, "bad arguments");
    if (int rc = check_map(mw, mh, n_comp)) return rc;
    const size_t npx = (size_t)dw * dh;
    if (!npx) return DRESSI_OK;
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    hipLaunchKernelGGL(k_eq_sample, dim3((uint32_t)((npx + 255) / 256)), dim3(256), 0,
                       ctx->stream, map, (int)mw, (int)mh, n_comp, dir, npx, out);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int dressi_equirect_sample_bwd(dressi_ctx* ctx, const float* gy, uint32_t n_comp,
                               const float* dir, uint32_t dw, uint32_t dh, uint32_t mw,
                               uint32_t mh, float* out) {
    DRESSI_REQUIRE(ctx && gy && dir && out, "bad arguments");
    if (int rc = check_map(mw, mh, n_comp)) return rc;
    const size_t npx = (size_t)dw * dh, cnt = (size_t)mw * mh * n_comp;
    DRESSI_REQUIRE(npx < (1ull << 40), "too many pixels");
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    void *acc = nullptr, *mx = nullptr;
    if (int rc = ctx_workspace(ctx, 12, cnt * sizeof(unsigned long long), &acc)) return rc;
    if (int rc = ctx_workspace(ctx, 13, sizeof(uint32_t), &mx)) return rc;
    if (int rc = launch_zero(ctx->stream, acc, cnt * sizeof(unsigned long long))) return rc;
    if (int rc = launch_zero(ctx->stream, mx, sizeof(uint32_t))) return rc;
    if (npx) {
        const size_t ng = npx * n_comp;
        const uint32_t blocks = (uint32_t)std::min<size_t>((ng + 255) / 256, 1024);
        hipLaunchKernelGGL(k_max_abs, dim3(blocks), dim3(256), 0, ctx->stream, gy, ng,
                           (uint32_t*)mx);
        DRESSI_CHECK_LAUNCH();
        hipLaunchKernelGGL(k_eq_scatter, dim3((uint32_t)((npx + 255) / 256)), dim3(256), 0,
                           ctx->stream, gy, n_comp, dir, npx, (int)mw, (int)mh,
                           (const uint32_t*)mx, (unsigned long long*)acc);
        DRESSI_CHECK_LAUNCH();
    }
    hipLaunchKernelGGL(k_fixed_resolve, dim3((uint32_t)((cnt + 255) / 256)), dim3(256), 0,
                       ctx->stream, (const unsigned long long*)acc, cnt, (const uint32_t*)mx,
                       (double)npx, out);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int dressi_avg_pool2x2(dressi_ctx* ctx, const float* x, uint32_t w, uint32_t h, uint32_t n_comp,
                       float* out) {
    DRESSI_REQUIRE(ctx && x && out, "bad arguments");
    if (int rc = check_map(w, h, n_comp)) return rc;
    const uint32_t ow = (w + 1) / 2, oh = (h + 1) / 2;
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    hipLaunchKernelGGL(k_pool_fwd, dim3(div_up(ow * oh, 256)), dim3(256), 0, ctx->stream, x,
                       (int)w, (int)h, n_comp, (int)ow, (int)oh, out);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int dressi_avg_pool2x2_bwd(dressi_ctx* ctx, const float* gy, uint32_t w, uint32_t h,
                           uint32_t n_comp, float* out) {
    DRESSI_REQUIRE(ctx && gy && out, "bad arguments");
    if (int rc = check_map(w, h, n_comp)) return rc;
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    hipLaunchKernelGGL(k_pool_bwd, dim3(div_up(w * h, 256)), dim3(256), 0, ctx->stream, gy,
                       (int)w, (int)h, n_comp, (int)((w + 1) / 2), out);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int dressi_irradiance_conv(dressi_ctx* ctx, const float* env, uint32_t sw, uint32_t sh,
                           uint32_t n_comp, uint32_t ow, uint32_t oh, float* out) {
    DRESSI_REQUIRE(ctx && env && out, "bad arguments");
    if (int rc = check_map(sw, sh, n_comp)) return rc;
    if (int rc = check_map(ow, oh, n_comp)) return rc;
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    return run_conv<kIrrFwd>(ctx, env, sw, sh, n_comp, ow, oh, 0.f, nullptr, out);
}

int dressi_irradiance_conv_bwd(dressi_ctx* ctx, const float* gy, uint32_t ow, uint32_t oh,
                               uint32_t n_comp, uint32_t sw, uint32_t sh, float* out) {
    DRESSI_REQUIRE(ctx && gy && out, "bad arguments");
    if (int rc = check_map(sw, sh, n_comp)) return rc;
    if (int rc = check_map(ow, oh, n_comp)) return rc;
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    return run_conv<kIrrBwd>(ctx, gy, sw, sh, n_comp, ow, oh, 0.f, nullptr, out);
}

int dressi_prefilter_conv_norm(dressi_ctx* ctx, uint32_t ow, uint32_t oh, uint32_t sw,
                               uint32_t sh, float roughness, float* out) {
    DRESSI_REQUIRE(ctx && out, "bad arguments");
    if (int rc = check_map(sw, sh, 1)) return rc;
    if (int rc = check_map(ow, oh, 1)) return rc;
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    const float r = roughness > 0.045f ? roughness : 0.045f;
    return run_conv<kPrefNorm>(ctx, nullptr, sw, sh, 1, ow, oh, r * r, nullptr, out);
}

int dressi_prefilter_conv(dressi_ctx* ctx, const float* env, uint32_t sw, uint32_t sh,
                          uint32_t n_comp, uint32_t ow, uint32_t oh, float roughness,
                          const float* norm, float* out) {
    DRESSI_REQUIRE(ctx && env && norm && out, "bad arguments");
    if (int rc = check_map(sw, sh, n_comp)) return rc;
    if (int rc = check_map(ow, oh, n_comp)) return rc;
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    const float r = roughness > 0.045f ? roughness : 0.045f;
    return run_conv<kPrefFwd>(ctx, env, sw, sh, n_comp, ow, oh, r * r, norm, out);
}

int dressi_prefilter_conv_bwd(dressi_ctx* ctx, const float* gy, uint32_t ow, uint32_t oh,
                              uint32_t n_comp, uint32_t sw, uint32_t sh, float roughness,
                              const float* norm, float* out) {
    DRESSI_REQUIRE(ctx && gy && norm && out, "bad arguments");
    if (int rc = check_map(sw, sh, n_comp)) return rc;
    if (int rc = check_map(ow, oh, n_comp)) return rc;
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    const float r = roughness > 0.045f ? roughness : 0.045f;
    return run_conv<kPrefBwd>(ctx, gy, sw, sh, n_comp, ow, oh, r * r, norm, out);
}

int dressi_prefilter_env(dressi_ctx* ctx, const float* env, uint32_t sw, uint32_t sh,
                         uint32_t n_comp, uint32_t ow, uint32_t oh, float roughness,
                         uint32_t n_samples, float* out) {
    DRESSI_REQUIRE(ctx && env && out, "bad arguments");
    DRESSI_REQUIRE(n_samples > 0, "n_samples must be > 0");
    if (int rc = check_map(sw, sh, n_comp)) return rc;
    if (int rc = check_map(ow, oh, n_comp)) return rc;
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    const float4 *od = nullptr, *smp = nullptr;
    if (int rc = upload(ctx, 10, host_equirect_dirs(ow, oh), &od)) return rc;
    if (int rc = upload(ctx, 11, host_hammersley(n_samples), &smp)) return rc;
    hipLaunchKernelGGL(k_prefilter_env, dim3(div_up(ow * oh, 64)), dim3(64), 0, ctx->stream, od,
                       ow * oh, env, (int)sw, (int)sh, n_comp, smp, n_samples, roughness, out);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int dressi_brdf_lut(dressi_ctx* ctx, uint32_t w, uint32_t h, uint32_t n_samples, float* out) {
    DRESSI_REQUIRE(ctx && out, "bad arguments");
    DRESSI_REQUIRE(n_samples > 0, "n_samples must be > 0");
    if (int rc = check_map(w, h, 2)) return rc;
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    const float4* smp = nullptr;
    if (int rc = upload(ctx, 11, host_hammersley(n_samples), &smp)) return rc;
    hipLaunchKernelGGL(k_brdf_lut, dim3(div_up(w * h, 64)), dim3(64), 0, ctx->stream, (int)w,
                       (int)h, smp, n_samples, (float2*)out);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

}  // extern "C"
