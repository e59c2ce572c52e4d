/*
 * pbr_oracle.c -- CPU restatement of the reference's split-sum PBR / IBL
 * path (C5). TEST INFRASTRUCTURE ONLY: used by tests/, by
 * __graft_entry__.smoke() as the checker and by bench.py's cpu_baseline leg;
 * the product path never links, loads or calls it.
 *
 * Follows src/core/ibl_math.h (equirect mapping, bilinear taps, Hammersley,
 * GGX sampling, the GGX convolution weight), the CPU kernels of the IBL ops
 * in src/core/f_ops.cpp:2785-3415, the map builders of src/core/ibl.cpp and
 * the shading graph of examples/common/pbr_graph.cpp. Transcendentals are the
 * C library's float functions, as in the reference's CPU build; loops keep
 * the reference's summation order, so each per-op function reproduces the
 * reference's CPU result bit for bit.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "dressi_oracle.h"

#define K_PI 3.14159265358979323846f
#define K_TWO_PI 6.28318530717958647692f
#define K_INV_PI 0.31830988618379067154f
#define K_INV_TWO_PI 0.15915494309189533577f

typedef struct {
    float x, y, z;
} V3;

static V3 v3(float x, float y, float z) {
    V3 r = {x, y, z};
    return r;
}
static float dot3(V3 a, V3 b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
static V3 cross3(V3 a, V3 b) {
    return v3(a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x);
}
static V3 normalize3(V3 v) {
    const float len = sqrtf(dot3(v, v));
    return v3(v.x / len, v.y / len, v.z / len);
}
static float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }
static float maxf(float a, float b) { return a < b ? b : a; }
static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* ibl_math.h:41-46 */
static void equirect_uv(V3 d, float* u, float* v) {
    *u = atan2f(d.z, d.x) * K_INV_TWO_PI + 0.5f;
    *v = acosf(clampf(d.y, -1.f, 1.f)) * K_INV_PI;
}

/* ibl_math.h:48-54 */
static V3 dir_from_uv(float u, float v) {
    const float phi = (u - 0.5f) * K_TWO_PI;
    const float theta = v * K_PI;
    const float st = sinf(theta);
    return v3(st * cosf(phi), cosf(theta), st * sinf(phi));
}

/* ibl_math.h:58-89: u wraps, v clamps */
static void bilerp_wrap(const float* data, uint32_t w, uint32_t h, uint32_t n, float u, float v,
                        float* out) {
    const float sx = u * (float)w - 0.5f;
    const float sy = v * (float)h - 0.5f;
    const int ix = (int)floorf(sx);
    const int iy = (int)floorf(sy);
    const float fx = sx - (float)ix;
    const float fy = sy - (float)iy;
    for (uint32_t c = 0; c < n; c++) out[c] = 0.f;
    for (int dy = 0; dy <= 1; dy++) {
        for (int dx = 0; dx <= 1; dx++) {
            int x = ix + dx;
            if (x < 0) x += (int)w;
            if (x >= (int)w) x -= (int)w;
            const int y = clampi(iy + dy, 0, (int)h - 1);
            const float wgt = (dx == 0 ? 1.f - fx : fx) * (dy == 0 ? 1.f - fy : fy);
            const float* p = data + ((size_t)y * w + (size_t)x) * n;
            for (uint32_t c = 0; c < n; c++) out[c] += wgt * p[c];
        }
    }
}

/* ibl_math.h:92-115: both axes clamped */
static void bilerp_clamp(const float* data, uint32_t w, uint32_t h, uint32_t n, float u, float v,
                         float* out) {
    const float sx = u * (float)w - 0.5f;
    const float sy = v * (float)h - 0.5f;
    const int ix = (int)floorf(sx);
    const int iy = (int)floorf(sy);
    const float fx = sx - (float)ix;
    const float fy = sy - (float)iy;
    for (uint32_t c = 0; c < n; c++) out[c] = 0.f;
    for (int dy = 0; dy <= 1; dy++) {
        for (int dx = 0; dx <= 1; dx++) {
            const int x = clampi(ix + dx, 0, (int)w - 1);
            const int y = clampi(iy + dy, 0, (int)h - 1);
            const float wgt = (dx == 0 ? 1.f - fx : fx) * (dy == 0 ? 1.f - fy : fy);
            const float* p = data + ((size_t)y * w + (size_t)x) * n;
            for (uint32_t c = 0; c < n; c++) out[c] += wgt * p[c];
        }
    }
}

/* ibl_math.h:119-132 */
static float radical_inverse(uint32_t bits) {
    bits = (bits << 16u) | (bits >> 16u);
    bits = ((bits & 0x55555555u) << 1u) | ((bits & 0xAAAAAAAAu) >> 1u);
    bits = ((bits & 0x33333333u) << 2u) | ((bits & 0xCCCCCCCCu) >> 2u);
    bits = ((bits & 0x0F0F0F0Fu) << 4u) | ((bits & 0xF0F0F0F0u) >> 4u);
    bits = ((bits & 0x00FF00FFu) << 8u) | ((bits & 0xFF00FF00u) >> 8u);
    return (float)bits * 2.3283064365386963e-10f;
}

/* ibl_math.h:134-150 */
static V3 importance_sample_ggx(float xi0, float xi1, float roughness, V3 n) {
    const float a = roughness * roughness;
    const float phi = K_TWO_PI * xi0;
    const float ct = sqrtf((1.f - xi1) / (1.f + (a * a - 1.f) * xi1));
    const float st = sqrtf(maxf(1.f - ct * ct, 0.f));
    const V3 h_t = v3(cosf(phi) * st, sinf(phi) * st, ct);
    const V3 up = fabsf(n.z) < 0.999f ? v3(0.f, 0.f, 1.f) : v3(1.f, 0.f, 0.f);
    const V3 tx = normalize3(cross3(up, n));
    const V3 ty = cross3(n, tx);
    return normalize3(v3(tx.x * h_t.x + ty.x * h_t.y + n.x * h_t.z,
                         tx.y * h_t.x + ty.y * h_t.y + n.y * h_t.z,
                         tx.z * h_t.x + ty.z * h_t.y + n.z * h_t.z));
}

/* ibl_math.h:153-156 */
static float g1_ibl(float n_dot_x, float k) { return n_dot_x / (n_dot_x * (1.f - k) + k); }

/* ibl_math.h:162-170 */
static float ggx_conv_weight(float c, float alpha) {
    if (c <= 0.f) return 0.f;
    const float ch2 = (1.f + c) * 0.5f;
    const float a2 = alpha * alpha;
    const float d = ch2 * (a2 - 1.f) + 1.f;
    return a2 / (K_PI * d * d) * c;
}

/* ---- per-op kernels ------------------------------------------------------ */

/* EquirectSample (f_ops.cpp:2921-2964): zero-length directions give 0.
 * With gy: the map VJP of EquirectSampleBwd (f_ops.cpp:2823-2919): K
 * partial maps, one per band of rows_per dir rows, summed by TileSum
 * (f_ops.cpp:2786-2821) in band order. */
int or_equirect_sample(const float* map, uint32_t mw, uint32_t mh, uint32_t n, const float* dir,
                       uint32_t dw, uint32_t dh, const float* gy, float* out) {
    if (!gy) {
        for (size_t p = 0; p < (size_t)dw * dh; p++) {
            V3 d = v3(dir[p * 3 + 0], dir[p * 3 + 1], dir[p * 3 + 2]);
            float* o = &out[p * n];
            const float dlen = sqrtf(dot3(d, d));
            if (dlen < 1e-8f) {
                for (uint32_t c = 0; c < n; c++) o[c] = 0.f;
                continue;
            }
            d = v3(d.x / dlen, d.y / dlen, d.z / dlen);
            float u, v;
            equirect_uv(d, &u, &v);
            bilerp_wrap(map, mw, mh, n, u, v, o);
        }
        return 0;
    }
    uint32_t k = 1;
    while ((size_t)mw * mh * k < 65536 && k < dh) k *= 2;
    const uint32_t rows_per = (dh + k - 1) / k;
    const size_t msz = (size_t)mw * mh * n;
    float* part = (float*)calloc(msz * k, sizeof(float));
    if (!part) return -1;
    for (uint32_t py = 0; py < dh; py++) {
        const uint32_t tile = py / rows_per;
        for (uint32_t px = 0; px < dw; px++) {
            const size_t p = (size_t)py * dw + px;
            V3 d = v3(dir[p * 3 + 0], dir[p * 3 + 1], dir[p * 3 + 2]);
            const float dlen = sqrtf(dot3(d, d));
            if (dlen < 1e-8f) continue;
            d = v3(d.x / dlen, d.y / dlen, d.z / dlen);
            float u, v;
            equirect_uv(d, &u, &v);
            const float sx = u * (float)mw - 0.5f;
            const float sy = v * (float)mh - 0.5f;
            const int ix = (int)floorf(sx);
            const int iy = (int)floorf(sy);
            const float fx = sx - (float)ix;
            const float fy = sy - (float)iy;
            for (int dy = 0; dy <= 1; dy++) {
                for (int dx = 0; dx <= 1; dx++) {
                    int x = ix + dx;
                    if (x < 0) x += (int)mw;
                    if (x >= (int)mw) x -= (int)mw;
                    const int y = clampi(iy + dy, 0, (int)mh - 1);
                    const float w = (dx == 0 ? 1.f - fx : fx) * (dy == 0 ? 1.f - fy : fy);
                    float* o = &part[((size_t)(tile * mh + (uint32_t)y) * mw + (uint32_t)x) * n];
                    for (uint32_t c = 0; c < n; c++) o[c] += gy[p * n + c] * w;
                }
            }
        }
    }
    if (k == 1) {
        memcpy(out, part, msz * sizeof(float));
    } else {
        memset(out, 0, msz * sizeof(float));
        for (uint32_t t = 0; t < k; t++) {
            for (size_t i = 0; i < msz; i++) out[i] += part[t * msz + i];
        }
    }
    free(part);
    return 0;
}

/* AvgPool2x2 = Reduce2x2Sum(x) * 0.25 (f_ops.cpp:3411-3415, 996-1033); its
 * VJP is UpsampleNearest2x(gy * 0.25) (f_ops.cpp:958-994). x {w,h} x n. */
int or_avg_pool2x2(const float* x, uint32_t w, uint32_t h, uint32_t n, const float* gy,
                   float* out) {
    const uint32_t ow = (w + 1) / 2, oh = (h + 1) / 2;
    if (gy) {
        for (uint32_t py = 0; py < h; py++) {
            for (uint32_t px = 0; px < w; px++) {
                for (uint32_t c = 0; c < n; c++) {
                    out[((size_t)py * w + px) * n + c] =
                            gy[((size_t)(py / 2) * ow + px / 2) * n + c] * 0.25f;
                }
            }
        }
        return 0;
    }
    memset(out, 0, sizeof(float) * (size_t)ow * oh * n);
    for (uint32_t py = 0; py < h; py++) {
        for (uint32_t px = 0; px < w; px++) {
            for (uint32_t c = 0; c < n; c++) {
                out[((size_t)(py / 2) * ow + px / 2) * n + c] += x[((size_t)py * w + px) * n + c];
            }
        }
    }
    for (size_t i = 0; i < (size_t)ow * oh * n; i++) out[i] = out[i] * 0.25f;
    return 0;
}

/* IrradianceConv (f_ops.cpp:3006-3087) and, with gy, IrradianceConvBwd
 * (f_ops.cpp:2970-3004): the cos-weighted sum over every source texel with
 * the equirect sin(theta) area term, scaled by 2 pi / (sw sh). */
int or_irradiance_conv(const float* env, uint32_t sw, uint32_t sh, uint32_t n, uint32_t ow,
                       uint32_t oh, const float* gy, float* out) {
    const float scale = K_TWO_PI / ((float)sw * (float)sh);
    if (!gy) {
        memset(out, 0, sizeof(float) * (size_t)ow * oh * n);
        for (uint32_t oy = 0; oy < oh; oy++) {
            for (uint32_t ox = 0; ox < ow; ox++) {
                const V3 N = dir_from_uv(((float)ox + 0.5f) / (float)ow,
                                         ((float)oy + 0.5f) / (float)oh);
                float* o = &out[((size_t)oy * ow + ox) * n];
                for (uint32_t sy = 0; sy < sh; sy++) {
                    const float sv = ((float)sy + 0.5f) / (float)sh;
                    const float sin_th = sinf(sv * K_PI);
                    for (uint32_t sx = 0; sx < sw; sx++) {
                        const V3 d = dir_from_uv(((float)sx + 0.5f) / (float)sw, sv);
                        const float w = maxf(dot3(N, d), 0.f) * sin_th;
                        const float* e = &env[((size_t)sy * sw + sx) * n];
                        for (uint32_t c = 0; c < n; c++) o[c] += e[c] * w;
                    }
                }
                for (uint32_t c = 0; c < n; c++) o[c] *= scale;
            }
        }
        return 0;
    }
    memset(out, 0, sizeof(float) * (size_t)sw * sh * n);
    for (uint32_t sy = 0; sy < sh; sy++) {
        const float sv = ((float)sy + 0.5f) / (float)sh;
        const float sin_th = sinf(sv * K_PI);
        for (uint32_t sx = 0; sx < sw; sx++) {
            const V3 d = dir_from_uv(((float)sx + 0.5f) / (float)sw, sv);
            float* o = &out[((size_t)sy * sw + sx) * n];
            for (uint32_t ty = 0; ty < oh; ty++) {
                for (uint32_t tx = 0; tx < ow; tx++) {
                    const V3 N = dir_from_uv(((float)tx + 0.5f) / (float)ow,
                                             ((float)ty + 0.5f) / (float)oh);
                    const float w = maxf(dot3(N, d), 0.f) * sin_th;
                    const float* g = &gy[((size_t)ty * ow + tx) * n];
                    for (uint32_t c = 0; c < n; c++) o[c] += g[c] * w;
                }
            }
            for (uint32_t c = 0; c < n; c++) o[c] *= scale;
        }
    }
    return 0;
}

/* PrefilterConvNorm (f_ops.cpp:3166-3205): W(t) = sum_s w(t,s) sin(theta_s) */
static void prefilter_norm(uint32_t ow, uint32_t oh, uint32_t sw, uint32_t sh, float alpha,
                           float* out) {
    for (uint32_t oy = 0; oy < oh; oy++) {
        for (uint32_t ox = 0; ox < ow; ox++) {
            const V3 r = dir_from_uv(((float)ox + 0.5f) / (float)ow,
                                     ((float)oy + 0.5f) / (float)oh);
            float acc = 0.f;
            for (uint32_t sy = 0; sy < sh; sy++) {
                const float sv = ((float)sy + 0.5f) / (float)sh;
                const float sin_th = sinf(sv * K_PI);
                for (uint32_t sx = 0; sx < sw; sx++) {
                    const V3 d = dir_from_uv(((float)sx + 0.5f) / (float)sw, sv);
                    acc += ggx_conv_weight(dot3(r, d), alpha) * sin_th;
                }
            }
            out[(size_t)oy * ow + ox] = acc;
        }
    }
}

/* PrefilterConv (f_ops.cpp:3264-3348) at alpha = max(roughness, 0.045)^2;
 * with gy, PrefilterConvBwd (f_ops.cpp:3207-3262). */
int or_prefilter_conv(const float* env, uint32_t sw, uint32_t sh, uint32_t n, uint32_t ow,
                      uint32_t oh, float roughness, const float* gy, float* out) {
    const float alpha = maxf(roughness, 0.045f) * maxf(roughness, 0.045f);
    float* norm = (float*)malloc(sizeof(float) * (size_t)ow * oh);
    if (!norm) return -1;
    prefilter_norm(ow, oh, sw, sh, alpha, norm);
    if (!gy) {
        memset(out, 0, sizeof(float) * (size_t)ow * oh * n);
        for (uint32_t oy = 0; oy < oh; oy++) {
            for (uint32_t ox = 0; ox < ow; ox++) {
                const V3 r = dir_from_uv(((float)ox + 0.5f) / (float)ow,
                                         ((float)oy + 0.5f) / (float)oh);
                float* o = &out[((size_t)oy * ow + ox) * n];
                for (uint32_t sy = 0; sy < sh; sy++) {
                    const float sv = ((float)sy + 0.5f) / (float)sh;
                    const float sin_th = sinf(sv * K_PI);
                    for (uint32_t sx = 0; sx < sw; sx++) {
                        const V3 d = dir_from_uv(((float)sx + 0.5f) / (float)sw, sv);
                        const float w = ggx_conv_weight(dot3(r, d), alpha) * sin_th;
                        const float* e = &env[((size_t)sy * sw + sx) * n];
                        for (uint32_t c = 0; c < n; c++) o[c] += e[c] * w;
                    }
                }
                const float wn = maxf(norm[(size_t)oy * ow + ox], 1e-12f);
                for (uint32_t c = 0; c < n; c++) o[c] /= wn;
            }
        }
        free(norm);
        return 0;
    }
    memset(out, 0, sizeof(float) * (size_t)sw * sh * n);
    for (uint32_t sy = 0; sy < sh; sy++) {
        const float sv = ((float)sy + 0.5f) / (float)sh;
        const float sin_th = sinf(sv * K_PI);
        for (uint32_t sx = 0; sx < sw; sx++) {
            const V3 d = dir_from_uv(((float)sx + 0.5f) / (float)sw, sv);
            float* o = &out[((size_t)sy * sw + sx) * n];
            for (uint32_t ty = 0; ty < oh; ty++) {
                for (uint32_t tx = 0; tx < ow; tx++) {
                    const V3 r = dir_from_uv(((float)tx + 0.5f) / (float)ow,
                                             ((float)ty + 0.5f) / (float)oh);
                    const float w = ggx_conv_weight(dot3(r, d), alpha);
                    if (w <= 0.f) continue;
                    const float wn = w / maxf(norm[(size_t)ty * ow + tx], 1e-12f);
                    const float* g = &gy[((size_t)ty * ow + tx) * n];
                    for (uint32_t c = 0; c < n; c++) o[c] += g[c] * wn;
                }
            }
            for (uint32_t c = 0; c < n; c++) o[c] *= sin_th;
        }
    }
    free(norm);
    return 0;
}

/* PrefilterEnv (f_ops.cpp:3089-3157): GGX importance sampling with the
 * Hammersley sequence, NoL-weighted, V = N = R; forward only. */
int or_prefilter_env(const float* env, uint32_t sw, uint32_t sh, uint32_t n, uint32_t ow,
                     uint32_t oh, float roughness, uint32_t n_samples, float* out) {
    float tap[4];
    if (n > 4) return -1;
    memset(out, 0, sizeof(float) * (size_t)ow * oh * n);
    for (uint32_t oy = 0; oy < oh; oy++) {
        for (uint32_t ox = 0; ox < ow; ox++) {
            const V3 N = dir_from_uv(((float)ox + 0.5f) / (float)ow,
                                     ((float)oy + 0.5f) / (float)oh);
            float* o = &out[((size_t)oy * ow + ox) * n];
            float wsum = 0.f;
            for (uint32_t i = 0; i < n_samples; i++) {
                const float xi0 = (float)i / (float)n_samples;
                const float xi1 = radical_inverse(i);
                const V3 h = importance_sample_ggx(xi0, xi1, roughness, N);
                const float ndh2 = 2.f * dot3(N, h);
                const V3 l = normalize3(v3(ndh2 * h.x - N.x, ndh2 * h.y - N.y, ndh2 * h.z - N.z));
                const float nol = dot3(N, l);
                if (nol > 0.f) {
                    float u, v;
                    equirect_uv(l, &u, &v);
                    bilerp_wrap(env, sw, sh, n, u, v, tap);
                    for (uint32_t c = 0; c < n; c++) o[c] += tap[c] * nol;
                    wsum += nol;
                }
            }
            const float wden = maxf(wsum, 1e-4f);
            for (uint32_t c = 0; c < n; c++) o[c] /= wden;
        }
    }
    return 0;
}

/* BrdfIntegrationLut (f_ops.cpp:3350-3409): VEC2 (A, B) over (NdotV,
 * roughness) texel centres, Smith-G with k = roughness^2 / 2. */
int or_brdf_lut(uint32_t w, uint32_t h, uint32_t n_samples, float* out) {
    for (uint32_t oy = 0; oy < h; oy++) {
        const float rough = ((float)oy + 0.5f) / (float)h;
        const float k = rough * rough / 2.f;
        for (uint32_t ox = 0; ox < w; ox++) {
            const float ndv = ((float)ox + 0.5f) / (float)w;
            const V3 V = v3(sqrtf(maxf(1.f - ndv * ndv, 0.f)), 0.f, ndv);
            float a = 0.f, b = 0.f;
            for (uint32_t i = 0; i < n_samples; i++) {
                const float xi0 = (float)i / (float)n_samples;
                const float xi1 = radical_inverse(i);
                const V3 hv = importance_sample_ggx(xi0, xi1, rough, v3(0.f, 0.f, 1.f));
                const float vdh2 = 2.f * dot3(V, hv);
                const V3 l = normalize3(v3(vdh2 * hv.x - V.x, vdh2 * hv.y - V.y,
                                           vdh2 * hv.z - V.z));
                const float nol = maxf(l.z, 0.f);
                const float noh = maxf(hv.z, 0.f);
                const float voh = maxf(dot3(V, hv), 0.f);
                if (nol > 0.f) {
                    const float g = g1_ibl(ndv, k) * g1_ibl(nol, k);
                    const float gv = g * voh / maxf(noh * ndv, 1e-8f);
                    const float fc = powf(1.f - voh, 5.f);
                    a += (1.f - fc) * gv;
                    b += fc * gv;
                }
            }
            const size_t o = ((size_t)oy * w + ox) * 2;
            out[o + 0] = a / (float)n_samples;
            out[o + 1] = b / (float)n_samples;
        }
    }
    return 0;
}

/* ---- the C5 fit ---------------------------------------------------------- */

/* IBL maps of one env (src/core/ibl.cpp:12-93 with levels prefilter levels):
 * irradiance 32 x 16 from the env pooled to <= 64 x 32, prefiltered levels
 * from the env pooled to <= 128 x 64 (the top level no larger than that
 * source), halving per level, roughness i / (levels - 1). */
typedef struct {
    uint32_t ew, eh;             /* env */
    uint32_t iw, ih, isw, ish;   /* irradiance map and its pooled source */
    uint32_t psw, psh;           /* prefilter source */
    uint32_t levels;
    uint32_t lw[16], lh[16];     /* level sizes */
    size_t loff[16];             /* level offsets (floats) in pref */
    uint32_t n_irr_pool, n_pref_pool;
    float* irr;                  /* {iw,ih} x 3 */
    float* pref;                 /* all levels, x 3 */
    float* isrc;                 /* pooled sources */
    float* psrc;
} IblMaps;

static void ibl_layout(IblMaps* m, uint32_t ew, uint32_t eh, uint32_t levels) {
    memset(m, 0, sizeof(*m));
    m->ew = ew;
    m->eh = eh;
    m->iw = 32;
    m->ih = 16;
    m->isw = ew;
    m->ish = eh;
    while (m->isw > 64 || m->ish > 32) {
        m->isw = (m->isw + 1) / 2;
        m->ish = (m->ish + 1) / 2;
        m->n_irr_pool++;
    }
    m->psw = ew;
    m->psh = eh;
    while (m->psw > 128 || m->psh > 64) {
        m->psw = (m->psw + 1) / 2;
        m->psh = (m->psh + 1) / 2;
        m->n_pref_pool++;
    }
    m->levels = levels;
    uint32_t w = m->psw < 128 ? m->psw : 128, h = m->psh < 64 ? m->psh : 64;
    size_t off = 0;
    for (uint32_t i = 0; i < levels; i++) {
        m->lw[i] = w;
        m->lh[i] = h;
        m->loff[i] = off;
        off += (size_t)w * h * 3;
        w = w > 1 ? w / 2 : 1;
        h = h > 1 ? h / 2 : 1;
    }
    m->irr = (float*)calloc((size_t)m->iw * m->ih * 3, sizeof(float));
    m->pref = (float*)calloc(off, sizeof(float));
    m->isrc = (float*)calloc((size_t)m->isw * m->ish * 3, sizeof(float));
    m->psrc = (float*)calloc((size_t)m->psw * m->psh * 3, sizeof(float));
}

static void ibl_free(IblMaps* m) {
    free(m->irr);
    free(m->pref);
    free(m->isrc);
    free(m->psrc);
}

/* pool `env` n_pool times into dst (sizes halve, rounding up) */
static void pool_chain(const float* env, uint32_t w, uint32_t h, uint32_t n_pool, float* dst) {
    float* a = (float*)malloc(sizeof(float) * (size_t)w * h * 3);
    float* b = (float*)malloc(sizeof(float) * (size_t)w * h * 3);
    memcpy(a, env, sizeof(float) * (size_t)w * h * 3);
    for (uint32_t i = 0; i < n_pool; i++) {
        or_avg_pool2x2(a, w, h, 3, NULL, b);
        w = (w + 1) / 2;
        h = (h + 1) / 2;
        float* t = a;
        a = b;
        b = t;
    }
    memcpy(dst, a, sizeof(float) * (size_t)w * h * 3);
    free(a);
    free(b);
}

static void ibl_build(IblMaps* m, const float* env) {
    pool_chain(env, m->ew, m->eh, m->n_irr_pool, m->isrc);
    or_irradiance_conv(m->isrc, m->isw, m->ish, 3, m->iw, m->ih, NULL, m->irr);
    pool_chain(env, m->ew, m->eh, m->n_pref_pool, m->psrc);
    for (uint32_t i = 0; i < m->levels; i++) {
        const float rough = (float)i / (float)(m->levels - 1);
        or_prefilter_conv(m->psrc, m->psw, m->psh, 3, m->lw[i], m->lh[i], rough, NULL,
                          m->pref + m->loff[i]);
    }
}

/* env gradient from the map gradients: the transposed convolutions, then the
 * pooling chains' VJPs; adds into g_env {ew,eh} x 3. */
static void ibl_backward(const IblMaps* m, const float* g_irr, const float* g_pref, float* g_env) {
    const size_t ne = (size_t)m->ew * m->eh * 3;
    float* a = (float*)calloc(ne, sizeof(float));
    float* b = (float*)calloc(ne, sizeof(float));
    float* t = (float*)calloc(ne, sizeof(float));
    /* irradiance: conv transpose, then n_irr_pool pool VJPs */
    or_irradiance_conv(NULL, m->isw, m->ish, 3, m->iw, m->ih, g_irr, a);
    uint32_t w = m->isw, h = m->ish;
    for (uint32_t i = 0; i < m->n_irr_pool; i++) {
        /* the pooled size w x h came from (2w or 2w-1) x ...: the source
         * sizes are powers of two here, so 2w x 2h */
        or_avg_pool2x2(NULL, 2 * w, 2 * h, 3, a, b);
        w *= 2;
        h *= 2;
        float* s = a;
        a = b;
        b = s;
    }
    for (size_t i = 0; i < ne; i++) g_env[i] += a[i];
    /* prefilter: sum of the levels' conv transposes, then the pool VJPs */
    memset(a, 0, ne * sizeof(float));
    for (uint32_t i = 0; i < m->levels; i++) {
        const float rough = (float)i / (float)(m->levels - 1);
        or_prefilter_conv(NULL, m->psw, m->psh, 3, m->lw[i], m->lh[i], rough,
                          g_pref + m->loff[i], t);
        for (size_t j = 0; j < (size_t)m->psw * m->psh * 3; j++) a[j] += t[j];
    }
    w = m->psw;
    h = m->psh;
    for (uint32_t i = 0; i < m->n_pref_pool; i++) {
        or_avg_pool2x2(NULL, 2 * w, 2 * h, 3, a, b);
        w *= 2;
        h *= 2;
        float* s = a;
        a = b;
        b = s;
    }
    for (size_t i = 0; i < ne; i++) g_env[i] += a[i];
    free(a);
    free(b);
    free(t);
}

/* Per-pixel static G-buffer terms of one view (BuildPbrGBuffer and the
 * geometry-only part of BuildPbrShade, pbr_graph.cpp:34-137). */
typedef struct {
    float mask, u, v;
    V3 n, view, refl, ray;
    float ndv, ndl, ndh, vdh, dist2;
} Gpx;

static V3 safe_normalize(V3 v) {
    const float s = 1.f / sqrtf(dot3(v, v) + 1e-12f);
    return v3(v.x * s, v.y * s, v.z * s);
}

/* Forward shading of one pixel (pbr_graph.cpp:47-137, normal mapping off,
 * AO texture 1, emissive 0) and, when gh != NULL, its backward for
 * d loss / d hdr = gh: material gradients (albedo, roughness channel before
 * the clamp, metallic) and the sampled-map gradients (irradiance, the
 * prefilter levels, the background env). */
typedef struct {
    const float *albedo, *mr, *irr, *pref, *lut, *env;
    const IblMaps* maps;
    uint32_t tw, th, lutw, luth;
    V3 light_col;
} ShadeCtx;

typedef struct {
    float hdr[3];
    /* backward outputs */
    float g_albedo[3], g_mr[3], g_irr[3], g_bg[3];
    float g_pref[16][3];
    V3 n, refl, ray; /* sample directions */
} ShadeOut;

static void sample_eq(const float* map, uint32_t w, uint32_t h, V3 d, float* out) {
    const float dlen = sqrtf(dot3(d, d));
    if (dlen < 1e-8f) {
        out[0] = out[1] = out[2] = 0.f;
        return;
    }
    d = v3(d.x / dlen, d.y / dlen, d.z / dlen);
    float u, v;
    equirect_uv(d, &u, &v);
    bilerp_wrap(map, w, h, 3, u, v, out);
}

static void shade_px(const ShadeCtx* s, const Gpx* g, const float* gh, ShadeOut* o) {
    const IblMaps* m = s->maps;
    float bg[3];
    sample_eq(s->env, m->ew, m->eh, g->ray, bg);
    o->n = g->n;
    o->refl = g->refl;
    o->ray = g->ray;
    if (g->mask == 0.f) {
        for (int c = 0; c < 3; c++) o->hdr[c] = bg[c];
        if (gh) {
            memset(o->g_albedo, 0, sizeof(o->g_albedo));
            memset(o->g_mr, 0, sizeof(o->g_mr));
            memset(o->g_irr, 0, sizeof(o->g_irr));
            memset(o->g_pref, 0, sizeof(o->g_pref));
            for (int c = 0; c < 3; c++) o->g_bg[c] = gh[c];
        }
        return;
    }
    float a[3], mr[3], lut[2];
    bilerp_clamp(s->albedo, s->tw, s->th, 3, g->u, g->v, a);
    bilerp_clamp(s->mr, s->tw, s->th, 3, g->u, g->v, mr);
    /* AO: the all-ones texture's bilinear sum */
    float ao;
    {
        const float sx = g->u * (float)s->tw - 0.5f, sy = g->v * (float)s->th - 0.5f;
        const float fx = sx - floorf(sx), fy = sy - floorf(sy);
        ao = 0.f;
        ao += (1.f - fx) * (1.f - fy) * 1.f;
        ao += fx * (1.f - fy) * 1.f;
        ao += (1.f - fx) * fy * 1.f;
        ao += fx * fy * 1.f;
    }
    const float rough = clampf(mr[1], 0.045f, 1.f);
    const float metal = mr[2];
    const float ndv = g->ndv, ndl = g->ndl, ndh = g->ndh, vdh = g->vdh;
    float f0[3], F[3], kd[3], fib[3], kdi[3], irr[3];
    for (int c = 0; c < 3; c++) f0[c] = 0.04f + (a[c] - 0.04f) * metal;
    const float alpha = rough * rough;
    const float alpha2 = alpha * alpha;
    const float dd = ndh * ndh * (alpha2 - 1.f) + 1.f;
    const float D = alpha2 / (K_PI * dd * dd);
    const float k = (rough + 1.f) * (rough + 1.f) / 8.f;
    const float gvd = ndv * (1.f - k) + k;
    const float g_v = ndv / gvd;
    const float ndlc = maxf(ndl, 1e-4f);
    const float gld = ndlc * (1.f - k) + k;
    const float g_l = ndlc / gld;
    const float p5v = powf(1.f - vdh, 5.f);
    const float den = 4.f * ndv * ndl + 1e-4f;
    const float S = D * g_v * g_l / den;
    const float p5n = powf(1.f - ndv, 5.f);
    float R0[3];
    const float rl[3] = {s->light_col.x, s->light_col.y, s->light_col.z};
    for (int c = 0; c < 3; c++) {
        F[c] = f0[c] + (1.f - f0[c]) * p5v;
        kd[c] = (1.f - F[c]) * (1.f - metal);
        R0[c] = rl[c] / g->dist2;
        const float mx = maxf(1.f - rough, f0[c]);
        fib[c] = f0[c] + (mx - f0[c]) * p5n;
        kdi[c] = (1.f - fib[c]) * (1.f - metal);
    }
    sample_eq(s->irr, m->iw, m->ih, g->n, irr);
    /* prefilter levels: tent weights over lod = rough * (levels - 1) */
    const float lod = rough * (float)(m->levels - 1);
    float pref[3] = {0.f, 0.f, 0.f};
    float P[16][3], wl[16], xl[16];
    for (uint32_t i = 0; i < m->levels; i++) {
        xl[i] = 1.f - fabsf(lod - (float)i);
        wl[i] = clampf(xl[i], 0.f, 1.f);
        if (xl[i] >= 0.f) {
            sample_eq(s->pref + m->loff[i], m->lw[i], m->lh[i], g->refl, P[i]);
            for (int c = 0; c < 3; c++) pref[c] += P[i][c] * wl[i];
        }
    }
    bilerp_clamp(s->lut, s->lutw, s->luth, 2, ndv, rough, lut);
    for (int c = 0; c < 3; c++) {
        const float lo = (kd[c] * a[c] / K_PI + F[c] * S) * R0[c] * ndl;
        const float spec_ibl = pref[c] * (f0[c] * lut[0] + lut[1]);
        const float amb = (kdi[c] * irr[c] * a[c] + spec_ibl) * ao;
        const float shaded = lo + amb + 0.f;
        o->hdr[c] = g->mask * shaded + (1.f - g->mask) * bg[c];
    }
    if (!gh) return;
    float ga[3] = {0, 0, 0}, gm = 0.f, gr = 0.f, gS = 0.f, gf0[3];
    for (int c = 0; c < 3; c++) {
        const float gs = g->mask * gh[c];
        o->g_bg[c] = (1.f - g->mask) * gh[c];
        /* lo = (kd a / pi + F S) R0 ndl */
        const float q = gs * R0[c] * ndl;
        ga[c] += q * kd[c] / K_PI;
        const float gkd = q * a[c] / K_PI;
        const float gF = q * S - gkd * (1.f - metal);
        gS += q * F[c];
        gm -= gkd * (1.f - F[c]);
        /* ambient = (kdi irr a + pref (f0 A + B)) ao */
        const float u = gs * ao;
        o->g_irr[c] = u * kdi[c] * a[c];
        ga[c] += u * kdi[c] * irr[c];
        const float gkdi = u * irr[c] * a[c];
        const float gpref = u * (f0[c] * lut[0] + lut[1]);
        gf0[c] = u * pref[c] * lut[0];
        const float gfib = -gkdi * (1.f - metal);
        gm -= gkdi * (1.f - fib[c]);
        /* f_ibl = f0 + (max(1 - r, f0) - f0) p5n: Max picks x0 = 1 - r when
         * x0 >= f0 */
        const int pick_r = (1.f - rough) >= f0[c];
        gf0[c] += gfib * (1.f - p5n) + (pick_r ? 0.f : gfib * p5n);
        if (pick_r) gr -= gfib * p5n;
        /* F = f0 + (1 - f0) p5v */
        gf0[c] += gF * (1.f - p5v);
        /* f0 = 0.04 + (a - 0.04) m */
        ga[c] += gf0[c] * metal;
        gm += gf0[c] * (a[c] - 0.04f);
        /* prefilter levels */
        for (uint32_t i = 0; i < m->levels; i++) {
            o->g_pref[i][c] = xl[i] >= 0.f ? gpref * wl[i] : 0.f;
        }
    }
    /* lod weights: w_i = clamp(1 - |lod - i|, 0, 1) */
    float glod = 0.f;
    for (uint32_t i = 0; i < m->levels; i++) {
        if (xl[i] < 0.f || xl[i] > 1.f) continue;
        float gw = 0.f;
        for (int c = 0; c < 3; c++) {
            const float u = g->mask * gh[c] * ao;
            gw += u * (f0[c] * lut[0] + lut[1]) * P[i][c];
        }
        const float dl = lod - (float)i;
        const float sgn = (float)((dl > 0.f) - (dl < 0.f));
        glod -= gw * sgn;
    }
    gr += glod * (float)(m->levels - 1);
    /* S = D g_v g_l / den */
    const float gD = gS * g_v * g_l / den;
    const float ggv = gS * D * g_l / den;
    const float ggl = gS * D * g_v / den;
    const float galpha2 = gD * (1.f / (K_PI * dd * dd) - 2.f * alpha2 * ndh * ndh / (K_PI * dd * dd * dd));
    gr += galpha2 * 2.f * alpha * 2.f * rough;
    const float gk = ggv * (-ndv * (1.f - ndv) / (gvd * gvd)) +
                     ggl * (-ndlc * (1.f - ndlc) / (gld * gld));
    gr += gk * (rough + 1.f) / 4.f;
    for (int c = 0; c < 3; c++) o->g_albedo[c] = ga[c];
    o->g_mr[0] = 0.f;
    o->g_mr[1] = (mr[1] >= 0.045f && 1.f >= mr[1]) ? gr : 0.f;
    o->g_mr[2] = gm;
}

/* See the header: the C5 split-sum PBR/IBL material + environment fit. */
/* F::Sum (f_ops.cpp:1037-1043): Reduce2x2Sum (f_ops.cpp:999-1033: each
 * output texel of the (w + 1) / 2 x (h + 1) / 2 image adds, from 0, the
 * source texels in row order) until the image is 1 x 1. `img` (w x h x n) is
 * overwritten; out[n] receives the sums. */
static void sum_image(float* img, uint32_t w, uint32_t h, uint32_t n, float* out) {
    while (w > 1 || h > 1) {
        const uint32_t ow = (w + 1) / 2, oh = (h + 1) / 2;
        float* y = (float*)calloc((size_t)ow * oh * n, sizeof(float));
        for (uint32_t py = 0; py < h; py++) {
            for (uint32_t px = 0; px < w; px++) {
                const size_t si = ((size_t)py * w + px) * n;
                const size_t di = ((size_t)(py / 2) * ow + px / 2) * n;
                for (uint32_t c = 0; c < n; c++) y[di + c] += img[si + c];
            }
        }
        memcpy(img, y, sizeof(float) * (size_t)ow * oh * n);
        free(y);
        w = ow;
        h = oh;
    }
    for (uint32_t c = 0; c < n; c++) out[c] = img[c];
}

/* SumPixelWise over scalars (f_ops.cpp:893-950): groups of at most four,
 * each added from 0 in order (a lone entry passed up), until one is left. */
static float sum_pixelwise(float* v, uint32_t n) {
    while (n > 1) {
        uint32_t m = 0;
        for (uint32_t i = 0; i < n; i += 4) {
            const uint32_t k = n - i < 4 ? n - i : 4;
            if (k == 1) {
                v[m++] = v[i];
            } else {
                float acc = 0.f;
                for (uint32_t j = 0; j < k; j++) acc += v[i + j];
                v[m++] = acc;
            }
        }
        n = m;
    }
    return v[0];
}

int or_pbr_fit(const float* pos, const float* normal, uint32_t n_verts, const float* uv,
               const float* faces, uint32_t n_faces, const float* mvps, const float* frames,
               const float* light, uint32_t n_views, uint32_t screen_px, uint32_t tex_w,
               uint32_t tex_h, uint32_t env_w, uint32_t env_h, uint32_t levels,
               const float* gt_albedo, const float* gt_mr, const float* gt_env,
               const float* albedo0, const float* mr0, const float* env0, float lr,
               uint32_t iters, float* out_albedo, float* out_mr, float* out_env, float* out_loss,
               float* out_g_albedo0, float* out_g_mr0, float* out_g_env0, float* out_pred0,
               float* out_target0, float* out_mask0) {
    if (levels < 2 || levels > 16 || n_views == 0 || n_views > 64) return -1;
    const uint32_t S = screen_px;
    const size_t px = (size_t)S * S, ntx = (size_t)tex_w * tex_h, nev = (size_t)env_w * env_h;
    const uint32_t lutw = 256, luth = 256;
    float* lut = (float*)malloc(sizeof(float) * lutw * luth * 2);
    or_brdf_lut(lutw, luth, 512, lut);

    /* static per-view G-buffer and inverse-UV tables */
    Gpx* gb = (Gpx*)calloc(px * n_views, sizeof(Gpx));
    float* g_uv = (float*)calloc(px * n_views * 2, sizeof(float));
    float* inv = (float*)calloc(ntx * n_views * 4, sizeof(float));
    float* clip = (float*)malloc(sizeof(float) * n_verts * 4);
    float* attr = (float*)malloc(sizeof(float) * n_verts * 4);
    float* uvh = (float*)malloc(sizeof(float) * n_verts * 4);
    float* uvc = (float*)malloc(sizeof(float) * n_verts * 4);
    float* r4 = (float*)malloc(sizeof(float) * px * 4);
    float* r3n = (float*)malloc(sizeof(float) * px * 3);
    float* r3p = (float*)malloc(sizeof(float) * px * 3);
    for (uint32_t i = 0; i < n_verts; i++) {
        uvh[i * 4 + 0] = uv[i * 2 + 0];
        uvh[i * 4 + 1] = uv[i * 2 + 1];
        uvh[i * 4 + 2] = 1.f;
        uvh[i * 4 + 3] = 1.f;
    }
    or_uv_as_clip(uv, n_verts, uvc);
    const V3 lpos = v3(light[0], light[1], light[2]);
    for (uint32_t view = 0; view < n_views; view++) {
        const float* mv = mvps + 16 * view;
        for (uint32_t i = 0; i < n_verts; i++) {
            const float p[4] = {pos[i * 3 + 0], pos[i * 3 + 1], pos[i * 3 + 2], 1.f};
            for (int row = 0; row < 4; row++) {
                float acc = 0.f;
                for (int k = 0; k < 4; k++) acc += mv[k * 4 + row] * p[k];
                clip[i * 4 + row] = acc;
            }
        }
        or_rasterize(clip, n_verts, uvh, 4, faces, n_faces, S, S, r4);
        or_rasterize(clip, n_verts, normal, 3, faces, n_faces, S, S, r3n);
        or_rasterize(clip, n_verts, pos, 3, faces, n_faces, S, S, r3p);
        or_screen_attr(clip, n_verts, S, S, attr);
        or_rasterize(uvc, n_verts, attr, 4, faces, n_faces, tex_w, tex_h, inv + ntx * 4 * view);
        const float* fr = frames + 12 * view;
        const V3 cam = v3(fr[0], fr[1], fr[2]), fwd = v3(fr[3], fr[4], fr[5]);
        const V3 right = v3(fr[6], fr[7], fr[8]), up = v3(fr[9], fr[10], fr[11]);
        for (uint32_t y = 0; y < S; y++) {
            for (uint32_t x = 0; x < S; x++) {
                const size_t p = (size_t)y * S + x;
                Gpx* g = &gb[view * px + p];
                g->u = r4[p * 4 + 0];
                g->v = r4[p * 4 + 1];
                g->mask = r4[p * 4 + 2];
                g_uv[(view * px + p) * 2 + 0] = g->u;
                g_uv[(view * px + p) * 2 + 1] = g->v;
                const V3 gn = v3(r3n[p * 3 + 0], r3n[p * 3 + 1], r3n[p * 3 + 2]);
                const V3 gp = v3(r3p[p * 3 + 0], r3p[p * 3 + 1], r3p[p * 3 + 2]);
                const V3 n = safe_normalize(gn);
                const V3 vv = safe_normalize(v3(cam.x - gp.x, cam.y - gp.y, cam.z - gp.z));
                const V3 tl = v3(lpos.x - gp.x, lpos.y - gp.y, lpos.z - gp.z);
                const V3 l = safe_normalize(tl);
                const V3 h = safe_normalize(v3(vv.x + l.x, vv.y + l.y, vv.z + l.z));
                g->n = n;
                g->view = vv;
                g->ndv = maxf(dot3(n, vv), 1e-4f);
                g->dist2 = maxf(dot3(tl, tl), 1e-4f);
                g->ndl = maxf(dot3(n, l), 0.f);
                g->ndh = maxf(dot3(n, h), 0.f);
                g->vdh = maxf(dot3(vv, h), 0.f);
                /* Reflect(-v, n) = I - (2 dot(n, I)) n */
                const V3 I = v3(-vv.x, -vv.y, -vv.z);
                const float t2 = 2.f * dot3(n, I);
                g->refl = v3(I.x - t2 * n.x, I.y - t2 * n.y, I.z - t2 * n.z);
                /* background ray through the pixel centre */
                const float ndc_x = ((float)x + 0.5f) * (2.f / (float)S) - 1.f;
                const float ndc_y = ((float)y + 0.5f) * (2.f / (float)S) - 1.f;
                g->ray = v3(fwd.x + right.x * ndc_x - up.x * ndc_y,
                            fwd.y + right.y * ndc_x - up.y * ndc_y,
                            fwd.z + right.z * ndc_x - up.z * ndc_y);
            }
        }
    }
    free(clip);
    free(attr);
    free(uvh);
    free(uvc);
    free(r4);
    free(r3n);
    free(r3p);

    IblMaps gt_maps, maps;
    ibl_layout(&gt_maps, env_w, env_h, levels);
    ibl_layout(&maps, env_w, env_h, levels);
    ibl_build(&gt_maps, gt_env);
    ShadeCtx sc;
    ShadeOut so;
    sc.lut = lut;
    sc.lutw = lutw;
    sc.luth = luth;
    sc.tw = tex_w;
    sc.th = tex_h;
    sc.light_col = v3(light[3], light[4], light[5]);
    /* static target (mapped) */
    float* target = (float*)malloc(sizeof(float) * px * n_views * 3);
    sc.albedo = gt_albedo;
    sc.mr = gt_mr;
    sc.env = gt_env;
    sc.maps = &gt_maps;
    sc.irr = gt_maps.irr;
    sc.pref = gt_maps.pref;
    for (size_t p = 0; p < px * n_views; p++) {
        shade_px(&sc, &gb[p], NULL, &so);
        for (int c = 0; c < 3; c++) target[p * 3 + c] = so.hdr[c] / (so.hdr[c] + 1.f);
    }
    if (out_target0) memcpy(out_target0, target, sizeof(float) * px * n_views * 3);
    if (out_mask0) {
        for (size_t p = 0; p < px * n_views; p++) out_mask0[p] = gb[p].mask;
    }

    float* alb = (float*)malloc(sizeof(float) * ntx * 3);
    float* mrt = (float*)malloc(sizeof(float) * ntx * 3);
    float* env = (float*)malloc(sizeof(float) * nev * 3);
    memcpy(alb, albedo0, sizeof(float) * ntx * 3);
    memcpy(mrt, mr0, sizeof(float) * ntx * 3);
    memcpy(env, env0, sizeof(float) * nev * 3);
    float* st_m[3] = {(float*)calloc(ntx * 3, 4), (float*)calloc(ntx * 3, 4),
                      (float*)calloc(nev * 3, 4)};
    float* st_v[3] = {(float*)calloc(ntx * 3, 4), (float*)calloc(ntx * 3, 4),
                      (float*)calloc(nev * 3, 4)};
    float* gya = (float*)malloc(sizeof(float) * px * 3);
    float* gym = (float*)malloc(sizeof(float) * px * 3);
    float* gt = (float*)malloc(sizeof(float) * ntx * 3);
    float* g_alb = (float*)malloc(sizeof(float) * ntx * 3);
    float* g_mr = (float*)malloc(sizeof(float) * ntx * 3);
    float* g_env = (float*)malloc(sizeof(float) * nev * 3);
    const size_t npref = maps.loff[levels - 1] + (size_t)maps.lw[levels - 1] * maps.lh[levels - 1] * 3;
    float* g_irr = (float*)malloc(sizeof(float) * maps.iw * maps.ih * 3);
    float* g_pref = (float*)malloc(sizeof(float) * npref);
    float* tmp = (float*)malloc(sizeof(float) * (nev > 8192 ? nev : 8192) * 3);
    /* per-view per-pixel sample gradients and directions for the map VJPs */
    float* gy_irr = (float*)malloc(sizeof(float) * px * 3);
    float* gy_bg = (float*)malloc(sizeof(float) * px * 3);
    float* gy_pref = (float*)malloc(sizeof(float) * px * 3 * levels);
    float* dn = (float*)malloc(sizeof(float) * px * 3);
    float* dr = (float*)malloc(sizeof(float) * px * 3);
    float* dy = (float*)malloc(sizeof(float) * px * 3);
    const float inv_n = 1.f / ((float)S * (float)S * 3.f);
    float* adiff = (float*)malloc(sizeof(float) * px * 3);  /* |diff| image of a view */
    float vloss[64];
    float t_state = 0.f;
    for (uint32_t it = 0; it < iters; it++) {
        ibl_build(&maps, env);
        sc.albedo = alb;
        sc.mr = mrt;
        sc.env = env;
        sc.maps = &maps;
        sc.irr = maps.irr;
        sc.pref = maps.pref;
        memset(g_alb, 0, sizeof(float) * ntx * 3);
        memset(g_mr, 0, sizeof(float) * ntx * 3);
        memset(g_env, 0, sizeof(float) * nev * 3);
        memset(g_irr, 0, sizeof(float) * maps.iw * maps.ih * 3);
        memset(g_pref, 0, sizeof(float) * npref);
        for (uint32_t view = 0; view < n_views; view++) {
            for (size_t p = 0; p < px; p++) {
                const size_t q = view * px + p;
                shade_px(&sc, &gb[q], NULL, &so);
                float gh[3];
                for (int c = 0; c < 3; c++) {
                    const float hdr = so.hdr[c];
                    const float mapped = hdr / (hdr + 1.f);
                    if (it == 0 && out_pred0) out_pred0[q * 3 + c] = mapped;
                    const float diff = target[q * 3 + c] - mapped;
                    adiff[p * 3 + c] = fabsf(diff);
                    const float sg = (float)((diff > 0.f) - (diff < 0.f));
                    const float gmp = -(inv_n * sg);
                    gh[c] = gmp / (hdr + 1.f) - gmp * hdr / ((hdr + 1.f) * (hdr + 1.f));
                }
                shade_px(&sc, &gb[q], gh, &so);
                for (int c = 0; c < 3; c++) {
                    gya[p * 3 + c] = so.g_albedo[c];
                    gym[p * 3 + c] = so.g_mr[c];
                    gy_irr[p * 3 + c] = so.g_irr[c];
                    gy_bg[p * 3 + c] = so.g_bg[c];
                    for (uint32_t i = 0; i < levels; i++) {
                        gy_pref[(i * px + p) * 3 + c] = so.g_pref[i][c];
                    }
                }
                dn[p * 3 + 0] = so.n.x;
                dn[p * 3 + 1] = so.n.y;
                dn[p * 3 + 2] = so.n.z;
                dr[p * 3 + 0] = so.refl.x;
                dr[p * 3 + 1] = so.refl.y;
                dr[p * 3 + 2] = so.refl.z;
                dy[p * 3 + 0] = so.ray.x;
                dy[p * 3 + 1] = so.ray.y;
                dy[p * 3 + 2] = so.ray.z;
            }
            /* the view's loss: Mean = CompSum(Sum(|diff|)) * inv_n
             * (f_ops.cpp:743-770, 1045-1050) */
            float ssum[3];
            sum_image(adiff, S, S, 3, ssum);
            float cs = 0.f;
            for (int c = 0; c < 3; c++) cs += ssum[c];
            vloss[view] = cs * inv_n;
            /* texture gradients: inverse-UV gathers */
            const float* ivv = inv + ntx * 4 * view;
            const float* uvv = g_uv + px * 2 * view;
            or_gather_inv_uv_bilinear(gya, 3, S, S, ivv, tex_w, tex_h, uvv, gt);
            for (size_t i = 0; i < ntx * 3; i++) g_alb[i] += gt[i];
            or_gather_inv_uv_bilinear(gym, 3, S, S, ivv, tex_w, tex_h, uvv, gt);
            for (size_t i = 0; i < ntx * 3; i++) g_mr[i] += gt[i];
            /* map gradients: EquirectSample VJPs */
            or_equirect_sample(NULL, maps.iw, maps.ih, 3, dn, S, S, gy_irr, tmp);
            for (size_t i = 0; i < (size_t)maps.iw * maps.ih * 3; i++) g_irr[i] += tmp[i];
            for (uint32_t i = 0; i < levels; i++) {
                or_equirect_sample(NULL, maps.lw[i], maps.lh[i], 3, dr, S, S,
                                   gy_pref + (size_t)i * px * 3, tmp);
                for (size_t j = 0; j < (size_t)maps.lw[i] * maps.lh[i] * 3; j++) {
                    g_pref[maps.loff[i] + j] += tmp[j];
                }
            }
            or_equirect_sample(NULL, env_w, env_h, 3, dy, S, S, gy_bg, tmp);
            for (size_t i = 0; i < nev * 3; i++) g_env[i] += tmp[i];
        }
        ibl_backward(&maps, g_irr, g_pref, g_env);
        const float loss = sum_pixelwise(vloss, n_views);
        if (out_loss) out_loss[it] = loss;
        if (it == 0) {
            if (out_g_albedo0) memcpy(out_g_albedo0, g_alb, sizeof(float) * ntx * 3);
            if (out_g_mr0) memcpy(out_g_mr0, g_mr, sizeof(float) * ntx * 3);
            if (out_g_env0) memcpy(out_g_env0, g_env, sizeof(float) * nev * 3);
        }
        /* Adam (shared step counter), clamps as in the examples */
        const float tn = t_state + 1.f;
        const float bc1 = 1.f - powf(0.9f, tn), bc2 = 1.f - powf(0.999f, tn);
        float* xs[3] = {alb, mrt, env};
        float* gs[3] = {g_alb, g_mr, g_env};
        const size_t ns[3] = {ntx * 3, ntx * 3, nev * 3};
        for (int j = 0; j < 3; j++) {
            for (size_t i = 0; i < ns[j]; i++) {
                const float g = gs[j][i];
                const float mn = st_m[j][i] * 0.9f + g * (1.f - 0.9f);
                const float vn = st_v[j][i] * 0.999f + g * g * (1.f - 0.999f);
                const float step = (mn / bc1) / (sqrtf(vn / bc2) + 1e-8f) * lr;
                const float x = xs[j][i] - step;
                xs[j][i] = j < 2 ? (x < 0.f ? 0.f : (x > 1.f ? 1.f : x)) : (x < 0.f ? 0.f : x);
                st_m[j][i] = mn;
                st_v[j][i] = vn;
            }
        }
        t_state = tn;
    }
    if (out_albedo) memcpy(out_albedo, alb, sizeof(float) * ntx * 3);
    if (out_mr) memcpy(out_mr, mrt, sizeof(float) * ntx * 3);
    if (out_env) memcpy(out_env, env, sizeof(float) * nev * 3);
    ibl_free(&gt_maps);
    ibl_free(&maps);
    free(lut);
    free(gb);
    free(g_uv);
    free(inv);
    free(target);
    free(alb);
    free(mrt);
    free(env);
    for (int j = 0; j < 3; j++) {
        free(st_m[j]);
        free(st_v[j]);
    }
    free(adiff);
    free(gya);
    free(gym);
    free(gt);
    free(g_alb);
    free(g_mr);
    free(g_env);
    free(g_irr);
    free(g_pref);
    free(tmp);
    free(gy_irr);
    free(gy_bg);
    free(gy_pref);
    free(dn);
    free(dr);
    free(dy);
    return 0;
}
