// executor.hip -- DressiAD on one HIP device (include/dressi/dressi_ad.h;
// the reference's src/dressi_ad.cpp:24-696 is the behaviour it keeps).
//
// execStep walks the reference's ladder only as far as the last change
// requires (src/dressi_ad.cpp:280-530):
//   BACKWARD   BuildBackward(loss)
//   OPTIMIZER  the optimizer's update graph; copy-back pairs (optimizer
//              outputs are rebuilt here, addUpdate pairs persist)
//   TRAVERSE   the functions the roots need, in creation order; the leaves
//   SUBSTAGE   demand filter (static branches whose images are computed
//              are skipped: the reactive cache of src/pack/reactive.cpp:
//              10-68), then packing into steps
//   STAGE      step-level demand filter (the fast rebuild)
//   VULKAN     device buffers, step programs, and the captured hipGraph
// then runs the iteration: pending / fused uploads, one hipGraph launch
// (steps + end-of-frame copy-backs), fused downloads.
//
// Steps: with PackingMode::RSP every run of consecutive elementwise
// functions producing images of one size becomes ONE kernel, a per-pixel
// program over registers (the reference's fused substage: intermediate
// values never touch memory; images consumed outside the step, roots and
// copy-back sources are stored); the other ops run through the library's
// per-op entry points (include/dressi_hip.h). PackingMode::Naive gives every
// function its own step. Every op keeps the reference CPU kernel's float
// semantics, so results do not depend on the packing.
//
// A graph recognised as the reference's silhouette-fit example (HardSoftRas
// or AA) or as the texture fit (see route.h) runs on its fused plan instead.
#include <dlfcn.h>
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <functional>
#include <map>
#include <mutex>
#include <sstream>
#include <string>
#include <set>
#include <unordered_map>
#include <unordered_set>

#include "graph_ir.h"
#include "internal.h"
#include "libm_f32.h"
#include "route.h"

namespace dressi {

struct HipContext {
    dressi_ctx* ctx = nullptr;
    int device = 0;
    ~HipContext() {
        if (ctx) {
            dressi_ctx_destroy(ctx);
        }
    }
};

namespace {

void check(int rc, const char* what) {
    if (rc != DRESSI_OK) {
        throw DressiError(std::string(what) + ": " + dressi_last_error());
    }
}

void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        throw DressiError(std::string(what) + ": " + hipGetErrorString(e));
    }
}

// ---- fused elementwise stage ------------------------------------------------

constexpr int kMaxStepInstrs = 48;  // instructions of one fused program
constexpr int kMaxInputs = 4;

// Where an instruction input comes from
enum : int { kSrcReg = 0, kSrcBuf = 1, kSrcImm = 2 };

struct FInput {
    int src;
    uint32_t idx;  // register, buffer slot or immediate offset
    uint32_t nc;   // components
    uint32_t uniform;
};

struct FInstr {
    int op;
    uint32_t n_in;
    uint32_t ny;
    uint32_t a0;
    int out_slot;  // buffer slot to store to, -1: register only
    uint32_t reg;  // register (LDS slot) of the result
    FInput in[kMaxInputs];
};

struct FProgram {
    const FInstr* code;
    uint32_t n;
    uint32_t n_regs;  // LDS register slots
    size_t n_px;
    float* const* bufs;  // slot -> device buffer
    const float* imm;
};

__device__ __forceinline__ float std_min(float a, float b) { return b < a ? b : a; }
__device__ __forceinline__ float std_max(float a, float b) { return a < b ? b : a; }

// component i (0..3) of a 4-vector without run-time indexing (which would
// place the array in private memory)
__device__ __forceinline__ float sel4(const float (&a)[4], uint32_t i) {
    return i == 0 ? a[0] : (i == 1 ? a[1] : (i == 2 ? a[2] : a[3]));
}

// one elementwise op on one pixel: `v[i][c]` = component c of input i
// (1-component inputs replicated), the reference's CPU float semantics.
// Every array index is a compile-time constant (unrolled loops with
// predicates), so v and y stay in registers.
__device__ __forceinline__ void ew_eval(Op op, uint32_t n_in, const uint32_t (&nc)[kMaxInputs],
                                        const float (&v)[kMaxInputs][4], uint32_t ny,
                                        uint32_t a0, float (&y)[4]) {
    switch (op) {
        case Op::kCompose: {
            uint32_t o = 0;
#pragma unroll
            for (uint32_t i = 0; i < kMaxInputs; i++) {
#pragma unroll
                for (uint32_t c = 0; c < 4; c++) {
                    if (i < n_in && c < nc[i]) {
#pragma unroll
                        for (uint32_t j = 0; j < 4; j++) {
                            if (o == j) {
                                y[j] = v[i][c];
                            }
                        }
                        o++;
                    }
                }
            }
            return;
        }
        case Op::kExtract:
#pragma unroll
            for (uint32_t c = 0; c < 4; c++) {
                if (c < ny) {
                    y[c] = sel4(v[0], a0 + c);
                }
            }
            return;
        case Op::kDot: {
            float acc = 0.f;
#pragma unroll
            for (uint32_t c = 0; c < 4; c++) {
                if (c < nc[0]) {
                    acc += v[0][c] * v[1][c];
                }
            }
            y[0] = acc;
            return;
        }
        case Op::kCompSum: {
            float acc = 0.f;
#pragma unroll
            for (uint32_t c = 0; c < 4; c++) {
                if (c < nc[0]) {
                    acc += v[0][c];
                }
            }
            y[0] = acc;
            return;
        }
        case Op::kLength: {
            float acc = 0.f;
#pragma unroll
            for (uint32_t c = 0; c < 4; c++) {
                if (c < nc[0]) {
                    acc += v[0][c] * v[0][c];
                }
            }
            y[0] = sqrtf(acc);
            return;
        }
        case Op::kNormalize: {
            float acc = 0.f;
#pragma unroll
            for (uint32_t c = 0; c < 4; c++) {
                if (c < nc[0]) {
                    acc += v[0][c] * v[0][c];
                }
            }
            const float inv = 1.f / sqrtf(acc);
#pragma unroll
            for (uint32_t c = 0; c < 4; c++) {
                if (c < ny) {
                    y[c] = v[0][c] * inv;
                }
            }
            return;
        }
        case Op::kCross:
            y[0] = v[0][1] * v[1][2] - v[0][2] * v[1][1];
            y[1] = v[0][2] * v[1][0] - v[0][0] * v[1][2];
            y[2] = v[0][0] * v[1][1] - v[0][1] * v[1][0];
            return;
        default:
            break;
    }
#pragma unroll
    for (uint32_t c = 0; c < 4; c++) {
        if (c >= ny) {
            continue;
        }
        const float a = v[0][c];
        const float b = n_in > 1 ? v[1][c] : 0.f;
        const float t = n_in > 2 ? v[2][c] : 0.f;
        float r = 0.f;
        switch (op) {
            case Op::kAdd: r = a + b; break;
            case Op::kSub: r = a - b; break;
            case Op::kMul: r = a * b; break;
            case Op::kDiv: r = a / b; break;
            case Op::kNeg: r = -a; break;
            case Op::kSin: r = sinf(a); break;
            case Op::kCos: r = cosf(a); break;
            case Op::kTan: r = tanf(a); break;
            case Op::kAsin: r = asinf(a); break;
            case Op::kAcos: r = libm::acosf(a); break;
            case Op::kAtan: r = libm::atanf(a); break;
            case Op::kAtan2: r = libm::atan2f(a, b); break;
            case Op::kExp: r = libc_expf(a); break;
            case Op::kExp2: r = exp2f(a); break;
            case Op::kLog: r = logf(a); break;
            case Op::kLog2: r = log2f(a); break;
            case Op::kSqrt: r = sqrtf(a); break;
            case Op::kInvSqrt: r = 1.f / sqrtf(a); break;
            case Op::kAbs: r = fabsf(a); break;
            case Op::kSign: r = (float)((a > 0.f) - (a < 0.f)); break;
            case Op::kFloor: r = floorf(a); break;
            case Op::kFract: r = a - floorf(a); break;
            case Op::kMod: r = a - b * floorf(a / b); break;
            case Op::kPow: r = (b == 5.f && a >= 0.f && a <= 1.f) ? libm::pow5f(a) : powf(a, b); break;
            case Op::kMax: r = std_max(a, b); break;
            case Op::kMin: r = std_min(a, b); break;
            case Op::kClamp: r = std_min(std_max(a, b), t); break;
            case Op::kMix: r = a + (b - a) * t; break;
            case Op::kStep: r = b < a ? 0.f : 1.f; break;
            case Op::kSmoothStep: {
                const float s = std_min(std_max((t - a) / (b - a), 0.f), 1.f);
                r = s * s * (3.f - 2.f * s);
                break;
            }
            case Op::kSigmoid: r = 1.f / (1.f + libc_expf(-a)); break;
            case Op::kLess: r = (float)(a < b); break;
            case Op::kLessEq: r = (float)(a <= b); break;
            case Op::kGreater: r = (float)(a > b); break;
            case Op::kGreaterEq: r = (float)(a >= b); break;
            case Op::kCopy: r = a; break;
            case Op::kSumPw: {
                float acc = 0.f;
#pragma unroll
                for (uint32_t i = 0; i < kMaxInputs; i++) {
                    if (i < n_in) {
                        acc += v[i][c];
                    }
                }
                r = acc;
                break;
            }
            default: break;
        }
        y[c] = r;
    }
}

// One fused stage: every thread runs the program on its pixel.
// The program's registers live in LDS (P.n_regs x kFusedThreads float4, a
// thread's own slots only; slots reused once their value is dead): indexed
// at run time they would otherwise be private memory.
constexpr uint32_t kFusedThreads = 64;
__global__ __launch_bounds__(kFusedThreads) void k_fused(FProgram P) {
    extern __shared__ float4 sreg[];  // [register][thread]
    const size_t p = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= P.n_px) {
        return;
    }
    // the program and the buffer table are the same for every lane: read
    // through the constant address space (scalar loads)
    typedef const __attribute__((address_space(4))) uint32_t* UniformWords;
    typedef const __attribute__((address_space(4))) uint64_t* UniformPtrs;
    const auto buf_at = [&](uint32_t k) {
        return (float*)((UniformPtrs)P.bufs)[k];
    };
    for (uint32_t i = 0; i < P.n; i++) {
        constexpr int kWords = (int)(sizeof(FInstr) / 4);
        union {
            FInstr f;
            uint32_t w[kWords];
        } u;
        const UniformWords src = (UniformWords)(P.code + i);
#pragma unroll
        for (int k = 0; k < kWords; k++) {
            u.w[k] = src[k];
        }
        const FInstr ins = u.f;
        float v[kMaxInputs][4];
        uint32_t nc[kMaxInputs];
#pragma unroll
        for (uint32_t k = 0; k < kMaxInputs; k++) {
            nc[k] = 0;
#pragma unroll
            for (uint32_t c = 0; c < 4; c++) {
                v[k][c] = 0.f;
            }
            if (k >= ins.n_in) {
                continue;
            }
            const FInput in = ins.in[k];
            nc[k] = in.nc;
            if (in.src == kSrcReg) {
                const float4 r = sreg[in.idx * kFusedThreads + threadIdx.x];  // slot
                const float rc[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
                for (uint32_t c = 0; c < 4; c++) {
                    v[k][c] = sel4(rc, in.nc == 1 ? 0 : (c < in.nc ? c : 0));
                }
            } else {
                const float* src = in.src == kSrcBuf
                                           ? buf_at(in.idx) + (in.uniform ? 0 : p * in.nc)
                                           : P.imm + in.idx;
#pragma unroll
                for (uint32_t c = 0; c < 4; c++) {
                    v[k][c] = src[in.nc == 1 ? 0 : (c < in.nc ? c : 0)];
                }
            }
        }
        float y[4] = {0.f, 0.f, 0.f, 0.f};
        ew_eval((Op)ins.op, ins.n_in, nc, v, ins.ny, ins.a0, y);
        sreg[ins.reg * kFusedThreads + threadIdx.x] = make_float4(y[0], y[1], y[2], y[3]);
        if (ins.out_slot >= 0) {
            float* dst = buf_at((uint32_t)ins.out_slot) + p * ins.ny;
#pragma unroll
            for (uint32_t c = 0; c < 4; c++) {
                if (c < ins.ny) {
                    dst[c] = y[c];
                }
            }
        }
    }
}

__global__ __launch_bounds__(64) void k_fill(float* y, uint32_t n, float v0, float v1, float v2,
                                             float v3) {
    const uint32_t c = threadIdx.x;
    if (c < n) {
        y[c] = c == 0 ? v0 : c == 1 ? v1 : c == 2 ? v2 : v3;
    }
}

// Elementwise ops on matrix-typed images (more than 4 components): one
// thread per (pixel, component); 1-component and {1,1} inputs broadcast
struct WideIn {
    const float* p;
    uint32_t nc;
    uint32_t uniform;
};
struct WideArgs {
    int op;
    uint32_t n_in, ny;
    size_t n_px;
    WideIn in[kMaxInputs];
    float* y;
};

__global__ __launch_bounds__(256) void k_wide(WideArgs A) {
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= A.n_px * A.ny) {
        return;
    }
    const size_t p = q / A.ny;
    const uint32_t c = (uint32_t)(q % A.ny);
    float v[kMaxInputs];
    for (uint32_t k = 0; k < A.n_in; k++) {
        const WideIn in = A.in[k];
        v[k] = in.p[(in.uniform ? 0 : p * in.nc) + (in.nc == 1 ? 0 : c)];
    }
    float r = 0.f;
    switch ((Op)A.op) {
        case Op::kAdd: r = v[0] + v[1]; break;
        case Op::kSub: r = v[0] - v[1]; break;
        case Op::kMul: r = v[0] * v[1]; break;
        case Op::kDiv: r = v[0] / v[1]; break;
        case Op::kNeg: r = -v[0]; break;
        case Op::kCopy: r = v[0]; break;
        case Op::kSumPw: {
            float acc = 0.f;
            for (uint32_t k = 0; k < A.n_in; k++) {
                acc += v[k];
            }
            r = acc;
            break;
        }
        default: break;
    }
    A.y[q] = r;
}

// Reduce2x2Sum: each output pixel sums its 2x2 source block in row order
// from 0 (the reference CPU kernel's accumulation order).
__global__ __launch_bounds__(256) void k_reduce2x2(const float* x, uint32_t sw, uint32_t sh,
                                                   uint32_t nc, uint32_t ow, uint32_t oh,
                                                   float* y) {
    const uint32_t q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= ow * oh) {
        return;
    }
    const uint32_t ox = q % ow, oy = q / ow;
    for (uint32_t c = 0; c < nc; c++) {
        float acc = 0.f;
        for (uint32_t dy = 0; dy < 2; dy++) {
            for (uint32_t dx = 0; dx < 2; dx++) {
                const uint32_t sx = 2 * ox + dx, sy = 2 * oy + dy;
                if (sx < sw && sy < sh) {
                    acc += x[((size_t)sy * sw + sx) * nc + c];
                }
            }
        }
        y[(size_t)q * nc + c] = acc;
    }
}

__global__ __launch_bounds__(256) void k_upsample2x(const float* x, uint32_t sw, uint32_t nc,
                                                    uint32_t ow, uint32_t oh, float* y) {
    const uint32_t q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= ow * oh) {
        return;
    }
    const uint32_t ox = q % ow, oy = q / ow;
    for (uint32_t c = 0; c < nc; c++) {
        y[(size_t)q * nc + c] = x[((size_t)(oy / 2) * sw + ox / 2) * nc + c];
    }
}

__global__ __launch_bounds__(256) void k_screen_coord(uint32_t w, uint32_t h, float* y) {
    const uint32_t q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= w * h) {
        return;
    }
    y[2 * (size_t)q + 0] = (float)(q % w) + 0.5f;
    y[2 * (size_t)q + 1] = (float)(q / w) + 0.5f;
}

// SumAll (f_ops.cpp:1087-1149): above 256 pixels, 64 strided partial sums in
// double (pixels p, p + 64, ..., components in order), each rounded to
// float; then the double sum of those (or of every value) rounded once
__global__ __launch_bounds__(64) void k_sum_all(const float* x, size_t n_px, uint32_t nc,
                                                float* y) {
    __shared__ float part[64];
    const uint32_t t = threadIdx.x;
    if (n_px > 256) {
        double s = 0.0;
        for (size_t i = t; i < n_px; i += 64) {
            for (uint32_t c = 0; c < nc; c++) {
                s += (double)x[i * nc + c];
            }
        }
        part[t] = (float)s;
        __syncthreads();
        if (t == 0) {
            double a = 0.0;
            for (int k = 0; k < 64; k++) {
                a += (double)part[k];
            }
            y[0] = (float)a;
        }
    } else if (t == 0) {
        double a = 0.0;
        for (size_t i = 0; i < n_px * nc; i++) {
            a += (double)x[i];
        }
        y[0] = (float)a;
    }
}

// PixelFetch / TileFetch (f_ops.cpp:1826-1888): row = uint(int64(v + 0.5))
__global__ __launch_bounds__(64) void k_pixel_fetch(const float* tex, uint32_t w, uint32_t h,
                                                    uint32_t nc, uint32_t x, const float* row,
                                                    float* y, uint32_t* err) {
    const uint32_t r = (uint32_t)(int64_t)(row[0] + 0.5f);
    if (r >= h) {
        if (threadIdx.x == 0) {
            atomicOr(err, 0x200u);
        }
        return;
    }
    if (threadIdx.x < nc) {
        y[threadIdx.x] = tex[((size_t)r * w + x) * nc + threadIdx.x];
    }
}

__global__ __launch_bounds__(256) void k_tile_fetch(const float* atlas, uint32_t w, uint32_t h,
                                                    uint32_t nc, uint32_t tile_h,
                                                    const float* idx, float* y, uint32_t* err) {
    const size_t n = (size_t)w * tile_h * nc;
    const uint32_t t = (uint32_t)(int64_t)(idx[0] + 0.5f);
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= n) {
        return;
    }
    if (t >= h / tile_h) {
        if (q == 0) {
            atomicOr(err, 0x200u);
        }
        return;
    }
    y[q] = atlas[(size_t)t * n + q];
}

// Per-pixel matrix ops, column-major (f_ops.cpp:767-870)
__global__ __launch_bounds__(256) void k_matrix(int op, const float* a, uint32_t a_uni,
                                                const float* b, uint32_t b_uni, uint32_t dim,
                                                uint32_t vec_rhs, size_t n_px, float* y) {
    const size_t p = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= n_px) {
        return;
    }
    const uint32_t dd = dim * dim;
    if ((Op)op == Op::kMatMul) {
        const float* m = a + (a_uni ? 0 : p * dd);
        if (vec_rhs) {
            const float* r = b + (b_uni ? 0 : p * dim);
            for (uint32_t row = 0; row < dim; row++) {
                float acc = 0.f;
                for (uint32_t col = 0; col < dim; col++) {
                    acc += m[col * dim + row] * r[col];
                }
                y[p * dim + row] = acc;
            }
        } else {
            const float* r = b + (b_uni ? 0 : p * dd);
            for (uint32_t col = 0; col < dim; col++) {
                for (uint32_t row = 0; row < dim; row++) {
                    float acc = 0.f;
                    for (uint32_t k = 0; k < dim; k++) {
                        acc += m[k * dim + row] * r[col * dim + k];
                    }
                    y[p * dd + col * dim + row] = acc;
                }
            }
        }
    } else if ((Op)op == Op::kTranspose) {
        const float* m = a + (a_uni ? 0 : p * dd);
        for (uint32_t col = 0; col < dim; col++) {
            for (uint32_t row = 0; row < dim; row++) {
                y[p * dd + col * dim + row] = m[row * dim + col];
            }
        }
    } else {
        const float* u = a + (a_uni ? 0 : p * dim);
        const float* w = b + (b_uni ? 0 : p * dim);
        for (uint32_t c = 0; c < dim; c++) {
            for (uint32_t r = 0; r < dim; r++) {
                y[p * dd + c * dim + r] = u[r] * w[c];
            }
        }
    }
}

// VertexNeighborMean (f_ops.cpp:1983-2029)
__global__ __launch_bounds__(256) void k_vertex_neighbor_mean(const float* pos, uint32_t nv,
                                                              const float* adj, uint32_t deg,
                                                              float* out, uint32_t* err) {
    const uint32_t v = blockIdx.x * blockDim.x + threadIdx.x;
    if (v >= nv) {
        return;
    }
    float mean[3] = {0.f, 0.f, 0.f};
    uint32_t count = 0;
    for (uint32_t d = 0; d < deg; d++) {
        const float a = adj[(size_t)d * nv + v];
        if (a < -0.5f) {
            continue;
        }
        const size_t n = (size_t)(int64_t)(a + 0.5f);
        if (n >= nv) {
            atomicOr(err, 0x200u);
            continue;
        }
        for (int c = 0; c < 3; c++) {
            mean[c] += pos[n * 3 + c];
        }
        count++;
    }
    for (int c = 0; c < 3; c++) {
        out[(size_t)v * 3 + c] = count > 0 ? mean[c] / (float)count : pos[(size_t)v * 3 + c];
    }
}

// vertex ids of face f, false (error bit set) when one is out of range
__device__ __forceinline__ bool face_ids(const float* faces, uint32_t f, uint32_t nv,
                                         uint32_t idx[3], uint32_t* err) {
    for (int k = 0; k < 3; k++) {
        idx[k] = (uint32_t)(int64_t)(faces[(size_t)f * 3 + k] + 0.5f);
        if (idx[k] >= nv) {
            atomicOr(err, 0x200u);
            return false;
        }
    }
    return true;
}

__device__ __forceinline__ bool face_cross(const float* pos, uint32_t nv, const float* faces,
                                           uint32_t f, float c[3], uint32_t* err) {
    uint32_t idx[3];
    if (!face_ids(faces, f, nv, idx, err)) {
        c[0] = c[1] = c[2] = 0.f;
        return false;
    }
    const float* p0 = pos + (size_t)idx[0] * 3;
    const float* p1 = pos + (size_t)idx[1] * 3;
    const float* p2 = pos + (size_t)idx[2] * 3;
    const float e1[3] = {p1[0] - p0[0], p1[1] - p0[1], p1[2] - p0[2]};
    const float e2[3] = {p2[0] - p0[0], p2[1] - p0[1], p2[2] - p0[2]};
    c[0] = e1[1] * e2[2] - e1[2] * e2[1];
    c[1] = e1[2] * e2[0] - e1[0] * e2[2];
    c[2] = e1[0] * e2[1] - e1[1] * e2[0];
    return true;
}

// NormalConsistencyFaceTerm (f_ops.cpp:2031-2098)
__global__ __launch_bounds__(256) void k_nc_face_term(const float* pos, uint32_t nv,
                                                      const float* faces, const float* fadj,
                                                      uint32_t nf, float* out, uint32_t* err) {
    const uint32_t f = blockIdx.x * blockDim.x + threadIdx.x;
    if (f >= nf) {
        return;
    }
    float g[3] = {0.f, 0.f, 0.f};
    float ca[3];
    face_cross(pos, nv, faces, f, ca, err);
    const float la = sqrtf(ca[0] * ca[0] + ca[1] * ca[1] + ca[2] * ca[2]);
    if (!(la < 1e-12f)) {
        const float na[3] = {ca[0] / la, ca[1] / la, ca[2] / la};
        for (int j = 0; j < 3; j++) {
            const float gv = fadj[(size_t)f * 3 + j];
            if (gv < -0.5f) {
                continue;
            }
            const uint32_t fb = (uint32_t)(int64_t)(gv + 0.5f);
            float cb[3];
            if (fb >= nf) {
                atomicOr(err, 0x200u);
                continue;
            }
            face_cross(pos, nv, faces, fb, cb, err);
            const float lb = sqrtf(cb[0] * cb[0] + cb[1] * cb[1] + cb[2] * cb[2]);
            if (lb < 1e-12f) {
                continue;
            }
            const float nb[3] = {cb[0] / lb, cb[1] / lb, cb[2] / lb};
            const float d = na[0] * nb[0] + na[1] * nb[1] + na[2] * nb[2];
            for (int c = 0; c < 3; c++) {
                g[c] += -(nb[c] - d * na[c]) / la;
            }
        }
    }
    for (int c = 0; c < 3; c++) {
        out[(size_t)f * 3 + c] = g[c];
    }
}

// NormalConsistencyVertexGrad (f_ops.cpp:2100-2181)
__global__ __launch_bounds__(256) void k_nc_vertex_grad(const float* term, const float* pos,
                                                        const float* faces, uint32_t nf,
                                                        const float* vf, uint32_t nv,
                                                        uint32_t deg, float* out, uint32_t* err) {
    const uint32_t v = blockIdx.x * blockDim.x + threadIdx.x;
    if (v >= nv) {
        return;
    }
    float acc[3] = {0.f, 0.f, 0.f};
    for (uint32_t d = 0; d < deg; d++) {
        const float fv = vf[(size_t)d * nv + v];
        if (fv < -0.5f) {
            continue;
        }
        const uint32_t f = (uint32_t)(int64_t)(fv + 0.5f);
        uint32_t idx[3];
        if (f >= nf) {
            atomicOr(err, 0x200u);
            continue;
        }
        if (!face_ids(faces, f, nv, idx, err)) {
            continue;
        }
        const float* p0 = pos + (size_t)idx[0] * 3;
        const float* p1 = pos + (size_t)idx[1] * 3;
        const float* p2 = pos + (size_t)idx[2] * 3;
        const float e1[3] = {p1[0] - p0[0], p1[1] - p0[1], p1[2] - p0[2]};
        const float e2[3] = {p2[0] - p0[0], p2[1] - p0[1], p2[2] - p0[2]};
        const float* g = term + (size_t)f * 3;
        const float g1[3] = {e2[1] * g[2] - e2[2] * g[1], e2[2] * g[0] - e2[0] * g[2],
                             e2[0] * g[1] - e2[1] * g[0]};
        const float g2[3] = {g[1] * e1[2] - g[2] * e1[1], g[2] * e1[0] - g[0] * e1[2],
                             g[0] * e1[1] - g[1] * e1[0]};
        for (int c = 0; c < 3; c++) {
            if (idx[1] == v) {
                acc[c] += g1[c];
            }
            if (idx[2] == v) {
                acc[c] += g2[c];
            }
            if (idx[0] == v) {
                acc[c] -= g1[c] + g2[c];
            }
        }
    }
    for (int c = 0; c < 3; c++) {
        out[(size_t)v * 3 + c] = acc[c];
    }
}

uint32_t blocks256(size_t n) { return (uint32_t)((n + 255) / 256); }

size_t n_floats(const VariableNode& n) {
    return (size_t)n.size.w * n.size.h * NumComponents(n.vtype);
}

}  // namespace

// ---- the executor ------------------------------------------------------------------

namespace {

// One launch group of the iteration: a fused elementwise program or one
// function through its kernel / entry point.
// ---- compiled fused programs ---------------------------------------------
// A fused program can also be compiled at run time (hipRTC) into a kernel
// of straight-line code: the same operations in the same order as ew_eval,
// the same device math (libc_expf, libm::*), built with the library's own
// floating-point flags, so its results are the interpreter's bit for bit.
// Programs are compiled per device, all new ones of a packing in one unit,
// and cached for the process by their text. Any failure falls back to the
// interpreter (as does DRESSI_NO_JIT=1).

std::string f32_lit(float v) {
    uint32_t u;
    std::memcpy(&u, &v, 4);
    char b[64];
    snprintf(b, sizeof b, "__builtin_bit_cast(float, 0x%08xu)", u);
    return b;
}

// The statements of one program: r<i>_<c> = component c of instruction i's
// result; B[k] the program's buffer table; p the pixel.
std::string jit_body(const std::vector<FInstr>& code, const std::vector<float>& imm,
                     bool* uses_libm) {
    std::ostringstream o;
    *uses_libm = false;
    for (size_t i = 0; i < code.size(); i++) {
        const FInstr& ins = code[i];
        const Op op = (Op)ins.op;
        // operand component c of input k
        auto v = [&](uint32_t k, uint32_t c) -> std::string {
            const FInput& in = ins.in[k];
            const uint32_t ci = in.nc == 1 ? 0 : (c < in.nc ? c : 0);
            std::ostringstream e;
            if (in.src == kSrcReg) {
                e << "r" << in.idx << "_" << ci;
            } else if (in.src == kSrcBuf) {
                if (in.uniform) {
                    e << "B[" << in.idx << "][" << ci << "]";
                } else {
                    e << "B[" << in.idx << "][p * " << in.nc << "ull + " << ci << "]";
                }
            } else {
                e << f32_lit(imm[in.idx + ci]);
            }
            return e.str();
        };
        std::string y[4] = {"0.f", "0.f", "0.f", "0.f"};
        o << "float r" << i << "_0, r" << i << "_1, r" << i << "_2, r" << i << "_3;\n{\n";
        auto acc_loop = [&](const std::string& init, uint32_t n,
                            const std::function<std::string(uint32_t)>& term) {
            o << "float acc = " << init << ";\n";
            for (uint32_t c = 0; c < n; c++) {
                o << "acc += " << term(c) << ";\n";
            }
        };
        switch (op) {
            case Op::kCompose: {
                uint32_t q = 0;
                for (uint32_t k = 0; k < ins.n_in; k++) {
                    for (uint32_t c = 0; c < ins.in[k].nc && q < 4; c++) {
                        y[q++] = v(k, c);
                    }
                }
                break;
            }
            case Op::kExtract:
                for (uint32_t c = 0; c < ins.ny && c < 4; c++) {
                    y[c] = v(0, std::min<uint32_t>(ins.a0 + c, 3));
                }
                break;
            case Op::kDot:
                acc_loop("0.f", ins.in[0].nc,
                         [&](uint32_t c) { return v(0, c) + " * " + v(1, c); });
                y[0] = "acc";
                break;
            case Op::kCompSum:
                acc_loop("0.f", ins.in[0].nc, [&](uint32_t c) { return v(0, c); });
                y[0] = "acc";
                break;
            case Op::kLength:
                acc_loop("0.f", ins.in[0].nc,
                         [&](uint32_t c) { return v(0, c) + " * " + v(0, c); });
                y[0] = "sqrtf(acc)";
                break;
            case Op::kNormalize:
                acc_loop("0.f", ins.in[0].nc,
                         [&](uint32_t c) { return v(0, c) + " * " + v(0, c); });
                o << "const float inv = 1.f / sqrtf(acc);\n";
                for (uint32_t c = 0; c < ins.ny && c < 4; c++) {
                    y[c] = v(0, c) + " * inv";
                }
                break;
            case Op::kCross:
                y[0] = v(0, 1) + " * " + v(1, 2) + " - " + v(0, 2) + " * " + v(1, 1);
                y[1] = v(0, 2) + " * " + v(1, 0) + " - " + v(0, 0) + " * " + v(1, 2);
                y[2] = v(0, 0) + " * " + v(1, 1) + " - " + v(0, 1) + " * " + v(1, 0);
                break;
            default:
                for (uint32_t c = 0; c < ins.ny && c < 4; c++) {
                    const std::string a = "(" + v(0, c) + ")";
                    const std::string b = ins.n_in > 1 ? "(" + v(1, c) + ")" : "0.f";
                    const std::string t = ins.n_in > 2 ? "(" + v(2, c) + ")" : "0.f";
                    std::string r;
                    switch (op) {
                        case Op::kAdd: r = a + " + " + b; break;
                        case Op::kSub: r = a + " - " + b; break;
                        case Op::kMul: r = a + " * " + b; break;
                        case Op::kDiv: r = a + " / " + b; break;
                        case Op::kNeg: r = "-" + a; break;
                        case Op::kSin: r = "sinf" + a; break;
                        case Op::kCos: r = "cosf" + a; break;
                        case Op::kTan: r = "tanf" + a; break;
                        case Op::kAsin: r = "asinf" + a; break;
                        case Op::kAcos: r = "dressi::libm::acosf" + a; *uses_libm = true; break;
                        case Op::kAtan: r = "dressi::libm::atanf" + a; *uses_libm = true; break;
                        case Op::kAtan2:
                            r = "dressi::libm::atan2f(" + a + ", " + b + ")";
                            *uses_libm = true;
                            break;
                        case Op::kExp: r = "dressi::libc_expf" + a; break;
                        case Op::kExp2: r = "exp2f" + a; break;
                        case Op::kLog: r = "logf" + a; break;
                        case Op::kLog2: r = "log2f" + a; break;
                        case Op::kSqrt: r = "sqrtf" + a; break;
                        case Op::kInvSqrt: r = "1.f / sqrtf" + a; break;
                        case Op::kAbs: r = "fabsf" + a; break;
                        case Op::kSign: r = "(float)((" + a + " > 0.f) - (" + a + " < 0.f))"; break;
                        case Op::kFloor: r = "floorf" + a; break;
                        case Op::kFract: r = a + " - floorf" + a; break;
                        case Op::kMod: r = a + " - " + b + " * floorf(" + a + " / " + b + ")"; break;
                        case Op::kPow:
                            r = "((" + b + " == 5.f && " + a + " >= 0.f && " + a +
                                " <= 1.f) ? dressi::libm::pow5f(" + a + ") : powf(" + a + ", " +
                                b + "))";
                            *uses_libm = true;
                            break;
                        case Op::kMax: r = "jit_max(" + a + ", " + b + ")"; break;
                        case Op::kMin: r = "jit_min(" + a + ", " + b + ")"; break;
                        case Op::kClamp: r = "jit_min(jit_max(" + a + ", " + b + "), " + t + ")"; break;
                        case Op::kMix: r = a + " + (" + b + " - " + a + ") * " + t; break;
                        case Op::kStep: r = "(" + b + " < " + a + " ? 0.f : 1.f)"; break;
                        case Op::kSmoothStep:
                            r = "jit_smooth(" + a + ", " + b + ", " + t + ")";
                            break;
                        case Op::kSigmoid: r = "1.f / (1.f + dressi::libc_expf(-" + a + "))"; break;
                        case Op::kLess: r = "(float)(" + a + " < " + b + ")"; break;
                        case Op::kLessEq: r = "(float)(" + a + " <= " + b + ")"; break;
                        case Op::kGreater: r = "(float)(" + a + " > " + b + ")"; break;
                        case Op::kGreaterEq: r = "(float)(" + a + " >= " + b + ")"; break;
                        case Op::kCopy: r = a; break;
                        case Op::kSumPw: {
                            o << "float s" << c << " = 0.f;\n";
                            for (uint32_t k = 0; k < ins.n_in; k++) {
                                o << "s" << c << " += " << v(k, c) << ";\n";
                            }
                            r = "s" + std::to_string(c);
                            break;
                        }
                        default: return std::string();  // not compiled: interpreted
                    }
                    y[c] = r;
                }
                break;
        }
        for (uint32_t c = 0; c < 4; c++) {
            o << "r" << i << "_" << c << " = " << (c < ins.ny ? y[c] : std::string("0.f"))
              << ";\n";
        }
        o << "}\n";
        if (ins.out_slot >= 0) {
            for (uint32_t c = 0; c < ins.ny && c < 4; c++) {
                o << "B[" << ins.out_slot << "][p * " << ins.ny << "ull + " << c << "] = r" << i
                  << "_" << c << ";\n";
            }
        }
    }
    return o.str();
}

std::string read_text(const std::string& path) {
    std::ifstream f(path);
    if (!f) {
        return std::string();
    }
    std::stringstream s;
    s << f.rdbuf();
    return s.str();
}

// the library's csrc directory (the headers the programs include)
std::string csrc_dir() {
    Dl_info info{};
    if (!dladdr((void*)&csrc_dir, &info) || !info.dli_fname) {
        return std::string();
    }
    std::string p = info.dli_fname;
    const size_t k = p.find_last_of('/');
    return (k == std::string::npos ? std::string(".") : p.substr(0, k)) + "/csrc/";
}

struct JitCache {
    std::mutex mu;
    std::map<std::pair<int, std::string>, hipFunction_t> fns;  // (device, body)
    bool disabled = false;
};

JitCache& jit_cache() {
    static JitCache c;
    return c;
}

bool jit_enabled() {
    const char* e = getenv("DRESSI_NO_JIT");
    return !(e && e[0] && e[0] != '0');
}

// Compiles the steps' new programs for `device` in one unit; sets jit_fn of
// every step whose program is compiled (cached or new).
template <typename StepT>
void jit_compile(std::vector<StepT>& steps, int device) {
    if (!jit_enabled()) {
        return;
    }
    JitCache& jc = jit_cache();
    std::lock_guard<std::mutex> lock(jc.mu);
    if (jc.disabled) {
        return;
    }
    std::map<std::string, std::string> todo;  // body -> kernel name
    bool libm = false;
    for (auto& s : steps) {
        if (s.jit_body.empty()) {
            continue;
        }
        auto it = jc.fns.find({device, s.jit_body});
        if (it != jc.fns.end()) {
            s.jit_fn = it->second;
            continue;
        }
        if (!todo.count(s.jit_body)) {
            const std::string name = "dressi_fp_" + std::to_string(todo.size());
            todo.emplace(s.jit_body, name);
        }
        libm = libm || s.jit_body.find("dressi::libm::") != std::string::npos;
    }
    if (todo.empty()) {
        return;
    }
    const std::string dir = csrc_dir();
    std::vector<std::string> names = {"dressi_math.h", "hip/hip_runtime.h", "stdint.h", "cstdint"};
    const std::string stdint_stub =
            "#pragma once\nusing __hip_internal::uint8_t; using __hip_internal::uint16_t; "
            "using __hip_internal::uint32_t; using __hip_internal::uint64_t; "
            "using __hip_internal::int8_t; using __hip_internal::int16_t; "
            "using __hip_internal::int32_t; using __hip_internal::int64_t;\n";
    std::vector<std::string> texts = {read_text(dir + "dressi_math.h"), "#pragma once\n",
                                      stdint_stub, stdint_stub};
    if (libm) {
        names.push_back("libm_f32.h");
        texts.push_back(read_text(dir + "libm_f32.h"));
        names.push_back("libm_pow5_table.h");
        texts.push_back(read_text(dir + "libm_pow5_table.h"));
    }
    for (size_t i = 0; i < texts.size(); i++) {
        if (texts[i].empty()) {
            fprintf(stderr, "dressi: run-time compilation off (no %s in %s)\n", names[i].c_str(),
                    dir.c_str());
            jc.disabled = true;
            return;
        }
    }
    std::ostringstream src;
    src << "#include \"dressi_math.h\"\n";
    if (libm) {
        src << "#include \"libm_f32.h\"\n";
    }
    src << "__device__ __forceinline__ float jit_min(float a, float b) { return b < a ? b : a; }\n"
           "__device__ __forceinline__ float jit_max(float a, float b) { return a < b ? b : a; }\n"
           "__device__ __forceinline__ float jit_smooth(float a, float b, float t) {\n"
           "    const float s = jit_min(jit_max((t - a) / (b - a), 0.f), 1.f);\n"
           "    return s * s * (3.f - 2.f * s);\n}\n";
    for (const auto& [body, name] : todo) {
        src << "extern \"C\" __global__ void __launch_bounds__(256) " << name
            << "(float* const* __restrict__ B, unsigned long long n) {\n"
               "const unsigned long long p = (unsigned long long)blockIdx.x * 256ull + threadIdx.x;\n"
               "if (p >= n) return;\n"
            << body << "}\n";
    }
    const std::string text = src.str();
    std::vector<const char*> hn, ht;
    for (size_t i = 0; i < names.size(); i++) {
        hn.push_back(names[i].c_str());
        ht.push_back(texts[i].c_str());
    }
    hipDeviceProp_t prop{};
    std::string arch = "--offload-arch=gfx950";
    if (hipGetDeviceProperties(&prop, device) == hipSuccess && prop.gcnArchName[0]) {
        std::string a = prop.gcnArchName;
        arch = "--offload-arch=" + a.substr(0, a.find(':'));
    }
    const char* opts[] = {arch.c_str(), "-O3", "-std=c++17", "-ffp-contract=off",
                          "-fhip-fp32-correctly-rounded-divide-sqrt", "-Xclang",
                          "-target-feature", "-Xclang", "-packed-fp32-ops"};
    hiprtcProgram prog = nullptr;
    bool ok = hiprtcCreateProgram(&prog, text.c_str(), "dressi_fused.hip", (int)names.size(),
                                  ht.data(), hn.data()) == HIPRTC_SUCCESS;
    ok = ok && hiprtcCompileProgram(prog, (int)(sizeof(opts) / sizeof(opts[0])), opts) ==
                       HIPRTC_SUCCESS;
    std::vector<char> code;
    if (ok) {
        size_t n = 0;
        ok = hiprtcGetCodeSize(prog, &n) == HIPRTC_SUCCESS && n > 0;
        code.resize(n);
        ok = ok && hiprtcGetCode(prog, code.data()) == HIPRTC_SUCCESS;
    } else if (prog) {
        size_t n = 0;
        hiprtcGetProgramLogSize(prog, &n);
        std::string log(n, '\0');
        hiprtcGetProgramLog(prog, &log[0]);
        fprintf(stderr, "dressi: run-time compilation failed, fused programs interpreted:\n%s\n",
                log.substr(0, 2000).c_str());
    }
    if (prog) {
        hiprtcDestroyProgram(&prog);
    }
    hipModule_t mod = nullptr;
    ok = ok && hipModuleLoadData(&mod, code.data()) == hipSuccess;
    if (!ok) {
        hipGetLastError();
        jc.disabled = true;
        return;
    }
    for (const auto& [body, name] : todo) {
        hipFunction_t f = nullptr;
        if (hipModuleGetFunction(&f, mod, name.c_str()) != hipSuccess) {
            hipGetLastError();
            jc.disabled = true;
            return;
        }
        jc.fns[{device, body}] = f;
    }
    for (auto& s : steps) {
        if (!s.jit_body.empty() && !s.jit_fn) {
            auto it = jc.fns.find({device, s.jit_body});
            if (it != jc.fns.end()) {
                s.jit_fn = it->second;
            }
        }
    }
}

struct Step {
    bool fused = false;
    std::vector<std::shared_ptr<FunctionNode>> fns;  // in order
    // fused program (host copy, device copy)
    std::vector<FInstr> code;
    std::vector<float> imm;
    std::vector<const VariableNode*> slots;  // slot -> variable (inputs and stored outputs)
    FInstr* d_code = nullptr;
    float* d_imm = nullptr;
    float** d_bufs = nullptr;
    size_t n_px = 0;
    uint32_t n_regs = 0;  // fused program: LDS register slots
    std::string jit_body;          // fused program as HIP statements (empty: interpreted)
    hipFunction_t jit_fn = nullptr;  // its compiled kernel
    // the variables whose images this step writes
    std::vector<const VariableNode*> outs;
};

}  // namespace

struct DressiAD::Impl {
    HipContextPtr hctx;
    PackingMode packing = PackingMode::RSP;
    InitStatus status = BACKWARD;
    Variable loss{nullptr};
    Optimizer optimizer;
    Variables input_vars, input_grad_vars, updated_vars;
    std::vector<std::pair<Variable, Variable>> copy_backs;  // (updated, input)
    Functions all_funcs;
    Variables leaf_vars;
    Variables extra_outputs;
    std::vector<std::pair<Variable, Variable>> extra_updates;  // (input, updated)
    // extra_updates[opt_updates_from ..) were added by the optimizer's last
    // call (addUpdate from inside it); the next optimizer rebuild replaces them
    size_t opt_updates_from = 0;
    bool in_optimizer = false;
    bool grad_outputs = false;
    // reactive cache
    uint32_t fast_count = 2, full_count = 8, static_cnt = 0;
    std::set<uint64_t> prev_dirty;
    bool pruning_active = false;
    std::set<uint64_t> dynamic_ids;
    // device state
    std::unordered_map<const VariableNode*, float*> bufs;
    std::unordered_set<const VariableNode*> computed;
    std::vector<std::shared_ptr<VariableNode>> keep;  // owners of the buffer keys
    std::vector<Step> packed, steps;
    bool plan_valid = false;
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    uint64_t graph_ws_gen = 0;  // workspace generation the graph was captured at
    bool graph_failed = false;
    uint32_t eager_runs = 0;
    // transfers
    std::map<Variable, CpuImage> pending;
    std::vector<std::pair<Variable, CpuImageView>> batch_uploads;
    Variables batch_downloads;
    bool have_download = false;
    CpuImage download;
    // the fused plan (silhouette or texture fit), when the graph is recognised
    std::unique_ptr<FusedRoute> route;
    bool route_rejected = false;
    // This instance's own C-ABI context on the shared context's stream: its
    // per-op workspaces are used by this instance only, so the device
    // pointers a captured hipGraph holds stay valid whatever other
    // instances on the shared context do.
    dressi_ctx* ws = nullptr;

    ~Impl() {
        route.reset();
        release_plan();
        if (ws) {
            dressi_ctx_synchronize(ws);
            for (auto& [n, p] : bufs) {
                dressi_free(ws, p);
            }
            dressi_ctx_destroy(ws);
        }
    }

    dressi_ctx* ctx() {
        ensure_ctx();
        return ws;
    }
    hipStream_t stream() { return (hipStream_t)dressi_ctx_stream(ctx()); }

    void ensure_ctx() {
        if (!hctx) {
            hctx = DressiAD::createContext();
        }
        if (!ws) {
            check(dressi_ctx_create(hctx->device, &ws), "DressiAD context");
            check(dressi_ctx_set_stream(ws, dressi_ctx_stream(hctx->ctx)), "DressiAD context");
        }
    }

    void release_graph() {
        if (graph_exec) {
            hipGraphExecDestroy(graph_exec);
            graph_exec = nullptr;
        }
        if (graph) {
            hipGraphDestroy(graph);
            graph = nullptr;
        }
    }

    void release_steps(std::vector<Step>& v) {
        for (auto& s : v) {
            if (s.d_code) {
                hipFree(s.d_code);
                hipFree(s.d_imm);
                hipFree(s.d_bufs);
                s.d_code = nullptr;
            }
        }
        v.clear();
    }

    void release_plan() {
        release_graph();
        if (ws) {
            dressi_ctx_synchronize(ws);
        }
        release_steps(steps);
        release_steps(packed);
        plan_valid = false;
    }

    Variables roots() const {
        Variables r = updated_vars;
        r.push_back(loss);
        for (const auto& v : extra_outputs) {
            r.push_back(v);
        }
        for (const auto& [inp, upd] : extra_updates) {
            r.push_back(upd);
        }
        if (grad_outputs) {
            for (const auto& g : input_grad_vars) {
                r.push_back(g);
            }
        }
        return r;
    }

    // Clears the dirty flag of every leaf and of everything computed
    // downstream of one: the result of setDirtyRecursively(false) on each
    // leaf (src/dressi_ad.cpp:526-528) in one walk, so a node downstream of
    // several leaves is visited once.
    void clear_dirty() {
        std::unordered_set<const VariableNode*> seen;
        std::vector<VariableNode*> stack;
        for (const auto& v : leaf_vars) {
            stack.push_back(NodeAccess::Node(v).get());
        }
        while (!stack.empty()) {
            VariableNode* n = stack.back();
            stack.pop_back();
            if (!n || !seen.insert(n).second) {
                continue;
            }
            n->dirty = false;
            for (const auto& wu : n->users) {
                if (const auto u = wu.lock()) {
                    if (const auto y = u->y.lock()) {
                        stack.push_back(y.get());
                    }
                }
            }
        }
    }

    std::set<uint64_t> dirty_leaf_ids() const {
        std::set<uint64_t> ids;
        for (const auto& v : leaf_vars) {
            if (v.IsDirty()) {
                ids.insert(v.id());
            }
        }
        return ids;
    }

    // dirty leaves, the optimizer's parameters and the addUpdate targets:
    // what changes this iteration (src/dressi_ad.cpp:101-118)
    Variables dynamic_seeds() const {
        Variables seeds;
        for (const auto& v : leaf_vars) {
            if (v.IsDirty()) {
                seeds.push_back(v);
            }
        }
        if (optimizer) {
            for (const auto& v : input_vars) {
                seeds.push_back(v);
            }
        }
        for (const auto& [inp, upd] : extra_updates) {
            seeds.push_back(inp);
        }
        return seeds;
    }

    bool has_cached(const VariableNode* n) const { return computed.count(n) != 0; }

    float* buf(const std::shared_ptr<VariableNode>& n) {
        auto it = bufs.find(n.get());
        if (it != bufs.end()) {
            return it->second;
        }
        void* p = nullptr;
        const size_t bytes = std::max<size_t>(n_floats(*n), 1) * sizeof(float);
        check(dressi_malloc(ctx(), &p, bytes), "device allocation");
        check(dressi_memset(ctx(), p, 0, bytes), "device clear");
        bufs[n.get()] = (float*)p;
        keep.push_back(n);
        return (float*)p;
    }
    float* buf(const Variable& v) { return buf(NodeAccess::Node(v)); }

    // Frees the device images of variables the current traversal no longer
    // reaches (setting the loss or the optimiser again builds new backward
    // and update nodes), with their cache entries and owners; the plan that
    // referred to them is released first.
    void prune_buffers() {
        std::unordered_set<const VariableNode*> live;
        auto add = [&](const Variable& v) {
            if (v) live.insert(NodeAccess::Node(v).get());
        };
        for (const auto& f : all_funcs) {
            for (const auto& x : f.getInputVars()) {
                add(x);
            }
            if (const auto y = NodeAccess::Node(f)->y.lock()) {
                live.insert(y.get());
            }
        }
        for (const auto& v : leaf_vars) add(v);
        for (const auto& [upd, inp] : copy_backs) {
            add(upd);
            add(inp);
        }
        for (const auto& v : extra_outputs) add(v);
        for (const auto& v : input_grad_vars) add(v);
        for (const auto& v : updated_vars) add(v);
        add(loss);
        bool released = false;
        for (auto it = bufs.begin(); it != bufs.end();) {
            if (live.count(it->first)) {
                ++it;
                continue;
            }
            if (!released) {
                release_plan();
                released = true;
            }
            dressi_free(ctx(), it->second);
            computed.erase(it->first);
            it = bufs.erase(it);
        }
        if (released) {
            keep.erase(std::remove_if(keep.begin(), keep.end(),
                                      [&](const std::shared_ptr<VariableNode>& n) {
                                          return !bufs.count(n.get());
                                      }),
                       keep.end());
        }
    }
    bool has_buf(const Variable& v) const { return bufs.count(NodeAccess::Node(v).get()) != 0; }

    // ---- packing -------------------------------------------------------------

    // The demand filter of the reactive cache over functions
    // (src/pack/reactive.cpp:38-68): creators reached from the roots,
    // stopping at static variables whose images are computed.
    Functions filter_funcs(const Functions& funcs) const {
        std::unordered_set<uint64_t> needed, seen;
        Variables stack = const_cast<Impl*>(this)->roots();
        while (!stack.empty()) {
            Variable v = stack.back();
            stack.pop_back();
            if (!v || !seen.insert(v.id()).second) {
                continue;
            }
            Function c = v.getCreator();
            if (!c) {
                continue;
            }
            if (!dynamic_ids.count(v.id()) && has_cached(NodeAccess::Node(v).get())) {
                continue;
            }
            if (needed.insert(c.id()).second) {
                for (const auto& x : c.getInputVars()) {
                    stack.push_back(x);
                }
            }
        }
        Functions out;
        for (const auto& f : funcs) {
            if (needed.count(f.id())) {
                out.push_back(f);
            }
        }
        return out;
    }

    // A topological order for RSP fusion: constants first (a fused program
    // reads them as immediates), then elementwise functions (pure, per
    // pixel) as soon as their inputs exist, those of the current run's image
    // size first, so that fewer runs break; every other function keeps its
    // place in the original order relative to the others of its kind. Any
    // topological order computes the same images.
    static Functions fusion_order(const Functions& funcs) {
        const size_t n = funcs.size();
        std::unordered_map<const FunctionNode*, size_t> idx;
        for (size_t i = 0; i < n; i++) {
            idx[NodeAccess::Node(funcs[i]).get()] = i;
        }
        std::vector<uint32_t> waiting(n, 0);
        std::vector<std::vector<size_t>> users(n);
        std::vector<char> ew(n, 0);
        std::vector<size_t> others, consts;  // non-elementwise, original order
        for (size_t i = 0; i < n; i++) {
            const auto& fn = NodeAccess::Node(funcs[i]);
            const auto y = fn->y.lock();
            ew[i] = IsElementwise(fn->op) && y && NumComponents(y->vtype) <= 4;
            if (fn->op == Op::kConst) {
                consts.push_back(i);
            } else if (!ew[i]) {
                others.push_back(i);
            }
            std::unordered_set<size_t> deps;
            for (const auto& x : fn->xs) {
                if (x->creator) {
                    auto it = idx.find(x->creator.get());
                    if (it != idx.end() && deps.insert(it->second).second) {
                        users[it->second].push_back(i);
                        waiting[i]++;
                    }
                }
            }
        }
        Functions out;
        out.reserve(n);
        std::vector<size_t> ready_ew;  // kept in original order
        std::vector<char> done(n, 0);
        size_t next_other = 0;
        ImgSize run_size{0, 0};
        const auto emit = [&](size_t i) {
            done[i] = 1;
            out.push_back(funcs[i]);
            for (size_t u : users[i]) {
                if (--waiting[u] == 0 && ew[u]) {
                    ready_ew.insert(std::upper_bound(ready_ew.begin(), ready_ew.end(), u), u);
                }
            }
        };
        for (size_t i = 0; i < n; i++) {
            if (ew[i] && waiting[i] == 0) {
                ready_ew.push_back(i);
            }
        }
        for (size_t i : consts) {
            emit(i);
        }
        while (out.size() < n) {
            if (!ready_ew.empty()) {
                // the earliest ready one of the current run's size, else the earliest
                size_t pick = 0;
                for (size_t k = 0; k < ready_ew.size(); k++) {
                    const auto y = NodeAccess::Node(funcs[ready_ew[k]])->y.lock();
                    if (y->size == run_size) {
                        pick = k;
                        break;
                    }
                }
                const size_t i = ready_ew[pick];
                ready_ew.erase(ready_ew.begin() + (ptrdiff_t)pick);
                run_size = NodeAccess::Node(funcs[i])->y.lock()->size;
                emit(i);
                continue;
            }
            DRESSI_CHECK(next_other < others.size() && waiting[others[next_other]] == 0,
                         "fusion order: the function graph is not acyclic");
            run_size = ImgSize{0, 0};
            emit(others[next_other++]);
        }
        return out;
    }

    // variables that must have an image: roots, copy-back sources and every
    // input of a step other than the one that produces it
    void pack(const Functions& funcs_in) {
        const Functions funcs = packing == PackingMode::RSP ? fusion_order(funcs_in) : funcs_in;
        release_graph();
        release_steps(packed);
        std::unordered_set<const VariableNode*> must_store;
        for (const auto& r : roots()) {
            if (r) {
                must_store.insert(NodeAccess::Node(r).get());
            }
        }
        std::vector<Step> out;
        const bool fuse = packing == PackingMode::RSP;
        for (const auto& f : funcs) {
            const auto& fn = NodeAccess::Node(f);
            const auto y = fn->y.lock();
            // matrix-typed elementwise ops run alone (k_wide)
            const bool ew = IsElementwise(fn->op) && NumComponents(y->vtype) <= 4;
            bool joined = false;
            if (fuse && ew && !out.empty() && out.back().fused &&
                out.back().fns.size() < (size_t)kMaxStepInstrs) {
                const auto& prev = out.back().fns.back()->y.lock();
                if (prev->size == y->size) {
                    out.back().fns.push_back(fn);
                    joined = true;
                }
            }
            if (!joined) {
                Step s;
                s.fused = ew;
                s.fns.push_back(fn);
                out.push_back(std::move(s));
            }
        }
        // which outputs leave their step
        std::unordered_map<const VariableNode*, size_t> step_of;
        for (size_t i = 0; i < out.size(); i++) {
            for (const auto& fn : out[i].fns) {
                step_of[fn->y.lock().get()] = i;
            }
        }
        for (size_t i = 0; i < out.size(); i++) {
            for (const auto& fn : out[i].fns) {
                for (const auto& x : fn->xs) {
                    if (out[i].fused && x->creator && x->creator->op == Op::kConst) {
                        continue;  // an immediate of the fused program
                    }
                    auto it = step_of.find(x.get());
                    if (it == step_of.end() || it->second != i) {
                        must_store.insert(x.get());
                    }
                }
            }
        }
        // constants only fused programs read need no step of their own
        out.erase(std::remove_if(out.begin(), out.end(),
                                 [&](const Step& st) {
                                     return !st.fused && st.fns[0]->op == Op::kConst &&
                                            !must_store.count(st.fns[0]->y.lock().get());
                                 }),
                  out.end());
        for (auto& s : out) {
            for (const auto& fn : s.fns) {
                const auto y = fn->y.lock();
                if (!s.fused || must_store.count(y.get())) {
                    s.outs.push_back(y.get());
                }
            }
        }
        packed = std::move(out);
        store_set = std::move(must_store);
    }
    std::unordered_set<const VariableNode*> store_set;

    // step-level demand filter (src/pack/reactive.cpp:70-111): walking the
    // steps backwards, keep a step iff a demanded image it writes is
    // dynamic or not computed yet
    void filter_steps() {
        release_graph();
        std::unordered_set<const VariableNode*> needed;
        for (const auto& r : roots()) {
            if (r) {
                needed.insert(NodeAccess::Node(r).get());
            }
        }
        std::vector<const Step*> kept;
        for (auto it = packed.rbegin(); it != packed.rend(); ++it) {
            bool run = false;
            for (const VariableNode* o : it->outs) {
                if (needed.count(o) && (dynamic_ids.count(o->id) || !has_cached(o))) {
                    run = true;
                    break;
                }
            }
            if (!run) {
                continue;
            }
            kept.push_back(&*it);
            for (const auto& fn : it->fns) {
                for (const auto& x : fn->xs) {
                    needed.insert(x.get());
                }
            }
        }
        release_steps(steps);
        for (auto it = kept.rbegin(); it != kept.rend(); ++it) {
            Step s;
            s.fused = (*it)->fused;
            s.fns = (*it)->fns;
            s.outs = (*it)->outs;
            steps.push_back(std::move(s));
        }
    }

    // device buffers and fused programs of the kept steps
    void build_device_plan() {
        for (const auto& f : all_funcs) {
            const auto& fn = NodeAccess::Node(f);
            for (const auto& x : fn->xs) {
                if (!x->creator || store_set.count(x.get())) {
                    buf(x);
                }
            }
        }
        for (auto& s : steps) {
            for (const VariableNode* o : s.outs) {
                for (const auto& fn : s.fns) {
                    auto y = fn->y.lock();
                    if (y.get() == o) {
                        buf(y);
                    }
                }
            }
            if (s.fused) {
                compile_fused(s);
            }
        }
        jit_compile(steps, ctx()->device);
        for (const auto& [upd, inp] : copy_backs) {
            buf(upd);
            buf(inp);
        }
        for (const auto& v : leaf_vars) {
            buf(v);
        }
        plan_valid = true;
    }

    void compile_fused(Step& s) {
        std::unordered_map<const VariableNode*, uint32_t> reg_of, slot_of;
        s.code.clear();
        s.imm.clear();
        s.slots.clear();
        auto slot = [&](const VariableNode* v) {
            auto it = slot_of.find(v);
            if (it != slot_of.end()) {
                return it->second;
            }
            const uint32_t k = (uint32_t)s.slots.size();
            s.slots.push_back(v);
            slot_of[v] = k;
            return k;
        };
        for (uint32_t i = 0; i < s.fns.size(); i++) {
            const auto& fn = s.fns[i];
            const auto y = fn->y.lock();
            FInstr ins{};
            ins.op = (int)fn->op;
            ins.n_in = (uint32_t)fn->xs.size();
            if (ins.n_in > (uint32_t)kMaxInputs) {
                throw DressiError(fn->name + ": more than 4 inputs in a fused stage");
            }
            ins.ny = NumComponents(y->vtype);
            ins.a0 = fn->a0;
            for (uint32_t k = 0; k < ins.n_in; k++) {
                const auto& x = fn->xs[k];
                FInput in{};
                in.nc = NumComponents(x->vtype);
                in.uniform = x->size.isUniform() ? 1u : 0u;
                auto r = reg_of.find(x.get());
                if (r != reg_of.end()) {
                    in.src = kSrcReg;
                    in.idx = r->second;
                } else if (x->creator && x->creator->op == Op::kConst) {
                    in.src = kSrcImm;
                    in.idx = (uint32_t)s.imm.size();
                    for (uint32_t c = 0; c < 4; c++) {
                        s.imm.push_back(c < x->creator->cval.size() ? x->creator->cval[c] : 0.f);
                    }
                } else {
                    in.src = kSrcBuf;
                    in.idx = slot(x.get());
                }
                ins.in[k] = in;
            }
            ins.out_slot = std::find(s.outs.begin(), s.outs.end(), y.get()) != s.outs.end()
                                   ? (int)slot(y.get())
                                   : -1;
            reg_of[y.get()] = i;
            s.code.push_back(ins);
            s.n_px = (size_t)y->size.w * y->size.h;
        }
        // the program as straight-line code for run-time compilation (SSA:
        // instruction indices, before the interpreter's slot reuse)
        {
            bool lm = false;
            s.jit_body = jit_body(s.code, s.imm, &lm);
            s.jit_fn = nullptr;
        }
        // registers: each result gets the lowest slot free when it is written
        // (a value is free after its last reader, which reads its inputs
        // before writing)
        {
            const uint32_t n = (uint32_t)s.code.size();
            std::vector<uint32_t> last(n, 0);
            for (uint32_t i = 0; i < n; i++) {
                last[i] = i;
                for (uint32_t k = 0; k < s.code[i].n_in; k++) {
                    if (s.code[i].in[k].src == kSrcReg) {
                        last[s.code[i].in[k].idx] = i;
                    }
                }
            }
            std::vector<uint32_t> slot_of_reg(n, 0);
            std::vector<int> holder;  // slot -> instruction holding it, -1 free
            for (uint32_t i = 0; i < n; i++) {
                for (size_t q = 0; q < holder.size(); q++) {
                    if (holder[q] >= 0 && last[(uint32_t)holder[q]] <= i) {
                        holder[q] = -1;
                    }
                }
                for (uint32_t k = 0; k < s.code[i].n_in; k++) {
                    FInput& in = s.code[i].in[k];
                    if (in.src == kSrcReg) {
                        in.idx = slot_of_reg[in.idx];
                    }
                }
                size_t q = 0;
                while (q < holder.size() && holder[q] >= 0) {
                    q++;
                }
                if (q == holder.size()) {
                    holder.push_back(-1);
                }
                holder[q] = (int)i;
                slot_of_reg[i] = (uint32_t)q;
                s.code[i].reg = (uint32_t)q;
            }
            s.n_regs = (uint32_t)std::max<size_t>(holder.size(), 1);
        }
        if (s.imm.empty()) {
            s.imm.push_back(0.f);
        }
        std::vector<float*> ptrs;
        for (const VariableNode* v : s.slots) {
            auto it = bufs.find(v);
            if (it == bufs.end()) {
                throw DressiError("fused stage: an input has no device image");
            }
            ptrs.push_back(it->second);
        }
        if (ptrs.empty()) {
            ptrs.push_back(nullptr);
        }
        check_hip(hipMalloc(&s.d_code, sizeof(FInstr) * s.code.size()), "fused program");
        check_hip(hipMalloc(&s.d_imm, sizeof(float) * s.imm.size()), "fused program");
        check_hip(hipMalloc(&s.d_bufs, sizeof(float*) * ptrs.size()), "fused program");
        check_hip(hipMemcpy(s.d_code, s.code.data(), sizeof(FInstr) * s.code.size(),
                            hipMemcpyHostToDevice),
                  "fused program");
        check_hip(hipMemcpy(s.d_imm, s.imm.data(), sizeof(float) * s.imm.size(),
                            hipMemcpyHostToDevice),
                  "fused program");
        check_hip(hipMemcpy(s.d_bufs, ptrs.data(), sizeof(float*) * ptrs.size(),
                            hipMemcpyHostToDevice),
                  "fused program");
    }

    // ---- running ---------------------------------------------------------------

    void run_step(const Step& s) {
        hipStream_t st = stream();
        if (s.fused && s.jit_fn) {
            float** bufs = s.d_bufs;
            unsigned long long n = s.n_px;
            void* args[] = {&bufs, &n};
            check_hip(hipModuleLaunchKernel(s.jit_fn, (uint32_t)((s.n_px + 255) / 256), 1, 1, 256, 1,
                                            1, 0, st, args, nullptr),
                      "compiled fused stage launch");
            return;
        }
        if (s.fused) {
            FProgram P{s.d_code, (uint32_t)s.code.size(), s.n_regs, s.n_px, s.d_bufs, s.d_imm};
            hipLaunchKernelGGL(k_fused, dim3((uint32_t)((s.n_px + kFusedThreads - 1) / kFusedThreads)),
                               dim3(kFusedThreads), sizeof(float4) * kFusedThreads * P.n_regs, st,
                               P);
            check_hip(hipGetLastError(), "fused stage launch");
            return;
        }
        run_single(*s.fns[0]);
    }

    void run_single(const FunctionNode& fn) {
        dressi_ctx* c = ctx();
        hipStream_t s = stream();
        const auto y = fn.y.lock();
        float* out = buf(y);
        const uint32_t ny = NumComponents(y->vtype);
        const size_t n_px = (size_t)y->size.w * y->size.h;
        std::vector<const float*> in;
        std::vector<const VariableNode*> xn;
        for (const auto& x : fn.xs) {
            in.push_back(buf(x));
            xn.push_back(x.get());
        }
        auto nc = [&](int i) { return NumComponents(xn[i]->vtype); };
        auto w_of = [&](int i) { return xn[i]->size.w; };
        auto h_of = [&](int i) { return xn[i]->size.h; };
        uint32_t* err = nullptr;
        switch (fn.op) {
            case Op::kConst: {
                const auto& v = fn.cval;
                hipLaunchKernelGGL(k_fill, dim3(1), dim3(64), 0, s, out, (uint32_t)v.size(), v[0],
                                   v.size() > 1 ? v[1] : 0.f, v.size() > 2 ? v[2] : 0.f,
                                   v.size() > 3 ? v[3] : 0.f);
                break;
            }
            case Op::kReduce2x2:
                hipLaunchKernelGGL(k_reduce2x2, dim3(blocks256(n_px)), dim3(256), 0, s, in[0],
                                   w_of(0), h_of(0), ny, y->size.w, y->size.h, out);
                break;
            case Op::kUpsample2x:
                hipLaunchKernelGGL(k_upsample2x, dim3(blocks256(n_px)), dim3(256), 0, s, in[0],
                                   w_of(0), ny, y->size.w, y->size.h, out);
                break;
            case Op::kScreenCoord:
                hipLaunchKernelGGL(k_screen_coord, dim3(blocks256(n_px)), dim3(256), 0, s,
                                   y->size.w, y->size.h, out);
                break;
            case Op::kSumAll:
                hipLaunchKernelGGL(k_sum_all, dim3(1), dim3(64), 0, s, in[0],
                                   (size_t)w_of(0) * h_of(0), nc(0), out);
                break;
            case Op::kPixelFetch:
                err = c->d_err;
                hipLaunchKernelGGL(k_pixel_fetch, dim3(1), dim3(64), 0, s, in[0], w_of(0), h_of(0),
                                   nc(0), fn.a0, in[1], out, err);
                break;
            case Op::kTileFetch:
                err = c->d_err;
                hipLaunchKernelGGL(k_tile_fetch, dim3(blocks256(n_px * ny)), dim3(256), 0, s,
                                   in[0], w_of(0), h_of(0), nc(0), fn.a0, in[1], out, err);
                break;
            case Op::kMatMul:
            case Op::kTranspose:
            case Op::kOuter:
                hipLaunchKernelGGL(k_matrix, dim3(blocks256(n_px)), dim3(256), 0, s, (int)fn.op,
                                   in[0], xn[0]->size.isUniform() ? 1u : 0u,
                                   in.size() > 1 ? in[1] : in[0],
                                   in.size() > 1 && xn[1]->size.isUniform() ? 1u : 0u, fn.a0,
                                   fn.a1, n_px, out);
                break;
            case Op::kVertexNeighborMean:
                DRESSI_CHECK(w_of(1) == w_of(0), "VertexNeighborMean: table width != vertices");
                hipLaunchKernelGGL(k_vertex_neighbor_mean, dim3(blocks256(w_of(0))), dim3(256), 0,
                                   s, in[0], w_of(0), in[1], h_of(1), out, c->d_err);
                break;
            case Op::kNcFaceTerm:
                DRESSI_CHECK(w_of(2) == w_of(1), "NormalConsistencyFaceTerm: adjacency != faces");
                hipLaunchKernelGGL(k_nc_face_term, dim3(blocks256(w_of(1))), dim3(256), 0, s,
                                   in[0], w_of(0), in[1], in[2], w_of(1), out, c->d_err);
                break;
            case Op::kNcVertexGrad:
                DRESSI_CHECK(w_of(0) == w_of(2) && w_of(3) == w_of(1),
                             "NormalConsistencyVertexGrad: term / table sizes");
                hipLaunchKernelGGL(k_nc_vertex_grad, dim3(blocks256(w_of(1))), dim3(256), 0, s,
                                   in[0], in[1], in[2], w_of(2), in[3], w_of(1), h_of(3), out,
                                   c->d_err);
                break;
            case Op::kRasterize:
                check(dressi_rasterize(c, in[0], w_of(0), in[1], nc(1), in[2], w_of(2), y->size.w,
                                       y->size.h, out),
                      "Rasterize");
                break;
            case Op::kRasterizeFaceId:
                check(dressi_rasterize_face_id(c, in[0], w_of(0), in[2], w_of(2), y->size.w,
                                               y->size.h, out),
                      "RasterizeFaceId");
                break;
            case Op::kSoftClip:
                check(dressi_soft_clip(c, in[0], w_of(0), in[1], w_of(1), fn.a0, fn.a1, fn.f0, out),
                      "SoftClip");
                break;
            case Op::kRasterizeSoft:
                check(dressi_rasterize_soft(c, in[0], in[1], in[2], in[3], w_of(3), in[4], w_of(4),
                                            fn.a0, fn.a1, fn.f0, fn.flag ? in[6] : nullptr, out),
                      "RasterizeSoft");
                break;
            case Op::kLookupFaces:
                check(dressi_lookup_faces(c, in[0], nc(0), w_of(0), in[1], w_of(1), fn.a0, out),
                      "LookupFaces");
                break;
            case Op::kLookupFacesBwd:
                check(dressi_lookup_faces_bwd(c, in[0], nc(0), in[1], w_of(1), in[2], w_of(2),
                                              h_of(2), fn.a0, out),
                      "LookupFacesBwd");
                break;
            case Op::kFaceFetch:
                check(dressi_face_fetch(c, in[0], nc(0), w_of(0), in[1], w_of(1), h_of(1), out),
                      "FaceFetch");
                break;
            case Op::kFaceFetchBwd:
                check(dressi_face_fetch_bwd(c, in[0], nc(0), in[1], w_of(1), h_of(1), in[2], in[3],
                                            in[4], w_of(2), in[5], fn.f0, fn.a0, out),
                      "FaceFetchBwd");
                break;
            case Op::kGatherDistGrad:
                check(dressi_gather_dist_grad(c, in[0], in[1], in[2], w_of(2), in[3], w_of(3),
                                              in[4], h_of(4), fn.f0, fn.flag, w_of(1), h_of(1),
                                              out),
                      "GatherDistGrad");
                break;
            case Op::kColSum:
                check(dressi_col_sum(c, in[0], nc(0), w_of(0), h_of(0), out), "ColSum");
                break;
            case Op::kAntiAlias:
                check(dressi_antialias(c, in[0], nc(0), in[1], in[2], w_of(2), in[3], w_of(3),
                                       w_of(0), h_of(0), out),
                      "AntiAlias");
                break;
            case Op::kAaBwdImg:
                check(dressi_antialias_bwd_img(c, in[0], nc(0), in[1], in[2], w_of(2), in[3],
                                               w_of(3), w_of(0), h_of(0), out),
                      "AntiAliasBwdImg");
                break;
            case Op::kAaBwdVtx:
                check(dressi_antialias_bwd_vtx(c, in[0], in[1], nc(0), in[2], in[3], w_of(3), in[4],
                                               w_of(4), in[5], h_of(5), in[6], fn.a0, fn.flag,
                                               w_of(0), h_of(0), out),
                      "AntiAliasBwdVtx");
                break;
            case Op::kTexture:
                check(dressi_texture_nearest(c, in[0], w_of(0), h_of(0), nc(0), in[1], w_of(1),
                                             h_of(1), out),
                      "Texture");
                break;
            case Op::kGatherInvUv:
                check(dressi_texture_nearest_bwd(c, in[0], nc(0), w_of(0), h_of(0), in[1], w_of(1),
                                                 h_of(1), in[2], out),
                      "GatherByInverseUV");
                break;
            case Op::kTextureBilinear:
                check(dressi_texture_bilinear(c, in[0], w_of(0), h_of(0), nc(0), in[1], w_of(1),
                                              h_of(1), out),
                      "TextureBilinear");
                break;
            case Op::kGatherInvUvBilinear:
                check(dressi_texture_bilinear_bwd(c, in[0], nc(0), w_of(0), h_of(0), in[1],
                                                  w_of(1), h_of(1), in[2], out),
                      "GatherByInverseUVBilinear");
                break;
            case Op::kEquirectSample:
                check(dressi_equirect_sample(c, in[0], w_of(0), h_of(0), nc(0), in[1], w_of(1),
                                             h_of(1), out),
                      "EquirectSample");
                break;
            case Op::kEquirectSampleBwd:
                check(dressi_equirect_sample_bwd(c, in[0], nc(0), in[1], w_of(1), h_of(1),
                                                 y->size.w, y->size.h, out),
                      "EquirectSampleBwd");
                break;
            case Op::kIrradianceConv:
                check(dressi_irradiance_conv(c, in[0], w_of(0), h_of(0), nc(0), y->size.w,
                                             y->size.h, out),
                      "IrradianceConv");
                break;
            case Op::kIrradianceConvBwd:
                check(dressi_irradiance_conv_bwd(c, in[0], w_of(0), h_of(0), nc(0), y->size.w,
                                                 y->size.h, out),
                      "IrradianceConvBwd");
                break;
            case Op::kPrefilterEnv:
                check(dressi_prefilter_env(c, in[0], w_of(0), h_of(0), nc(0), y->size.w, y->size.h,
                                           fn.f0, fn.a0, out),
                      "PrefilterEnv");
                break;
            case Op::kPrefilterConv:
                if (fn.flag) {  // the normaliser: a0 x a1 = the source size
                    check(dressi_prefilter_conv_norm(c, y->size.w, y->size.h, fn.a0, fn.a1, fn.f0,
                                                     out),
                          "PrefilterConvNorm");
                } else {
                    check(dressi_prefilter_conv(c, in[0], w_of(0), h_of(0), nc(0), y->size.w,
                                                y->size.h, fn.f0, in[1], out),
                          "PrefilterConv");
                }
                break;
            case Op::kPrefilterConvBwd:
                check(dressi_prefilter_conv_bwd(c, in[0], w_of(0), h_of(0), nc(0), y->size.w,
                                                y->size.h, fn.f0, in[1], out),
                      "PrefilterConvBwd");
                break;
            case Op::kBrdfLut:
                check(dressi_brdf_lut(c, y->size.w, y->size.h, fn.a0, out), "BrdfIntegrationLut");
                break;
            case Op::kCustom:
                throw DressiError("a Function built from GLSL text (\"" + fn.name +
                                  "\") cannot run on the HIP executor");
            case Op::kSetFragDepth:
            case Op::kPeelDepth:
                throw DressiError(fn.name +
                                  " belongs to a custom raster pass, which the HIP executor "
                                  "does not run");
            case Op::kAdd:
            case Op::kSub:
            case Op::kMul:
            case Op::kDiv:
            case Op::kNeg:
            case Op::kCopy:
            case Op::kSumPw: {
                WideArgs A{};
                A.op = (int)fn.op;
                A.n_in = (uint32_t)fn.xs.size();
                A.ny = ny;
                A.n_px = n_px;
                DRESSI_CHECK(A.n_in <= (uint32_t)kMaxInputs, fn.name + ": more than 4 inputs");
                for (uint32_t k = 0; k < A.n_in; k++) {
                    A.in[k] = {in[k], nc((int)k), xn[k]->size.isUniform() ? 1u : 0u};
                    DRESSI_CHECK(A.in[k].nc == 1 || A.in[k].nc == ny,
                                 fn.name + ": component count mismatch");
                }
                A.y = out;
                hipLaunchKernelGGL(k_wide, dim3(blocks256(n_px * ny)), dim3(256), 0, s, A);
                break;
            }
            default:
                throw DressiError(fn.name + (IsElementwise(fn.op)
                                                     ? ": not defined on matrix-typed images"
                                                     : ": no kernel"));
        }
        check_hip(hipGetLastError(), "kernel launch");
    }

    void run_copy_backs() {
        for (const auto& [upd, inp] : copy_backs) {
            check_hip(hipMemcpyAsync(buf(inp), buf(upd),
                                     n_floats(*NodeAccess::Node(inp)) * sizeof(float),
                                     hipMemcpyDeviceToDevice, stream()),
                      "copy-back");
        }
    }

    void run_steps() {
        for (const auto& s : steps) {
            run_step(s);
        }
        run_copy_backs();
    }

    // One iteration on the device. The step sequence is captured into a
    // hipGraph once it has run eagerly (so every per-op workspace exists),
    // then replayed; a capture the runtime rejects falls back to eager runs.
    // Ops whose entry points upload host tables synchronously: a step list
    // holding one runs eagerly (a capture would record a copy from a
    // temporary host buffer)
    static bool capturable(Op op) {
        switch (op) {
            case Op::kIrradianceConv:
            case Op::kIrradianceConvBwd:
            case Op::kPrefilterConv:
            case Op::kPrefilterConvBwd:
            case Op::kPrefilterEnv:
            case Op::kBrdfLut: return false;
            default: return true;
        }
    }

    bool steps_capturable() const {
        for (const auto& s : steps) {
            if (!s.fused && !capturable(s.fns[0]->op)) {
                return false;
            }
        }
        return true;
    }

    void execute() {
        if (graph_exec && dressi_ctx_workspace_generation(ctx()) != graph_ws_gen) {
            // a per-op call through context() regrew a workspace the graph
            // holds: run eagerly (which re-sizes them) and capture again
            release_graph();
            eager_runs = 0;
        }
        if (!graph_exec && !graph_failed && eager_runs >= 1 && !steps_capturable()) {
            graph_failed = true;
        }
        if (!graph_exec && !graph_failed && eager_runs >= 1) {
            hipStream_t s = stream();
            if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) == hipSuccess) {
                bool ok = true;
                try {
                    run_steps();
                } catch (const DressiError&) {
                    ok = false;
                }
                hipGraph_t g = nullptr;
                const hipError_t e = hipStreamEndCapture(s, &g);
                if (ok && e == hipSuccess && g &&
                    hipGraphInstantiate(&graph_exec, g, nullptr, nullptr, 0) == hipSuccess) {
                    graph = g;
                    graph_ws_gen = dressi_ctx_workspace_generation(ctx());
                } else {
                    if (g) {
                        hipGraphDestroy(g);
                    }
                    graph_exec = nullptr;
                    graph_failed = true;
                    hipGetLastError();
                }
            } else {
                graph_failed = true;
                hipGetLastError();
            }
        }
        if (graph_exec) {
            check_hip(hipGraphLaunch(graph_exec, stream()), "graph launch");
        } else {
            run_steps();
            eager_runs++;
        }
        for (const auto& s : steps) {
            for (const VariableNode* o : s.outs) {
                computed.insert(o);
            }
        }
    }

    // ---- the fused plans (route.h) ------------------------------------------

    // Hand the graph back to the generic executor: the route's leaf images
    // (current optimiser state included) become pending sends.
    void drop_route() {
        std::map<Variable, CpuImage> back;
        route->Export(&back);
        for (auto& [var, img] : back) {
            pending[var] = std::move(img);
        }
        route.reset();
        route_rejected = true;
        status = std::min(status, SUBSTAGE);
    }

    // One iteration on the fused plan; false when the graph went back to
    // the generic executor
    bool run_route() {
        for (auto it = pending.begin(); it != pending.end();) {
            if (!route->Accept(it->first, CpuImageView(it->second))) {
                drop_route();
                return false;
            }
            it = pending.erase(it);
        }
        for (const auto& [var, view] : batch_uploads) {
            if (!route->Accept(var, view)) {
                drop_route();
                return false;
            }
        }
        std::map<Variable, CpuImage> back;
        if (!route->Step(ctx(), &back)) {
            for (auto& [var, img] : back) {
                pending[var] = std::move(img);
            }
            route.reset();
            route_rejected = true;
            status = std::min(status, SUBSTAGE);
            return false;
        }
        if (!batch_downloads.empty()) {
            download = stack(batch_downloads, [&](const Variable& v) { return route->Recv(v); });
            have_download = true;
        }
        check(dressi_ctx_synchronize(ctx()), "execStep");
        return true;
    }

    // ---- the generic executor ----------------------------------------------

    void run_generic() {
        if (status <= STAGE) {
            dynamic_ids.clear();
            for (const auto& s : dynamic_seeds()) {
                dynamic_ids.insert(s.id());
            }
            for (const auto& f : all_funcs) {
                for (const auto& x : f.getInputVars()) {
                    if (dynamic_ids.count(x.id())) {
                        dynamic_ids.insert(f.getOutputVar().id());
                        break;
                    }
                }
            }
        }
        bool fn_pruned = pruning_active;
        if (status <= SUBSTAGE) {
            const Functions exec = filter_funcs(all_funcs);
            fn_pruned = exec.size() < all_funcs.size();
            pack(exec);
        }
        if (status <= STAGE) {
            filter_steps();
            pruning_active = fn_pruned || steps.size() < packed.size();
        }
        if (status <= VULKAN) {
            build_device_plan();
            eager_runs = 0;
            graph_failed = false;
        }
        // pending sends (images exist now), then this step's uploads
        for (auto& [var, img] : pending) {
            upload(var, CpuImageView(img));
        }
        pending.clear();
        for (const auto& [var, view] : batch_uploads) {
            upload(var, view);
        }
        execute();
        if (!batch_downloads.empty()) {
            download = stack(batch_downloads, [&](const Variable& v) {
                DRESSI_CHECK(has_buf(v), "stacked recv: the Variable has no device image");
                return download_of(v);
            });
            have_download = true;
        }
        check(dressi_ctx_synchronize(ctx()), "execStep");
    }

    // same-shape images stacked into one {w, h * n} image
    template <typename Fetch>
    static CpuImage stack(const Variables& vars, Fetch fetch) {
        const ImgSize s0 = vars[0].getImgSize();
        const uint32_t ch = NumComponents(vars[0].getVType());
        CpuImage out(s0.w, s0.h * (uint32_t)vars.size(), ch);
        size_t o = 0;
        for (const auto& v : vars) {
            DRESSI_CHECK(v.getImgSize() == s0 && NumComponents(v.getVType()) == ch,
                         "stacked recv: images must share one size and type");
            const CpuImage img = fetch(v);
            std::copy(img.data.begin(), img.data.end(), out.data.begin() + (ptrdiff_t)o);
            o += img.data.size();
        }
        return out;
    }

    // ---- transfers -------------------------------------------------------------

    static void check_view(const Variable& var, const CpuImageView& v) {
        DRESSI_CHECK(v.data || v.numElems() == 0, "sendImg: null data");
        const ImgSize s = var.getImgSize();
        DRESSI_CHECK(v.width == s.w && v.height == s.h,
                     "sendImg: image size differs from the Variable's");
        DRESSI_CHECK(v.channels == NumComponents(var.getVType()),
                     "sendImg: channel count differs from the Variable's type");
    }

    void upload(const Variable& var, const CpuImageView& v) {
        check(dressi_memcpy_h2d(ctx(), buf(var), v.data, v.numElems() * sizeof(float)),
              "sendImg");
        computed.insert(NodeAccess::Node(var).get());
    }

    CpuImage download_of(const Variable& var) {
        const ImgSize s = var.getImgSize();
        CpuImage img(s.w, s.h, NumComponents(var.getVType()));
        check(dressi_memcpy_d2h(ctx(), img.data.data(), buf(var), img.data.size() * sizeof(float)),
              "recvImg");
        check(dressi_ctx_synchronize(ctx()), "recvImg");
        return img;
    }
};

DressiAD::DressiAD() : m_impl(std::make_unique<Impl>()) {}

DressiAD::DressiAD(VkContextPtr ctx) : m_impl(std::make_unique<Impl>()) {
    DRESSI_CHECK(ctx, "DressiAD: null context");
    m_impl->hctx = std::move(ctx);
}

DressiAD::~DressiAD() = default;

VkContextPtr DressiAD::createContext(bool debug) {
    (void)debug;
    return createContextOnDevice(0);
}

VkContextPtr DressiAD::createContextOnDevice(int device) {
    auto c = std::make_shared<HipContext>();
    c->device = device;
    check(dressi_ctx_create(device, &c->ctx), "createContext");
    return c;
}

void DressiAD::setLossVar(const Variable& loss_var) {
    m_impl->loss = loss_var;
    m_impl->status = BACKWARD;
}

void DressiAD::setOptimizer(const Optimizer& optim_func) {
    m_impl->optimizer = optim_func;
    m_impl->status = BACKWARD;
}

void DressiAD::setPackingMode(PackingMode mode) {
    if (m_impl->packing != mode) {
        m_impl->packing = mode;
        if (m_impl->status > SUBSTAGE) {
            m_impl->status = SUBSTAGE;
        }
    }
}

void DressiAD::setRebuildCounts(uint32_t fast, uint32_t full) {
    m_impl->fast_count = fast;
    m_impl->full_count = full;
}

void DressiAD::markOutput(const Variable& var) {
    DRESSI_CHECK(var, "markOutput: null Variable");
    m_impl->extra_outputs.push_back(var);
    if (m_impl->status > TRAVERSE) {
        m_impl->status = TRAVERSE;
    }
}

void DressiAD::addUpdate(const Variable& input_leaf, const Variable& updated) {
    DRESSI_CHECK(input_leaf && updated, "addUpdate: null Variable");
    DRESSI_CHECK(!input_leaf.getCreator(), "addUpdate: input must be a leaf Variable");
    DRESSI_CHECK(updated.getCreator(), "addUpdate: updated must be a computed Variable");
    DRESSI_CHECK(input_leaf.getVType() == updated.getVType() &&
                         input_leaf.getImgSize() == updated.getImgSize(),
                 "addUpdate: updated must match the input's type and size");
    if (!m_impl->in_optimizer) {
        // a pair added outside the optimizer goes before the optimizer's own
        m_impl->extra_updates.insert(
                m_impl->extra_updates.begin() + (ptrdiff_t)m_impl->opt_updates_from,
                {input_leaf, updated});
        m_impl->opt_updates_from++;
    } else {
        m_impl->extra_updates.emplace_back(input_leaf, updated);
    }
    if (m_impl->status > OPTIMIZER) {
        m_impl->status = OPTIMIZER;
    }
}

void DressiAD::setGradOutputsEnabled(bool enable) {
    if (m_impl->grad_outputs != enable) {
        m_impl->grad_outputs = enable;
        if (m_impl->status > TRAVERSE) {
            m_impl->status = TRAVERSE;
        }
    }
}

std::vector<std::pair<Variable, Variable>> DressiAD::inputGrads() const {
    std::vector<std::pair<Variable, Variable>> r;
    for (size_t i = 0; i < m_impl->input_vars.size(); i++) {
        r.emplace_back(m_impl->input_vars[i], m_impl->input_grad_vars[i]);
    }
    return r;
}

size_t DressiAD::getFuncCount() const { return m_impl->all_funcs.size(); }

size_t DressiAD::getStageCount() const {
    if (m_impl->route) {
        return 1;
    }
    return m_impl->steps.size();
}

size_t DressiAD::getSubStageCount() const {
    if (m_impl->route) {
        return m_impl->route->kernels();
    }
    size_t n = 0;
    for (const auto& s : m_impl->steps) {
        n += s.fns.size();
    }
    return n;
}

std::string DressiAD::getDeviceName() const {
    if (!m_impl->hctx) {
        return {};
    }
    char b[256];
    check(dressi_ctx_device_name(m_impl->hctx->ctx, b, sizeof(b)), "getDeviceName");
    return b;
}

std::string DressiAD::getPlanName() const {
    return m_impl->route ? m_impl->route->name() : std::string("generic");
}

dressi_ctx* DressiAD::context() const { return m_impl->ctx(); }

void DressiAD::execStep() {
    Impl& im = *m_impl;
    DRESSI_CHECK(im.loss, "setLossVar() must be called before execStep()");
    im.ensure_ctx();
    // reactive cache: the dirty pattern of the data leaves
    if (im.status == FINISHED) {
        const std::set<uint64_t> cur = im.dirty_leaf_ids();
        if (cur != im.prev_dirty) {
            im.static_cnt = 0;
            if (im.pruning_active) {
                im.status = SUBSTAGE;
            }
        } else {
            im.static_cnt++;
            if (im.fast_count != 0 && im.static_cnt == im.fast_count) {
                im.status = STAGE;
            } else if (im.full_count != 0 && im.static_cnt == im.full_count) {
                im.status = SUBSTAGE;
            }
        }
        im.prev_dirty = cur;
    }
    if (im.status <= BACKWARD) {
        std::tie(im.input_vars, im.input_grad_vars) = BuildBackward(im.loss);
        im.route_rejected = false;
    }
    if (im.status <= OPTIMIZER) {
        im.updated_vars.clear();
        im.copy_backs.clear();
        // pairs the previous optimizer call registered belong to the graph
        // it built; the call below registers the current graph's
        if (im.opt_updates_from < im.extra_updates.size()) {
            im.extra_updates.resize(im.opt_updates_from);
        }
        im.opt_updates_from = im.extra_updates.size();
        if (im.optimizer) {
            im.in_optimizer = true;
            try {
                im.updated_vars = im.optimizer(im.input_vars, im.input_grad_vars);
            } catch (...) {
                im.in_optimizer = false;
                throw;
            }
            im.in_optimizer = false;
            DRESSI_CHECK(im.updated_vars.size() == im.input_vars.size(),
                         "Optimizer must return one output per input");
            for (size_t i = 0; i < im.updated_vars.size(); i++) {
                const Variable& u = im.updated_vars[i];
                const Variable& x = im.input_vars[i];
                DRESSI_CHECK(u.getVType() == x.getVType() && u.getImgSize() == x.getImgSize(),
                             "Optimizer output must match its input's type and size");
                im.copy_backs.emplace_back(u, x);
            }
        }
        // addUpdate pairs made outside the optimizer persist across rebuilds
        for (const auto& [inp, upd] : im.extra_updates) {
            im.copy_backs.emplace_back(upd, inp);
        }
    }
    if (im.status <= TRAVERSE) {
        im.all_funcs = TraverseFuncs(im.roots());
        im.leaf_vars.clear();
        std::set<uint64_t> seen;
        for (const auto& f : im.all_funcs) {
            for (const auto& x : f.getInputVars()) {
                if (!x.getCreator() && seen.insert(x.id()).second) {
                    im.leaf_vars.push_back(x);
                }
            }
        }
        for (const auto& [upd, inp] : im.copy_backs) {
            if (seen.insert(inp.id()).second) {
                im.leaf_vars.push_back(inp);
            }
        }
        im.prune_buffers();
        // a fused plan, when the graph is one of the examples'
        if (im.route) {
            im.drop_route();
        }
        if (im.packing == PackingMode::RSP && !im.route_rejected) {
            GraphRoots g;
            g.loss = im.loss;
            g.input_vars = im.input_vars;
            g.input_grad_vars = im.input_grad_vars;
            g.updated_vars = im.updated_vars;
            g.extra_updates = im.extra_updates;
            g.extra_outputs = im.extra_outputs;
            g.grad_outputs = im.grad_outputs;
            g.funcs = &im.all_funcs;
            im.route = RecogniseFusedRoute(g);
        }
    }
    bool routed = false;
    if (im.route) {
        routed = im.run_route();
    }
    if (!routed) {
        im.run_generic();
    }
    if (im.status != FINISHED) {
        im.prev_dirty = im.dirty_leaf_ids();
    }
    im.clear_dirty();
    im.status = FINISHED;
}

void DressiAD::execStepWithSends(const std::vector<std::pair<Variable, CpuImageView>>& items) {
    Impl& im = *m_impl;
    im.batch_uploads.clear();
    for (const auto& [var, view] : items) {
        DRESSI_CHECK(var, "execStepWithSends: null Variable");
        Impl::check_view(var, view);
        Variable v = var;
        v.setDirty(true);
        if (im.plan_valid || im.route) {
            im.batch_uploads.emplace_back(var, view);
        } else {
            CpuImage owned(view.width, view.height, view.channels);
            std::copy(view.data, view.data + view.numElems(), owned.data.begin());
            im.pending[var] = std::move(owned);
        }
    }
    try {
        execStep();
    } catch (...) {
        im.batch_uploads.clear();
        throw;
    }
    im.batch_uploads.clear();
}

CpuImage DressiAD::execStepWithSendsAndRecvImgsStacked(
        const std::vector<std::pair<Variable, CpuImageView>>& sends, const Variables& recvs) {
    Impl& im = *m_impl;
    DRESSI_CHECK(!recvs.empty(), "execStepWithSendsAndRecvImgsStacked: empty recv batch");
    im.batch_downloads = recvs;
    im.have_download = false;
    try {
        execStepWithSends(sends);
    } catch (...) {
        im.batch_downloads.clear();
        throw;
    }
    im.batch_downloads.clear();
    DRESSI_CHECK(im.have_download, "combined recv did not produce an image");
    im.have_download = false;
    return std::move(im.download);
}

void DressiAD::sendImg(const Variable& var, const CpuImage& cpu_img) {
    sendImg(var, CpuImageView(cpu_img));
}

void DressiAD::sendImg(const Variable& var, const CpuImageView& cpu_img) {
    Impl& im = *m_impl;
    DRESSI_CHECK(var, "sendImg: null Variable");
    Impl::check_view(var, cpu_img);
    Variable v = var;
    v.setDirty(true);
    if (im.route) {
        if (im.route->Accept(var, cpu_img)) {
            return;
        }
        // an image for a variable the plan computes: the generic executor
        // takes the graph over
        im.drop_route();
    }
    if (im.plan_valid && im.has_buf(var)) {
        im.upload(var, cpu_img);
        return;
    }
    CpuImage owned(cpu_img.width, cpu_img.height, cpu_img.channels);
    std::copy(cpu_img.data, cpu_img.data + cpu_img.numElems(), owned.data.begin());
    im.pending[var] = std::move(owned);
}

void DressiAD::sendImgs(const std::vector<std::pair<Variable, CpuImageView>>& items) {
    for (const auto& [var, view] : items) {
        sendImg(var, view);
    }
}

CpuImage DressiAD::recvImg(const Variable& var) {
    Impl& im = *m_impl;
    DRESSI_CHECK(var, "recvImg: null Variable");
    auto it = im.pending.find(var);
    if (it != im.pending.end()) {
        return it->second;
    }
    if (im.route) {
        return im.route->Recv(var);
    }
    DRESSI_CHECK(im.plan_valid, "recvImg before the first execStep()");
    DRESSI_CHECK(im.has_buf(var),
                 "recvImg: the Variable has no device image (markOutput it before execStep)");
    return im.download_of(var);
}

std::vector<CpuImage> DressiAD::recvImgs(const Variables& vars) {
    std::vector<CpuImage> out;
    for (const auto& v : vars) {
        out.push_back(recvImg(v));
    }
    return out;
}

CpuImage DressiAD::recvImgsStacked(const Variables& vars) {
    DRESSI_CHECK(!vars.empty(), "recvImgsStacked: empty batch");
    std::vector<CpuImage> imgs = recvImgs(vars);
    CpuImage out(imgs[0].width, imgs[0].height * (uint32_t)imgs.size(), imgs[0].channels);
    size_t o = 0;
    for (const auto& im : imgs) {
        DRESSI_CHECK(im.width == imgs[0].width && im.height == imgs[0].height &&
                             im.channels == imgs[0].channels,
                     "recvImgsStacked: images must share one size and type");
        std::copy(im.data.begin(), im.data.end(), out.data.begin() + (ptrdiff_t)o);
        o += im.data.size();
    }
    return out;
}

}  // namespace dressi
