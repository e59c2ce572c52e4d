// plan.h -- device-side state of the fused silhouette-fit plan (shared by
// the HardSoftRas kernels in hsr.hip and the AA kernels in aa.hip).
#pragma once

#include "aa_core.h"
#include "raster_core.h"

namespace dressi {

constexpr uint32_t kMaxViews = 8;

// ---------------------------------------------------------------------------
// Static reduction trees: SumContribs / SumPixelWise (src/core/build_backward.cpp:41-58,
// src/core/f_ops.cpp:921-948) fold n inputs in levels of <= 4-ary sequential
// sums; a lone trailing input passes through unchanged.
// ---------------------------------------------------------------------------
template <int N, int D>
struct Tree {
    static __device__ __forceinline__ void run(const float (&v)[N][D], float (&out)[D]) {
        constexpr int M = (N + 3) / 4;
        float nxt[M][D];
#pragma unroll
        for (int i = 0; i < M; i++) {
            const int cnt = (N - 4 * i) < 4 ? (N - 4 * i) : 4;
#pragma unroll
            for (int c = 0; c < D; c++) {
                if (cnt == 1) {
                    nxt[i][c] = v[4 * i][c];
                } else {
                    float acc = 0.f;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        if (j < cnt) {
                            acc += v[4 * i + j][c];
                        }
                    }
                    nxt[i][c] = acc;
                }
            }
        }
        Tree<M, D>::run(nxt, out);
    }
};
template <int D>
struct Tree<1, D> {
    static __device__ __forceinline__ void run(const float (&v)[1][D], float (&out)[D]) {
#pragma unroll
        for (int c = 0; c < D; c++) {
            out[c] = v[0][c];
        }
    }
};

// ---------------------------------------------------------------------------
// Kernels of one iteration
// ---------------------------------------------------------------------------
struct HsrDev {
    RasterGeom g;
    uint32_t n_verts, max_deg, n_samples, flags;
    float radius, sigma_scale, inv_px, lr, b1, b2, eps;
    float* pos;
    float* m;
    float* v;
    float* t;
    float* t_next;            // t + 1, written by the face backward for the vertex kernel
    const int32_t* faces;     // [F][3]
    const int32_t* vf;        // [deg][V], -1 pad
    const uint8_t* vf_mask;   // [deg][V], bit k: faces[vf][k] == v
    const float* mvps;        // [N][16]
    const float* targets;     // [N][S][S]
    const uint8_t* tgt8;      // [N][S][S] the same targets as bytes when every one is
                              // exactly 0 or 1 (hard-rasterized silhouettes), else null
    SoftRec* recs;            // [N][F]
    CullRec* cull;            // [N][F]
    BinBuffers bins;          // fixed-capacity soft bins, N x tiles; the
                              // face backward clears the counters
    HeavyList heavy;          // the bins the raster resolves first (kept by the
                              // setup's appends, segment counters cleared by the
                              // face backward)
    uint32_t* ids;            // [N][S][S] face + 1 (bit 31: rim winner), 0 bg
    uint8_t* rimf;            // [N][F] HardSoftRas: 1 if the face won a rim pixel
                              // (set by the raster, cleared by the face backward)
    float* loss;              // [S][S]
    float* pred;              // [N][S][S] or null
    float4* gtri;             // [N][3][F]
    float4* fscr;             // [N][F][2] HardSoftRas: the chain's screen corners of
                              // each face, (s0x, s0y, s1x, s1y), (s2x, s2y, 0, 0)
    float* grad;              // [V][3] or null
    // Adam bias corrections 1 - b1^t, 1 - b2^t for t = 1 .. bc_len, filled
    // on the host with the C library's powf (the reference evaluator's
    // F::Pow), so the in-graph Adam matches it bit for bit
    const float2* bc_tab;
    uint32_t bc_len;
    // technique aa (DRESSI_HSR_TECHNIQUE_AA): per-view clip positions, hard
    // raster records; pred is always kept (the vertex gather needs it)
    uint32_t technique;       // 0 HardSoftRas, 1 AA
    float4* clip;             // [N][V]
    AaRec* arecs;             // [N][F]
    // texture plan: per (view, face) the attribute corners of the screen
    // raster's perspective-correct interpolation, written by the AA setup:
    // (1 / w0, 1 / w1, 1 / w2, 0), (u0, v0, u1, v1), (u2, v2, 0, 0); null
    // elsewhere
    const float2* tf_uv;      // [V] uv of the vertices
    float4* tface;            // [N][F][3]
    uint32_t* aa_list;        // [N * F] faces with a sample where d loss / d pred != 0
    uint32_t* aa_count;       // entries of aa_list (reset by the clip kernel)
    uint32_t* gflag;          // [N][H][ceil(W / 256)] AA: 1 when a pixel of the 256-pixel row
                              // segment has d loss / d pred != 0 (the forward writes every
                              // segment each iteration; the face scan reads only those)
    // the largest bin count above bins.cap this iteration: the kernels that
    // clear the bins take the maximum in bin_over_max (device memory), and
    // one thread of the vertex Adam kernel, which runs after them, hands it
    // to bin_over (host-mapped, written only when a bin overflowed; the
    // plan's next step grows the bins from it) and clears bin_over_max
    uint32_t* bin_over;
    uint32_t* bin_over_max;
};

// The iteration's bin overflow (see HsrDev::bin_over) to the host report.
__device__ __forceinline__ void publish_bin_over(const HsrDev& d) {
    if (d.bin_over && d.bin_over_max && blockIdx.x == 0 && threadIdx.x == 0) {
        const uint32_t m = *d.bin_over_max;
        if (m) {
            *d.bin_over = m;
            *d.bin_over_max = 0;
        }
    }
}

constexpr uint32_t kBiasTableLen = 1u << 16;

constexpr uint32_t kRimFlag = 0x80000000u;

// Corner clips of face f in one view: TransformToClipVar of its vertices.
__device__ __forceinline__ void face_clips(const HsrDev& d, uint32_t view, uint32_t f,
                                           float4 c[3]) {
    const float* m = d.mvps + view * 16;
#pragma unroll
    for (int k = 0; k < 3; k++) {
        const int32_t vi = d.faces[f * 3 + k];
        c[k] = mvp_transform(m, d.pos[vi * 3 + 0], d.pos[vi * 3 + 1], d.pos[vi * 3 + 2]);
    }
}


// Vertex tail of both techniques: the per-view clip gradients of one vertex
// through TransformToClipVar (examples/common/geometry_utils.cpp:391-402:
// per view x / y / z get one 4-term sum over the clip rows; pos gets the
// GetZ, GetY, GetX contributions of view N-1 .. 0, newest first, through
// the SumContribs tree), then the in-graph Adam step
// (examples/silhouette_optimization/run.cpp:421-436) at step t_new = t + 1.
template <int NV>
__device__ __forceinline__ void pos_grad_adam(const HsrDev& d, uint32_t vtx,
                                              const float (&gc)[NV][4], float t_new) {
    float contrib[3 * NV][3];
#pragma unroll
    for (int vi = 0; vi < NV; vi++) {
        const int view = NV - 1 - vi;
        const float* m = d.mvps + view * 16;
        float gxyz[3];
#pragma unroll
        for (int comp = 0; comp < 3; comp++) {
            float acc = 0.f;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                acc += gc[view][r] * m[comp * 4 + r];
            }
            gxyz[comp] = acc;
        }
#pragma unroll
        for (int q = 0; q < 3; q++) {
            const int comp = 2 - q;
            contrib[vi * 3 + q][0] = 0.f;
            contrib[vi * 3 + q][1] = 0.f;
            contrib[vi * 3 + q][2] = 0.f;
            contrib[vi * 3 + q][comp] = gxyz[comp];
        }
    }
    float g[3];
    Tree<3 * NV, 3>::run(contrib, g);
    if (d.grad) {
#pragma unroll
        for (int c = 0; c < 3; c++) {
            d.grad[vtx * 3 + c] = g[c];
        }
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
    float m0[3], v0[3], p0[3];
#pragma unroll
    for (int c = 0; c < 3; c++) {
        const size_t j = (size_t)vtx * 3 + c;
        m0[c] = d.m[j];
        v0[c] = d.v[j];
        p0[c] = d.pos[j];
    }
#pragma unroll
    for (int c = 0; c < 3; c++) {
        const size_t j = (size_t)vtx * 3 + c;
        const float m_new = m0[c] * d.b1 + g[c] * cb1;
        const float v_new = v0[c] * d.b2 + g[c] * g[c] * cb2;
        const float step = (m_new / bc1) / (sqrtf(v_new / bc2) + d.eps) * d.lr;
        d.pos[j] = p0[c] - step;
        d.m[j] = m_new;
        d.v[j] = v_new;
    }
}

// A batch of kDegBatch adjacency slots of one vertex (VertexFacesTex rows
// d0 .. d0 + kDegBatch - 1; -1 = padding or beyond max_deg), loaded
// together so that their latencies overlap.
constexpr int kDegBatch = 8;
struct AdjBatch {
    int32_t f[kDegBatch];
    uint32_t mask[kDegBatch];
};

__device__ __forceinline__ void load_adjacency(const HsrDev& d, uint32_t vtx, uint32_t d0,
                                               AdjBatch& ab) {
#pragma unroll
    for (int i = 0; i < kDegBatch; i++) {
        const uint32_t dd = d0 + (uint32_t)i;
        const bool in = dd < d.max_deg;
        const size_t o = (size_t)(in ? dd : 0u) * d.n_verts + vtx;
        const int32_t f = d.vf[o];
        const uint32_t m = d.vf_mask[o];
        ab.f[i] = in ? f : -1;
        ab.mask[i] = in ? m : 0u;
    }
}

// The first corner (0, 1, 2) whose bit is set in an adjacency corner mask.
__device__ __forceinline__ int first_corner(uint32_t mask) {
    return (mask & 1u) ? 0 : ((mask & 2u) ? 1 : 2);
}

// Lanes per vertex of the vertex kernels: the NV views of one vertex run on
// L = next power of two >= NV adjacent lanes, so the per-view adjacency
// gathers (the latency of the kernel) are spread over NV lanes.
template <int NV>
struct VertexLanes {
    static constexpr int L = NV <= 1 ? 1 : NV <= 2 ? 2 : NV <= 4 ? 4 : 8;
};

template <int NV>
inline uint32_t vertex_grid(uint32_t n_verts) {
    return (uint32_t)(((uint64_t)n_verts * VertexLanes<NV>::L + 255) / 256);
}

// Body of both vertex kernels (blockDim.x = 256, grid vertex_grid<NV>):
// lane (vertex, view) computes that view's clip gradient g4 through
// `view_grad(vtx, view, g4)`; the vertex's first lane collects the NV
// gradients (shuffles) and runs pos_grad_adam. The step count t + 1 comes
// from t_next (written by the face backward, which runs before), so this
// kernel never reads t and its first thread can store t + 1 without racing
// the others.
template <int NV, typename ViewGrad>
__device__ __forceinline__ void vertex_views_adam(const HsrDev& d, ViewGrad&& view_grad) {
    constexpr int L = VertexLanes<NV>::L;
    const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t vtx = gid / L;
    const uint32_t view = gid % L;
    const float t_new = *d.t_next;
    const bool live = vtx < d.n_verts;
    float g4[4] = {0.f, 0.f, 0.f, 0.f};
    if (live && view < NV) {
        view_grad(vtx, view, g4);
    }
    const int base = (int)(threadIdx.x & 63u) & ~(L - 1);
    float gc[NV][4];
#pragma unroll
    for (int v = 0; v < NV; v++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            gc[v][r] = __shfl(g4[r], base + v);
        }
    }
    if (live && view == 0) {
        pos_grad_adam<NV>(d, vtx, gc, t_new);
    }
    if (gid == 0) {
        *d.t = t_new;
    }
}

// The face backward's first thread publishes t + 1 for the vertex kernel.
__device__ __forceinline__ void publish_t_next(const HsrDev& d, uint32_t gid) {
    if (gid == 0) {
        *d.t_next = *d.t + 1.f;
    }
}

// Launches kernel k (0 .. kAaKernels - 1) of one AA-technique iteration
// (aa.hip): 0 clip + setup + binning, 1 visibility raster, 2 AntiAlias +
// loss, 3 vertex-gradient gather, 4 ColSum + clip->pos + Adam.
constexpr int kAaKernels = 5;
extern const char* const kAaKernelNames[kAaKernels];
int launch_aa_kernel(const HsrDev& d, hipStream_t s, int k);
// The hard-raster part of that plan on its own, for any HsrDev whose g,
// n_verts, faces, clip, arecs, bins and ids are set: the per-(view, face)
// setup + bin append (bins empty on entry), and the face-id raster
// (RasterizeCore's winner + 1, 0 = background). Used by the texture plan.
int launch_aa_setup(const HsrDev& d, hipStream_t s);
int launch_aa_raster(const HsrDev& d, hipStream_t s);
// Renders the AA target of one view into `out` ({S,S} float):
// StopGradient(AntiAlias(Rasterize(tgt, 1), RasterizeFaceId(tgt), tgt_clip,
// tgt_faces, ...)) with zero seed (run.cpp:346-357).
int aa_render_target(dressi_ctx* ctx, const float* tgt_clip_dev, uint32_t n_tverts,
                     const float* tgt_faces_dev, uint32_t n_tfaces, uint32_t w, uint32_t h,
                     float* out);

}  // namespace dressi
