// raster.hip -- tile binning, the per-op rasterizers (RasterizeSoft,
// Rasterize, RasterizeFaceId) and SoftClip.
#include <mutex>

#include "raster_core.h"
#include "soft_clip.h"

namespace dressi {

// ---------------------------------------------------------------------------
// Binning
// ---------------------------------------------------------------------------

size_t bin_bytes(uint32_t n_bins, uint32_t cap) {
    return sizeof(uint32_t) * ((size_t)n_bins * 3 + 1 + cap) + 256;
}

void bin_carve(void* base, uint32_t n_bins, uint32_t cap, BinBuffers* b) {
    uint32_t* p = (uint32_t*)base;
    b->counts = p;
    b->offsets = p + n_bins;
    b->cursor = p + 2 * (size_t)n_bins + 1;
    b->list = p + 3 * (size_t)n_bins + 1;
    b->cap = cap;
    b->n_bins = n_bins;
}

uint32_t default_bin_cap(const RasterGeom& g, uint32_t per_face) {
    const uint64_t c = (uint64_t)g.n_faces * g.n_views * per_face + 4096;
    return c > 0x7fffffffull ? 0x7fffffffu : (uint32_t)c;
}

template <typename Rec>
__global__ __launch_bounds__(256) void k_count(RasterGeom g, const Rec* recs, BinBuffers b) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= g.n_views * g.n_faces) {
        return;
    }
    const Rec& r = recs[i];
    if (r.bx0 > r.bx1 || r.by0 > r.by1) {
        return;
    }
    const uint32_t view = i / g.n_faces;
    uint32_t* cnt = b.counts + (size_t)view * g.n_tiles;
    for (int ty = r.by0 / kTile; ty <= r.by1 / kTile; ty++) {
        for (int tx = r.bx0 / kTile; tx <= r.bx1 / kTile; tx++) {
            atomicAdd(&cnt[ty * g.tiles_x + tx], 1u);
        }
    }
}

template <typename Rec>
__global__ __launch_bounds__(256) void k_bin(RasterGeom g, const Rec* recs, BinBuffers b) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= g.n_views * g.n_faces) {
        return;
    }
    const Rec& r = recs[i];
    if (r.bx0 > r.bx1 || r.by0 > r.by1) {
        return;
    }
    const uint32_t view = i / g.n_faces;
    const uint32_t f = i - view * g.n_faces;
    uint32_t* cur = b.cursor + (size_t)view * g.n_tiles;
    for (int ty = r.by0 / kTile; ty <= r.by1 / kTile; ty++) {
        for (int tx = r.bx0 / kTile; tx <= r.bx1 / kTile; tx++) {
            const uint32_t slot = atomicAdd(&cur[ty * g.tiles_x + tx], 1u);
            if (slot < b.cap) {
                b.list[slot] = f;
            }
        }
    }
}

// Exclusive scan of the bin counts (one workgroup): writes offsets and
// cursors and clears the counts for the next use.
__global__ __launch_bounds__(1024) void k_scan(BinBuffers b) {
    __shared__ uint32_t part[1024];
    const uint32_t n = b.n_bins;
    const uint32_t per = (n + 1023) / 1024;
    const uint32_t beg = threadIdx.x * per;
    const uint32_t end = beg + per < n ? beg + per : n;
    uint32_t s = 0;
    for (uint32_t i = beg; i < end; i++) {
        s += b.counts[i];
    }
    part[threadIdx.x] = s;
    __syncthreads();
    for (uint32_t off = 1; off < 1024; off <<= 1) {
        const uint32_t v = threadIdx.x >= off ? part[threadIdx.x - off] : 0u;
        __syncthreads();
        part[threadIdx.x] += v;
        __syncthreads();
    }
    uint32_t run = part[threadIdx.x] - s;
    for (uint32_t i = beg; i < end; i++) {
        const uint32_t c = b.counts[i];
        b.offsets[i] = run;
        b.cursor[i] = run;
        b.counts[i] = 0;
        run += c;
    }
    if (threadIdx.x == 1023) {
        b.offsets[n] = part[1023];
    }
}

int launch_scan_bins(hipStream_t s, const BinBuffers& b) {
    hipLaunchKernelGGL(k_scan, dim3(1), dim3(1024), 0, s, b);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int launch_count_hard(hipStream_t s, const RasterGeom& g, const HardRec* recs, const BinBuffers& b) {
    const uint32_t n = g.n_views * g.n_faces;
    hipLaunchKernelGGL(k_count<HardRec>, dim3(div_up(n, 256)), dim3(256), 0, s, g, recs, b);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int launch_bin_hard(hipStream_t s, const RasterGeom& g, const HardRec* recs, const BinBuffers& b) {
    const uint32_t n = g.n_views * g.n_faces;
    hipLaunchKernelGGL(k_bin<HardRec>, dim3(div_up(n, 256)), dim3(256), 0, s, g, recs, b);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

// ---------------------------------------------------------------------------
// Hard rasterizer (Rasterize / RasterizeFaceId)
// ---------------------------------------------------------------------------

// clip [views][V] float4, faces int32 [F][3]; one thread per (view, face).
__global__ __launch_bounds__(256) void k_hard_setup(RasterGeom g, const float4* clip,
                                                     uint32_t n_verts, const int32_t* faces,
                                                     HardRec* recs) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= g.n_views * g.n_faces) {
        return;
    }
    const uint32_t view = i / g.n_faces;
    const uint32_t f = i - view * g.n_faces;
    HardRec r;
    int idx[3];
    float4 c[3];
    bool ok = true;
    for (int k = 0; k < 3; k++) {
        idx[k] = faces[(size_t)f * 3 + k];
        ok = ok && idx[k] >= 0 && (uint32_t)idx[k] < n_verts;
    }
    if (!ok) {
        r.bx0 = 1;
        r.bx1 = 0;
        r.by0 = 1;
        r.by1 = 0;
        recs[i] = r;
        return;
    }
    for (int k = 0; k < 3; k++) {
        c[k] = clip[(size_t)view * n_verts + idx[k]];
    }
    hard_setup(c, idx, g.width, g.height, &r);
    recs[i] = r;
}

int launch_hard_setup(hipStream_t s, const RasterGeom& g, const float* clip, uint32_t n_verts,
                      const int32_t* faces, HardRec* recs) {
    const uint32_t n = g.n_views * g.n_faces;
    hipLaunchKernelGGL(k_hard_setup, dim3(div_up(n, 256)), dim3(256), 0, s, g,
                       (const float4*)clip, n_verts, faces, recs);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

// One workgroup per (tile, view). mode 0: perspective-correct attribute of
// the winner (cpu_raster.cpp:205-223), mode 1: face + 1.
__global__ __launch_bounds__(kTileThreads) void k_raster_hard(RasterGeom g, const HardRec* recs,
                                                              BinBuffers b, const float* attr,
                                                              uint32_t n_comp, int mode,
                                                              float* out, size_t attr_view,
                                                              float* ids) {
    __shared__ HardRec lds_rec[kTileThreads];
    __shared__ uint32_t lds_face[kTileThreads];
    const uint32_t tile = blockIdx.x;
    const uint32_t view = blockIdx.y;
    const int px = (int)((tile % g.tiles_x) * kTile + (threadIdx.x % kTile));
    const int py = (int)((tile / g.tiles_x) * kTile + (threadIdx.x / kTile));
    const HardRec* vrec = recs + (size_t)view * g.n_faces;
    uint64_t best = kEmptyKey;
    walk_bin(vrec, b, view * g.n_tiles + tile, g.n_faces, lds_rec, lds_face,
             [&](const HardRec& r, uint32_t f) { hard_fragment(r, f, px, py, &best); });
    if (px >= (int)g.width || py >= (int)g.height) {
        return;
    }
    const size_t o = ((size_t)view * g.height + py) * g.width + px;
    if (ids) {
        ids[o] = best == kEmptyKey ? 0.f : (float)key_face(best) + 1.f;
    }
    if (best == kEmptyKey) {
        for (uint32_t c = 0; c < n_comp; c++) {
            out[o * n_comp + c] = 0.f;
        }
        return;
    }
    const uint32_t f = key_face(best);
    if (mode == 1) {
        out[o] = (float)f + 1.f;
        return;
    }
    attr += (size_t)view * attr_view;
    const HardRec& r = vrec[f];
    float l[3];
    barycentric((float)px + 0.5f, (float)py + 0.5f, r.x[0], r.y[0], r.x[1], r.y[1], r.x[2],
                r.y[2], r.inv_area, &l[0], &l[1], &l[2]);
    const float denom = l[0] * r.inv_w[0] + l[1] * r.inv_w[1] + l[2] * r.inv_w[2];
    for (uint32_t c = 0; c < n_comp; c++) {
        float num = 0.f;
        for (int k = 0; k < 3; k++) {
            num += l[k] * r.inv_w[k] * attr[(size_t)r.idx[k] * n_comp + c];
        }
        out[o * n_comp + c] = num / denom;
    }
}

int launch_raster_hard(hipStream_t s, const RasterGeom& g, const HardRec* recs,
                       const BinBuffers& b, const float* attr, uint32_t n_comp, int mode,
                       float* out, size_t attr_view, float* ids) {
    hipLaunchKernelGGL(k_raster_hard, dim3(g.n_tiles, g.n_views), dim3(kTileThreads), 0, s, g,
                       recs, b, attr, n_comp, mode, out, attr_view, ids);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

// ---------------------------------------------------------------------------
// Per-op soft rasterizer (RasterizeSoft)
// ---------------------------------------------------------------------------

// Fill kernel for counters (graph-capture safe, unlike a memset node).
__global__ void k_fill_u32(uint32_t* p, uint32_t n, uint32_t v) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        p[i] = v;
    }
}

// One thread per face: soft corners via faces_soft, face id from the last
// soft corner, hard corners via faces_tex[hard face] (cpu_raster.cpp:257-303);
// the face is appended to the fixed-capacity bins of the tiles its soft
// pixel bbox touches.
__global__ __launch_bounds__(256) void k_soft_setup_op(RasterGeom g, const float4* soft_clip,
                                                        const float* face_id,
                                                        const float* faces_soft,
                                                        const float4* hard_clip,
                                                        uint32_t n_verts,
                                                        const float* faces_tex, BinBuffers b,
                                                        uint32_t* err, SoftRec* recs,
                                                        CullRec* cull) {
    __shared__ BinLds blds;
    const uint32_t f = blockIdx.x * blockDim.x + threadIdx.x;
    SoftRec r;
    r.bx0 = 1;
    r.bx1 = 0;
    r.by0 = 1;
    r.by1 = 0;
    r.flags = 0;
    if (f < g.n_faces) {
        float4 sc[3], hc[3];
        float fid = 0.f;
        bool ok = true;
        const uint32_t n_soft = 3 * g.n_faces;
        for (int k = 0; k < 3 && ok; k++) {
            const uint32_t vi = (uint32_t)(int64_t)faces_soft[(size_t)f * 3 + k];
            if (vi >= n_soft) {
                atomicOr(err, 1u);
                ok = false;
                break;
            }
            sc[k] = soft_clip[vi];
            if (!clip_w_valid(sc[k].w)) {
                ok = false;  // the reference skips the face at the first bad corner
                break;
            }
            fid = face_id[vi];
        }
        const uint32_t hf = ok ? fid_u(fid) : 0u;
        if (ok && hf >= g.n_faces) {
            atomicOr(err, 2u);
            ok = false;
        }
        for (int k = 0; k < 3 && ok; k++) {
            const uint32_t vi = fid_u(faces_tex[(size_t)hf * 3 + k]);
            if (vi >= n_verts) {
                atomicOr(err, 4u);
                ok = false;
                break;
            }
            hc[k] = hard_clip[vi];
        }
        if (ok) {
            soft_setup(sc, hc, fid, g.width, g.height, &r);
        }
        recs[f] = r;
        cull[f] = cull_setup(r);
    }
    const bool valid = f < g.n_faces && r.bx0 <= r.bx1 && r.by0 <= r.by1;
    bin_append(b, g, valid, 0u, f, r.bx0, r.by0, r.bx1, r.by1, soft_bin_tri(r), blds);
}

// One wave per 8x8 block: resolves the winner, then re-evaluates its signed
// distance and hard z (the output channels) from its record.
__global__ __launch_bounds__(64) void k_raster_soft_op(RasterGeom g, const SoftRec* recs,
                                                       const CullRec* cull, BinBuffers b,
                                                       float radius, const float* prev,
                                                       float4* out) {
    const BlockPos blk = block_pos(blockIdx.x, g);
    if (!blk.valid) {
        return;
    }
    const int lane = threadIdx.x & 63;
    const int px = blk.bx + (lane & 7);
    const int py = blk.by + (lane >> 3);
    const BinView bv = bin_view(b, blk.tile, g.n_faces);
    __shared__ ResolveLds lds;
    const PixelBest best =
            resolve_block(recs, cull, bv, blk.bx, blk.by, radius, prev, g.width, lds);
    if (px >= (int)g.width || py >= (int)g.height) {
        return;
    }
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    if (best.key != kEmptyKey) {
        const SoftRec& r = recs[key_face(best.key)];
        const float p0 = (float)px + 0.5f;
        const float p1 = (float)py + 0.5f;
        const float dist = signed_dist(p0, p1, r.hx, r.hy, r.ex, r.ey, r.len2);
        o = make_float4(dist, r.fid, hard_z_at(r, p0, p1), 1.f);
    }
    out[(size_t)py * g.width + px] = o;
}

__global__ void k_soft_clip(const float4* clip, uint32_t n_verts, const float* faces,
                            uint32_t n_faces, uint32_t w, uint32_t h, float radius,
                            uint32_t* err, float4* out) {
    const uint32_t f = blockIdx.x * blockDim.x + threadIdx.x;
    if (f >= n_faces) {
        return;
    }
    float4 c[3];
    for (int k = 0; k < 3; k++) {
        const uint32_t vi = fid_u(faces[(size_t)f * 3 + k]);
        if (vi >= n_verts) {
            atomicOr(err, 8u);
            return;
        }
        c[k] = clip[vi];
    }
    float4 o[3];
    soft_clip_face(c, w, h, radius, o);
    for (int k = 0; k < 3; k++) {
        out[(size_t)f * 3 + k] = o[k];
    }
}

// faces float ids -> int32 (RasterizeCore decodes with uint32_t(int64_t(x)))
__global__ void k_faces_to_i32(const float* faces, uint32_t n, uint32_t n_verts,
                               uint32_t* err, int32_t* out) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const uint32_t v = (uint32_t)(int64_t)faces[i];
        if (v >= n_verts) {
            atomicOr(err, 16u);
        }
        out[i] = (int32_t)v;
    }
}

}  // namespace dressi

// Scratch of dressi_rasterize_soft_noalloc: one fixed array per GPU (each
// GPU the library runs on holds its own copy until the process ends). In
// host code the name `scratch` is a host-side stand-in, never the device
// array: kernels take the per-device address that hipGetSymbolAddress
// returns (noalloc_scratch below). Every call on a GPU shares that GPU's
// array: host calls are taken one at a time (g_noalloc_mu), calls on one
// stream run in order, and a call on another stream than the GPU's previous
// call first waits for that call's work (an event created with the array's
// address, recorded after every call). A call made while its stream is
// captured into a graph records no wait and no event, so replays of that
// graph race with every other call on the GPU.
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

using namespace dressi;

namespace {

int check_ctx(dressi_ctx* ctx) {
    DRESSI_REQUIRE(ctx != nullptr, "NULL context");
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    return DRESSI_OK;
}

int check_soft_args(const float* soft_clip, const float* face_id, const float* faces_soft,
                    const float* hard_clip, const float* faces_tex, uint32_t width,
                    uint32_t height, float radius_px, const float* out) {
    DRESSI_REQUIRE(soft_clip && face_id && faces_soft && hard_clip && faces_tex && out,
                   "dressi_rasterize_soft: NULL buffer");
    DRESSI_REQUIRE(radius_px > 0.f, "RasterizeSoft: radius_px must be > 0");
    DRESSI_REQUIRE(width > 0 && height > 0, "RasterizeSoft: empty screen");
    return DRESSI_OK;
}

// RasterizeSoft over caller-provided scratch: `recs` / `cull` hold one record
// per face, `bins` fixed_bin_bytes(tiles, kSoftBinCap) bytes (counts cleared
// here by a fill kernel, so the scratch may hold anything on entry).
int launch_rasterize_soft(dressi_ctx* ctx, const RasterGeom& g, const float* soft_clip,
                          const float* face_id, const float* faces_soft, const float* hard_clip,
                          uint32_t n_verts, const float* faces_tex, float radius_px,
                          const float* prev_shifted_depth, SoftRec* recs, void* bins,
                          CullRec* cull, float* out) {
    BinBuffers b;
    fixed_bin_carve(bins, g.n_tiles, kSoftBinCap, &b);
    hipLaunchKernelGGL(k_fill_u32, dim3(div_up(g.n_tiles, 256)), dim3(256), 0, ctx->stream,
                       b.counts, g.n_tiles, 0u);
    DRESSI_CHECK_LAUNCH();
    if (g.n_faces) {
        hipLaunchKernelGGL(k_soft_setup_op, dim3(div_up(g.n_faces, 256)), dim3(256), 0,
                           ctx->stream, g, (const float4*)soft_clip, face_id, faces_soft,
                           (const float4*)hard_clip, n_verts, faces_tex, b, ctx->d_err, recs,
                           cull);
        DRESSI_CHECK_LAUNCH();
    }
    hipLaunchKernelGGL(k_raster_soft_op, dim3(block_grid(g)), dim3(64), 0, ctx->stream, g,
                       (const SoftRec*)recs, (const CullRec*)cull, b, radius_px,
                       prev_shifted_depth, (float4*)out);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

inline size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

constexpr int kNoAllocMaxDevices = 64;
std::mutex g_noalloc_mu;
char* g_noalloc_ptr[kNoAllocMaxDevices] = {};
hipEvent_t g_noalloc_done[kNoAllocMaxDevices] = {};      // after the GPU's last call
hipStream_t g_noalloc_stream[kNoAllocMaxDevices] = {};   // the stream of that call
bool g_noalloc_used[kNoAllocMaxDevices] = {};

// The device address of this GPU's scratch array, looked up once per device
// with that device current (the caller has made it current), with its
// ordering event; the caller holds g_noalloc_mu.
int noalloc_scratch(int device, char** out) {
    DRESSI_REQUIRE(device >= 0 && device < kNoAllocMaxDevices, "device %d out of range", device);
    if (!g_noalloc_ptr[device]) {
        void* p = nullptr;
        DRESSI_TRY_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        DRESSI_REQUIRE(p != nullptr, "hipGetSymbolAddress returned NULL");
        DRESSI_TRY_HIP(hipEventCreateWithFlags(&g_noalloc_done[device], hipEventDisableTiming));
        g_noalloc_ptr[device] = (char*)p;
    }
    *out = g_noalloc_ptr[device];
    return DRESSI_OK;
}

bool stream_capturing(hipStream_t s) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(s, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

}  // namespace

extern "C" {

int dressi_soft_clip(dressi_ctx* ctx, const float* clip, uint32_t n_verts, const float* faces,
                     uint32_t n_faces, uint32_t width, uint32_t height, float radius_px,
                     float* out) {
    if (int rc = check_ctx(ctx)) return rc;
    DRESSI_REQUIRE(clip && faces && out, "dressi_soft_clip: NULL buffer");
    DRESSI_REQUIRE(radius_px >= 0.f, "SoftClip: radius_px must be >= 0");
    if (n_faces == 0) return DRESSI_OK;
    hipLaunchKernelGGL(k_soft_clip, dim3(div_up(n_faces, 256)), dim3(256), 0, ctx->stream,
                       (const float4*)clip, n_verts, faces, n_faces, width, height, radius_px,
                       ctx->d_err, (float4*)out);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int dressi_rasterize_soft(dressi_ctx* ctx, const float* soft_clip, const float* face_id,
                          const float* faces_soft, const float* hard_clip, uint32_t n_verts,
                          const float* faces_tex, uint32_t n_faces, uint32_t width,
                          uint32_t height, float radius_px, const float* prev_shifted_depth,
                          float* out) {
    if (int rc = check_ctx(ctx)) return rc;
    if (int rc = check_soft_args(soft_clip, face_id, faces_soft, hard_clip, faces_tex, width,
                                 height, radius_px, out)) return rc;
    const RasterGeom g = make_geom(width, height, 1, n_faces);
    void *recs = nullptr, *bins = nullptr, *cull = nullptr;
    const size_t nf1 = n_faces ? n_faces : 1;
    if (int rc = ctx_workspace(ctx, 0, sizeof(SoftRec) * nf1, &recs)) return rc;
    if (int rc = ctx_workspace(ctx, 1, fixed_bin_bytes(g.n_tiles, kSoftBinCap), &bins)) return rc;
    if (int rc = ctx_workspace(ctx, 3, sizeof(CullRec) * nf1, &cull)) return rc;
    return launch_rasterize_soft(ctx, g, soft_clip, face_id, faces_soft, hard_clip, n_verts,
                                 faces_tex, radius_px, prev_shifted_depth, (SoftRec*)recs, bins,
                                 (CullRec*)cull, out);
}

int dressi_rasterize_soft_noalloc(dressi_ctx* ctx, const float* soft_clip, const float* face_id,
                                  const float* faces_soft, const float* hard_clip,
                                  uint32_t n_verts, const float* faces_tex, uint32_t n_faces,
                                  uint32_t width, uint32_t height, float radius_px,
                                  const float* prev_shifted_depth, float* out) {
    if (int rc = check_ctx(ctx)) return rc;
    if (int rc = check_soft_args(soft_clip, face_id, faces_soft, hard_clip, faces_tex, width,
                                 height, radius_px, out)) return rc;
    const RasterGeom g = make_geom(width, height, 1, n_faces);
    const size_t nf1 = n_faces ? n_faces : 1;
    const size_t rec_bytes = align256(sizeof(SoftRec) * nf1);
    const size_t cull_bytes = align256(sizeof(CullRec) * nf1);
    const size_t bin_bytes_ = fixed_bin_bytes(g.n_tiles, kSoftBinCap);
    const size_t need = rec_bytes + cull_bytes + bin_bytes_;
    DRESSI_REQUIRE(need <= kNoAllocScratchBytes,
                   "dressi_rasterize_soft_noalloc: %u faces on a %ux%u screen need %zu bytes of "
                   "scratch, above the fixed %zu (use dressi_rasterize_soft)",
                   n_faces, width, height, need, kNoAllocScratchBytes);
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    char* base = nullptr;
    if (int rc = noalloc_scratch(ctx->device, &base)) return rc;
    const int dev = ctx->device;
    const bool capturing = stream_capturing(ctx->stream);
    if (!capturing && g_noalloc_used[dev] && g_noalloc_stream[dev] != ctx->stream) {
        DRESSI_TRY_HIP(hipStreamWaitEvent(ctx->stream, g_noalloc_done[dev], 0));
    }
    const int rc = launch_rasterize_soft(ctx, g, soft_clip, face_id, faces_soft, hard_clip,
                                         n_verts, faces_tex, radius_px, prev_shifted_depth,
                                         (SoftRec*)base, base + rec_bytes + cull_bytes,
                                         (CullRec*)(base + rec_bytes), out);
    if (rc == DRESSI_OK && !capturing) {
        DRESSI_TRY_HIP(hipEventRecord(g_noalloc_done[dev], ctx->stream));
        g_noalloc_stream[dev] = ctx->stream;
        g_noalloc_used[dev] = true;
    }
    return rc;
}

// `n_items` clip sets [n_items][n_verts] over one face list; attributes
// shared by the items (attr_view 0) or per item (attr_view = n_verts * n_comp
// floats apart); `ids` (optional) gets RasterizeFaceId's output alongside.
static int rasterize_hard_common(dressi_ctx* ctx, const float* clip, uint32_t n_verts,
                                 const float* attr, uint32_t n_comp, const float* faces,
                                 uint32_t n_faces, uint32_t width, uint32_t height, int mode,
                                 float* out, uint32_t n_items = 1, size_t attr_view = 0,
                                 float* ids = nullptr) {
    if (int rc = check_ctx(ctx)) return rc;
    DRESSI_REQUIRE(clip && (faces || n_faces == 0) && out && (mode == 1 || attr),
                   "rasterize: NULL buffer");
    DRESSI_REQUIRE(width > 0 && height > 0, "rasterize: empty screen");
    DRESSI_REQUIRE(mode == 1 || (n_comp >= 1 && n_comp <= 4), "rasterize: n_comp must be 1..4");
    DRESSI_REQUIRE(n_items >= 1 && (uint64_t)n_items * n_faces < (1ull << 31) &&
                           (uint64_t)n_items * n_verts < (1ull << 31),
                   "rasterize: too many items");
    const RasterGeom g = make_geom(width, height, n_items, n_faces);
    const uint32_t cap = default_bin_cap(g, 8);
    void *recs = nullptr, *bins = nullptr, *fi = nullptr;
    const size_t nf1 = n_faces ? n_faces : 1;
    if (int rc = ctx_workspace(ctx, 0, sizeof(HardRec) * nf1 * n_items, &recs)) return rc;
    if (int rc = ctx_workspace(ctx, 1, bin_bytes(g.n_tiles * n_items, cap), &bins)) return rc;
    if (int rc = ctx_workspace(ctx, 2, sizeof(int32_t) * 3 * nf1, &fi)) return rc;
    BinBuffers b;
    bin_carve(bins, g.n_tiles * n_items, cap, &b);
    if (int rc = launch_zero(ctx->stream, b.counts, sizeof(uint32_t) * g.n_tiles * n_items))
        return rc;
    if (n_faces) {
        hipLaunchKernelGGL(k_faces_to_i32, dim3(div_up(3 * n_faces, 256)), dim3(256), 0,
                           ctx->stream, faces, 3 * n_faces, n_verts, ctx->d_err, (int32_t*)fi);
        DRESSI_CHECK_LAUNCH();
        if (int rc = launch_hard_setup(ctx->stream, g, clip, n_verts, (const int32_t*)fi,
                                       (HardRec*)recs)) return rc;
        if (int rc = launch_count_hard(ctx->stream, g, (const HardRec*)recs, b)) return rc;
    }
    if (int rc = launch_scan_bins(ctx->stream, b)) return rc;
    if (n_faces) {
        if (int rc = launch_bin_hard(ctx->stream, g, (const HardRec*)recs, b)) return rc;
    }
    return launch_raster_hard(ctx->stream, g, (const HardRec*)recs, b, attr, mode == 1 ? 1 : n_comp,
                              mode, out, attr_view, ids);
}

int dressi_rasterize(dressi_ctx* ctx, const float* clip, uint32_t n_verts, const float* attr,
                     uint32_t n_comp, const float* faces, uint32_t n_faces, uint32_t width,
                     uint32_t height, float* out) {
    return rasterize_hard_common(ctx, clip, n_verts, attr, n_comp, faces, n_faces, width,
                                 height, 0, out);
}

int dressi_rasterize_face_id(dressi_ctx* ctx, const float* clip, uint32_t n_verts,
                             const float* faces, uint32_t n_faces, uint32_t width,
                             uint32_t height, float* out) {
    return rasterize_hard_common(ctx, clip, n_verts, nullptr, 1, faces, n_faces, width, height,
                                 1, out);
}

int dressi_rasterize_batch(dressi_ctx* ctx, const float* clip, uint32_t n_verts,
                           uint32_t n_items, const float* attr, uint32_t n_comp,
                           int attr_per_item, const float* faces, uint32_t n_faces,
                           uint32_t width, uint32_t height, float* out, float* face_id) {
    return rasterize_hard_common(ctx, clip, n_verts, attr, n_comp, faces, n_faces, width, height,
                                 0, out, n_items, attr_per_item ? (size_t)n_verts * n_comp : 0,
                                 face_id);
}

}  // extern "C"
