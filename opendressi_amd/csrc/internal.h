// internal.h -- runtime plumbing shared by the library's HIP sources:
// context, error reporting, workspace, and the tile-binned raster driver.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "../../include/dressi_hip.h"
#include "dressi_math.h"

struct dressi_ctx {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;  // current stream (own or caller's)
    // device word the kernels OR error bits into (bad indices); checked and
    // cleared by dressi_ctx_synchronize
    uint32_t* d_err = nullptr;
    // grow-only scratch for the per-op entry points. Each slot remembers the
    // stream of its last use: a call on another stream first waits (event)
    // for that stream, so reuse stays ordered across streams.
    std::vector<void*> ws_ptr;
    std::vector<size_t> ws_size;
    std::vector<hipStream_t> ws_stream;
    std::vector<hipEvent_t> ws_event;
    // bumped whenever a slot is freed and reallocated: a captured hipGraph
    // holding the old addresses is stale once this changes
    uint64_t ws_generation = 0;
};

namespace dressi {

// Items of a batched per-op launch (grid y dimension).
constexpr uint32_t kMaxBatchItems = 65535;

// thread-local last error; every C entry point returns a dressi_status
void set_error(const char* fmt, ...);
void clear_error();

#define DRESSI_TRY_HIP(expr)                                                   \
    do {                                                                       \
        hipError_t _e = (expr);                                                \
        if (_e != hipSuccess) {                                                \
            ::dressi::set_error("%s failed: %s (%s:%d)", #expr,                \
                                hipGetErrorString(_e), __FILE__, __LINE__);    \
            return DRESSI_ERR_HIP;                                             \
        }                                                                      \
    } while (0)

#define DRESSI_REQUIRE(cond, ...)                                              \
    do {                                                                       \
        if (!(cond)) {                                                         \
            ::dressi::set_error(__VA_ARGS__);                                  \
            return DRESSI_ERR_INVALID;                                         \
        }                                                                      \
    } while (0)

#define DRESSI_CHECK_LAUNCH()                                                  \
    do {                                                                       \
        hipError_t _e = hipGetLastError();                                     \
        if (_e != hipSuccess) {                                                \
            ::dressi::set_error("kernel launch failed: %s (%s:%d)",            \
                                hipGetErrorString(_e), __FILE__, __LINE__);    \
            return DRESSI_ERR_HIP;                                             \
        }                                                                      \
    } while (0)

// Workspace slot `i` of at least `bytes` (grow-only; contents undefined, or
// zero-filled on (re)allocation with ctx_workspace_zeroed), ordered on the
// context's current stream after every earlier use of the slot, whatever
// stream that use ran on.
int ctx_workspace(dressi_ctx* ctx, int slot, size_t bytes, void** out);
int ctx_workspace_zeroed(dressi_ctx* ctx, int slot, size_t bytes, void** out);

inline uint32_t div_up(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

// Fills `bytes` (a multiple of 4) at `p` with zero by a kernel on stream `s`
// (not hipMemsetAsync: memset nodes of captured graphs have given wrong
// results on replays, and per-op entry points may be captured).
int launch_zero(hipStream_t s, void* p, size_t bytes);

// ---------------------------------------------------------------------------
// Tile binning (16x16 pixel tiles)
// ---------------------------------------------------------------------------
constexpr int kTile = 16;
constexpr int kTileThreads = kTile * kTile;

// Per (view, face) setup record of the soft rasterizer: soft triangle
// (coverage), hard triangle (signed distance, edge-function filter, hard z)
// and the inclusive soft pixel bbox. 43 words, padded to 44 so that it
// moves with 16-byte loads; the first 16 words (edge functions, orientation,
// flags, hard-branch margin) are what the block cull reads per lane.
struct alignas(16) SoftRec {
    float ex[3], ey[3];   // hard edges a[k+1] - a[k]
    float cc[3], thr[3];  // edge-function filter: ex*py - ey*px + cc, threshold
    float h_inv_area;     // 1 / (2 x signed hard area), 0 if below 1e-6
    uint32_t flags;       // kRecHardArea | kRecSliver | kRecPos
    float s_inv_area;
    float a_margin;       // hard-branch pixels lie within the hard bbox +- this (px)
    float hx[3], hy[3], len2[3], hz[3];
    float sx[3], sy[3], sz[3];
    int bx0, by0, bx1, by1;  // bx0 > bx1: face produces no fragment
    float s_margin;          // soft coverage margin for the block cull, < 0: none
    float fid;               // face_id value written to the output
    float zc;                // >= 0, below the depth of every hard-branch fragment
};
static_assert(sizeof(SoftRec) == 44 * 4, "SoftRec layout");
// SoftRec::flags: the hard triangle's |area| passes the 1e-6 test (hard z is
// interpolated, else 0.5) ...
constexpr uint32_t kRecHardArea = 1u;
// ... and the hard triangle is thin (the winding test's inside may reach
// more than 0.51 px beyond its bbox): it takes the general classifier, and
// its a_margin widens the culls (infinite when no bound holds: the whole
// soft bbox).
constexpr uint32_t kRecSliver = 2u;
// ... and the signed hard area is positive (the orientation that the
// winding test's "inside" takes for a non-sliver face).
constexpr uint32_t kRecPos = 4u;

// Per (view, face) setup record of the hard rasterizer (RasterizeCore).
struct HardRec {
    float x[3], y[3], z[3], inv_w[3];
    float inv_area;
    int idx[3];
    int bx0, by0, bx1, by1;
};
static_assert(sizeof(HardRec) == 20 * 4, "HardRec layout");

// Device buffers of one binning problem: `n_bins` = views x tiles.
// Scan-based bins (hard rasterizer): counts -> offsets -> list[cap].
// Fixed-capacity bins (soft rasterizer): list[bin * cap + slot], counts
// cleared by the consumer; offsets / cursor unused.
struct BinBuffers {
    uint32_t* counts = nullptr;   // [n_bins], zero between uses
    uint32_t* offsets = nullptr;  // [n_bins + 1]
    uint32_t* cursor = nullptr;   // [n_bins]
    uint32_t* list = nullptr;     // [cap] or [n_bins][cap] face indices
    uint32_t cap = 0;
    uint32_t n_bins = 0;
};

// Fixed-capacity soft bins: n_bins counters + n_bins * cap entries.
inline size_t fixed_bin_bytes(uint32_t n_bins, uint32_t cap) {
    return sizeof(uint32_t) * ((size_t)n_bins + (size_t)n_bins * cap) + 256;
}
inline void fixed_bin_carve(void* base, uint32_t n_bins, uint32_t cap, BinBuffers* b) {
    uint32_t* p = (uint32_t*)base;
    b->counts = p;
    b->offsets = nullptr;
    b->cursor = nullptr;
    b->list = p + n_bins;
    b->cap = cap;
    b->n_bins = n_bins;
}
// Entries per soft bin (a 16x16 tile of one view).
constexpr uint32_t kSoftBinCap = 1024;
static_assert(kSoftBinCap >= 64, "bin_view reads a bin's first 64 entries unconditionally");
// Largest entries per bin a fit plan grows its bins to (after an iteration
// whose face backward saw an overflowed bin); past it an overflowed bin
// walks every face of its view.
constexpr uint32_t kSoftBinCapMax = 16384;

struct RasterGeom {
    uint32_t width, height, tiles_x, tiles_y, n_tiles, n_views, n_faces;
    // multipliers for the launch decoders' divisions by n_views, tiles_x and
    // n_tiles (geom_div); 0 where the short form is not exact
    uint32_t views_m, tiles_x_m, tiles_m;
};

// ceil(2^32 / d): then n / d = (n * m) >> 32 exactly for every n with
// n * d < 2^32 (the error n * (m d - 2^32) / (d 2^32) stays below 1 / d);
// 0 when d < 2 or when n_max * d reaches 2^32
inline uint32_t div_magic(uint32_t d, uint64_t n_max) {
    if (d < 2 || n_max * d >= (1ull << 32)) {
        return 0u;
    }
    return (uint32_t)(((1ull << 32) + d - 1) / d);
}

// n / d with the multiplier m of div_magic (m = 0: the plain division)
__host__ __device__ inline uint32_t geom_div(uint32_t n, uint32_t d, uint32_t m) {
    return m ? (uint32_t)(((uint64_t)n * m) >> 32) : n / d;
}

inline RasterGeom make_geom(uint32_t w, uint32_t h, uint32_t views, uint32_t faces) {
    RasterGeom g;
    g.width = w;
    g.height = h;
    g.tiles_x = div_up(w, kTile);
    g.tiles_y = div_up(h, kTile);
    g.n_tiles = g.tiles_x * g.tiles_y;
    g.n_views = views;
    g.n_faces = faces;
    // the decoders divide tile indices (< n_tiles + 8: a grid's last group
    // of 8 may pass the end) by tiles_x, bin indices (< n_tiles n_views) by
    // n_tiles, and tile-group indices (< n_tiles n_views) by n_views
    const uint64_t bins = (uint64_t)g.n_tiles * views;
    g.views_m = div_magic(views, bins);
    g.tiles_x_m = div_magic(g.tiles_x, (uint64_t)g.n_tiles + 8u);
    g.tiles_m = div_magic(g.n_tiles, bins);
    return g;
}

// Kernels shared between raster.hip and hsr.hip (launch helpers).
int launch_scan_bins(hipStream_t s, const BinBuffers& b);
int launch_bin_hard(hipStream_t s, const RasterGeom& g, const HardRec* recs, const BinBuffers& b);
int launch_count_hard(hipStream_t s, const RasterGeom& g, const HardRec* recs, const BinBuffers& b);
// Hard raster of a clip-space mesh into `out` ({views,S,S} x n_comp):
// mode 0 = attribute interpolation, 1 = face id + 1. `clip` is [views][V]
// float4, `faces` int32 [F][3].
int launch_hard_setup(hipStream_t s, const RasterGeom& g, const float* clip, uint32_t n_verts,
                      const int32_t* faces, HardRec* recs);
int launch_raster_hard(hipStream_t s, const RasterGeom& g, const HardRec* recs,
                       const BinBuffers& b, const float* attr, uint32_t n_comp, int mode,
                       float* out, size_t attr_view = 0, float* ids = nullptr);

// Sizes of the binning buffers for a problem; `cap` = list capacity.
size_t bin_bytes(uint32_t n_bins, uint32_t cap);
void bin_carve(void* base, uint32_t n_bins, uint32_t cap, BinBuffers* b);
// Default list capacity: `per_face` tile entries per face and view.
uint32_t default_bin_cap(const RasterGeom& g, uint32_t per_face);

}  // namespace dressi
