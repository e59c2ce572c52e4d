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
    // grow-only scratch for the per-op entry points (stream-ordered reuse)
    std::vector<void*> ws_ptr;
    std::vector<size_t> ws_size;
};

namespace dressi {

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

// Workspace slot `i` of at least `bytes` (grow-only; contents undefined).
int ctx_workspace(dressi_ctx* ctx, int slot, size_t bytes, void** out);

inline uint32_t div_up(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// Tile binning (16x16 pixel tiles)
// ---------------------------------------------------------------------------
constexpr int kTile = 16;
constexpr int kTileThreads = kTile * kTile;

// Per (view, face) setup record of the soft rasterizer: soft triangle
// (coverage), hard triangle (signed distance + hard z) and the inclusive
// pixel bbox. 36 words.
struct SoftRec {
    float sx[3], sy[3];
    float s_inv_area;
    float sz[3];
    float hx[3], hy[3], ex[3], ey[3], len2[3];
    float hz[3];
    float h_inv_area;
    int h_area_ok;
    int bx0, by0, bx1, by1;  // bx0 > bx1: face produces no fragment
    float fid;               // face_id value written to the output
    int pad;
};
static_assert(sizeof(SoftRec) == 36 * 4, "SoftRec layout");

// Per (view, face) setup record of the hard rasterizer (RasterizeCore).
struct HardRec {
    float x[3], y[3], z[3], inv_w[3];
    float inv_area;
    int idx[3];
    int bx0, by0, bx1, by1;
};
static_assert(sizeof(HardRec) == 20 * 4, "HardRec layout");

// Device buffers of one binning problem: `n_bins` = views x tiles.
struct BinBuffers {
    uint32_t* counts = nullptr;   // [n_bins], zero between uses
    uint32_t* offsets = nullptr;  // [n_bins + 1]
    uint32_t* cursor = nullptr;   // [n_bins]
    uint32_t* list = nullptr;     // [cap] face indices
    uint32_t cap = 0;
    uint32_t n_bins = 0;
};

struct RasterGeom {
    uint32_t width, height, tiles_x, tiles_y, n_tiles, n_views, n_faces;
};

inline RasterGeom make_geom(uint32_t w, uint32_t h, uint32_t views, uint32_t faces) {
    RasterGeom g;
    g.width = w;
    g.height = h;
    g.tiles_x = div_up(w, kTile);
    g.tiles_y = div_up(h, kTile);
    g.n_tiles = g.tiles_x * g.tiles_y;
    g.n_views = views;
    g.n_faces = faces;
    return g;
}

// Kernels shared between raster.hip and hsr.hip (launch helpers).
int launch_scan_bins(hipStream_t s, const BinBuffers& b);
int launch_bin_soft(hipStream_t s, const RasterGeom& g, const SoftRec* recs, const BinBuffers& b);
int launch_bin_hard(hipStream_t s, const RasterGeom& g, const HardRec* recs, const BinBuffers& b);
int launch_count_soft(hipStream_t s, const RasterGeom& g, const SoftRec* recs, const BinBuffers& b);
int launch_count_hard(hipStream_t s, const RasterGeom& g, const HardRec* recs, const BinBuffers& b);
// Hard raster of a clip-space mesh into `out` ({views,S,S} x n_comp):
// mode 0 = attribute interpolation, 1 = face id + 1. `clip` is [views][V]
// float4, `faces` int32 [F][3].
int launch_hard_setup(hipStream_t s, const RasterGeom& g, const float* clip, uint32_t n_verts,
                      const int32_t* faces, HardRec* recs);
int launch_raster_hard(hipStream_t s, const RasterGeom& g, const HardRec* recs,
                       const BinBuffers& b, const float* attr, uint32_t n_comp, int mode,
                       float* out);

// Sizes of the binning buffers for a problem; `cap` = list capacity.
size_t bin_bytes(uint32_t n_bins, uint32_t cap);
void bin_carve(void* base, uint32_t n_bins, uint32_t cap, BinBuffers* b);
// Default list capacity: `per_face` tile entries per face and view.
uint32_t default_bin_cap(const RasterGeom& g, uint32_t per_face);

}  // namespace dressi
