// raster_core.h -- device side of the tile-binned rasterizer.
//
// The reference rasterizes face by face over each face's pixel bbox and
// keeps, per pixel, the fragment of minimum depth with later faces winning
// ties (src/core/cpu_raster.cpp:31-110, 241-355). Here every 16x16 tile is
// one workgroup: the faces binned to the tile are staged through LDS in
// chunks of 256 setup records and each lane (one pixel) folds the fragments
// it covers into a 64-bit (depth | ~face) key. The min over keys is
// order-independent, so the atomically filled, unordered tile lists still
// give the reference's deterministic winner.
#pragma once

#include "internal.h"

namespace dressi {

// Soft raster setup of one face (src/core/cpu_raster.cpp:257-303 for the
// soft/hard projections, cpu_raster.cpp:177-193 for the barycentric
// constants). `sc` = soft corner clips, `hc` = hard corner clips.
__device__ __forceinline__ void soft_setup(const float4 sc[3], const float4 hc[3], float fid,
                                           uint32_t w, uint32_t h, SoftRec* r) {
    r->bx0 = 1;
    r->bx1 = 0;
    r->by0 = 1;
    r->by1 = 0;
    r->fid = fid;
    const float W = (float)w, H = (float)h;
    float sx[3], sy[3], hx[3], hy[3];
    for (int k = 0; k < 3; k++) {
        if (!clip_w_valid(sc[k].w)) {
            return;
        }
        const ScreenVert v = project_to_screen(sc[k].x, sc[k].y, sc[k].z, sc[k].w, W, H);
        sx[k] = v.x;
        sy[k] = v.y;
        r->sz[k] = v.z;
    }
    for (int k = 0; k < 3; k++) {
        if (!clip_w_valid(hc[k].w)) {
            return;
        }
        const ScreenVert v = project_to_screen(hc[k].x, hc[k].y, hc[k].z, hc[k].w, W, H);
        hx[k] = v.x;
        hy[k] = v.y;
        r->hz[k] = v.z;
    }
    // ScreenBarycentric on the soft triangle fails for |area| < 1e-6: no
    // pixel passes, so the face is dropped from binning altogether.
    const float s_area = tri_area(sx[0], sy[0], sx[1], sy[1], sx[2], sy[2]);
    if (fabsf(s_area) < kDistEps) {
        return;
    }
    r->s_inv_area = 1.f / s_area;
    const float h_area = tri_area(hx[0], hy[0], hx[1], hy[1], hx[2], hy[2]);
    r->h_area_ok = fabsf(h_area) < kDistEps ? 0 : 1;
    r->h_inv_area = r->h_area_ok ? 1.f / h_area : 0.f;
    for (int k = 0; k < 3; k++) {
        r->sx[k] = sx[k];
        r->sy[k] = sy[k];
    }
    HardTri ht;
    hard_tri_init(&ht, hx, hy);
    for (int k = 0; k < 3; k++) {
        r->hx[k] = ht.ax[k];
        r->hy[k] = ht.ay[k];
        r->ex[k] = ht.ex[k];
        r->ey[k] = ht.ey[k];
        r->len2[k] = ht.len2[k];
    }
    pixel_bbox(sx[0], sx[1], sx[2], sy[0], sy[1], sy[2], (int)w, (int)h, &r->bx0, &r->by0,
               &r->bx1, &r->by1);
}

// One soft fragment (cpu_raster.cpp:307-351). Folds into (best, dist, hz).
__device__ __forceinline__ void soft_fragment(const SoftRec& r, uint32_t f, int px, int py,
                                              float radius, const float* prev_depth,
                                              uint32_t width, uint64_t* best,
                                              float* best_dist, float* best_hz) {
    if (px < r.bx0 || px > r.bx1 || py < r.by0 || py > r.by1) {
        return;
    }
    const float p0 = (float)px + 0.5f;
    const float p1 = (float)py + 0.5f;
    float l0, l1, l2;
    barycentric(p0, p1, r.sx[0], r.sy[0], r.sx[1], r.sy[1], r.sx[2], r.sy[2], r.s_inv_area,
                &l0, &l1, &l2);
    if (l0 < 0.f || l1 < 0.f || l2 < 0.f) {
        return;
    }
    const float soft_z = l0 * r.sz[0] + l1 * r.sz[1] + l2 * r.sz[2];
    if (soft_z < 0.f || soft_z > 1.f) {
        return;
    }
    const float dist = signed_dist(p0, p1, r.hx, r.hy, r.ex, r.ey, r.len2);
    float hard_z = 0.5f;
    if (r.h_area_ok) {
        float h0, h1, h2;
        barycentric(p0, p1, r.hx[0], r.hy[0], r.hx[1], r.hy[1], r.hx[2], r.hy[2], r.h_inv_area,
                    &h0, &h1, &h2);
        hard_z = h0 * r.hz[0] + h1 * r.hz[1] + h2 * r.hz[2];
    }
    const float depth = eq3_depth(dist, hard_z, radius);
    if (prev_depth && depth <= prev_depth[(size_t)py * width + px] + 1e-4f) {
        return;
    }
    const uint64_t key = depth_key(depth, f);
    if (key < *best) {
        *best = key;
        *best_dist = dist;
        *best_hz = hard_z;
    }
}

// Hard raster setup (RasterizeCore, cpu_raster.cpp:42-94).
__device__ __forceinline__ void hard_setup(const float4 c[3], const int idx[3], uint32_t w,
                                           uint32_t h, HardRec* r) {
    r->bx0 = 1;
    r->bx1 = 0;
    r->by0 = 1;
    r->by1 = 0;
    const float W = (float)w, H = (float)h;
    for (int k = 0; k < 3; k++) {
        if (fabsf(c[k].w) <= kWEps || c[k].w < 0.f) {
            return;
        }
    }
    for (int k = 0; k < 3; k++) {
        const ScreenVert v = project_to_screen(c[k].x, c[k].y, c[k].z, c[k].w, W, H);
        r->x[k] = v.x;
        r->y[k] = v.y;
        r->z[k] = v.z;
        r->inv_w[k] = v.inv_w;
        r->idx[k] = idx[k];
    }
    const float area = tri_area(r->x[0], r->y[0], r->x[1], r->y[1], r->x[2], r->y[2]);
    if (fabsf(area) < kDistEps) {
        return;
    }
    r->inv_area = 1.f / area;
    pixel_bbox(r->x[0], r->x[1], r->x[2], r->y[0], r->y[1], r->y[2], (int)w, (int)h, &r->bx0,
               &r->by0, &r->bx1, &r->by1);
}

// One hard fragment (cpu_raster.cpp:76-106): coverage + NDC z test.
__device__ __forceinline__ void hard_fragment(const HardRec& r, uint32_t f, int px, int py,
                                              uint64_t* best) {
    if (px < r.bx0 || px > r.bx1 || py < r.by0 || py > r.by1) {
        return;
    }
    const float p0 = (float)px + 0.5f;
    const float p1 = (float)py + 0.5f;
    float l0, l1, l2;
    barycentric(p0, p1, r.x[0], r.y[0], r.x[1], r.y[1], r.x[2], r.y[2], r.inv_area, &l0, &l1,
                &l2);
    if (l0 < 0.f || l1 < 0.f || l2 < 0.f) {
        return;
    }
    const float z = l0 * r.z[0] + l1 * r.z[1] + l2 * r.z[2];
    if (z < 0.f || z > 1.f) {
        return;
    }
    const uint64_t key = depth_key(z, f);
    if (key < *best) {
        *best = key;
    }
}

// Walks the faces binned to one (view, tile): chunks of up to 256 records are
// staged through LDS and every lane folds each record via `frag(rec, f)`.
// When the bin's list overflowed the capacity the walk covers all faces
// (each face's own bbox test keeps the result exact).
template <typename Rec, typename Frag>
__device__ __forceinline__ void walk_bin(const Rec* recs, const BinBuffers& b, uint32_t bin,
                                         uint32_t n_faces, Rec* lds_rec, uint32_t* lds_face,
                                         Frag&& frag) {
    const uint32_t beg = b.offsets[bin];
    const uint32_t end = b.offsets[bin + 1];
    const bool implicit = end > b.cap;
    const uint32_t n = implicit ? n_faces : end - beg;
    for (uint32_t base = 0; base < n; base += kTileThreads) {
        const uint32_t cnt = (n - base) < (uint32_t)kTileThreads ? (n - base) : kTileThreads;
        __syncthreads();
        if (threadIdx.x < cnt) {
            const uint32_t f = implicit ? base + threadIdx.x : b.list[beg + base + threadIdx.x];
            lds_face[threadIdx.x] = f;
            lds_rec[threadIdx.x] = recs[f];
        }
        __syncthreads();
        for (uint32_t j = 0; j < cnt; j++) {
            frag(lds_rec[j], lds_face[j]);
        }
    }
}

}  // namespace dressi
