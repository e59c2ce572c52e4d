// raster_core.h -- device side of the tile-binned soft rasterizer.
//
// Reference semantics (src/core/cpu_raster.cpp:241-355): faces are rasterised
// one after another over their soft pixel bbox; a fragment passes when the
// pixel centre is inside the soft triangle (inclusive barycentrics) with soft
// z in [0,1]; its depth is the Eq.3 shift of the signed distance to the hard
// triangle (0.5 * clamp(hard_z) when dist >= 0, else
// 0.5 + 0.5 * min(-dist / r, 1)); the minimum depth wins, later faces win ties.
//
// Here one wave owns an 8x8 block of one view. Faces are binned per 16x16
// tile; the wave culls its tile's list against the block (one entry per
// lane, ballot) and walks the survivors with the face record in scalar
// registers; every lane folds the fragments of its pixel into a 64-bit
// (depth | ~face) key, whose minimum is the reference's winner independent of
// processing order. The work is split so that, exactly:
//  * phase A folds hard-branch fragments (pixel inside the hard triangle:
//    depth <= 0.5, no distance needed) and any fragment close enough to a
//    hard edge that the classification needs the full reference evaluation;
//  * phase B folds every other (rim) fragment, but only for lanes whose best
//    depth after phase A is >= 0.5 -- rim depths are >= 0.5, so elsewhere
//    they cannot win. Faces whose hard triangle lies more than r + 1 px from
//    the wave's block contribute depth exactly 1.0 there (-dist/r > 1), so
//    only their coverage is tested.
#pragma once

#include "internal.h"

namespace dressi {

// The smallest |edge function| that can still belong to a pixel centre lying
// exactly on the edge segment (signed distance -0.0 with a negative winding
// test, which the reference puts in the hard branch): with p == q = a + t e
// computed in float, |e x (p - a)| <= u (2|ex||ey| + 4|ex|(|py|+|ay|) +
// 4|ey|(|px|+|ax|)) + O(u^2), u = 2^-24. 2^-20 (...) bounds it with a wide
// margin. Fragments below the bound take the full reference evaluation.
__device__ __forceinline__ float boundary_eps(float ex, float ey, float ax, float ay, float px,
                                              float py) {
    return 0x1p-20f * (fabsf(ex) * fabsf(ey) + fabsf(ex) * (fabsf(py) + fabsf(ay)) +
                       fabsf(ey) * (fabsf(px) + fabsf(ax)));
}

// Soft raster setup of one face (src/core/cpu_raster.cpp:257-303 for the
// soft/hard projections, :177-193 for the barycentric constants).
// `sc` = soft corner clips, `hc` = hard corner clips.
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
    // Soft coverage margin (edge-function units) for the block cull. With s
    // the computed area's sign (exact when |2 area| > 2^-20 P), a pixel the
    // reference's float barycentrics call covered has s * E_k(p) >= -m on
    // each exact edge function E_k (twice the signed area of p and the
    // edge): l0, l1 >= 0 only lose the rounding of E_0, E_1 (<= 4u P_k; the
    // 1 / area factor scales them without changing their sign), and
    // l2 = 1 - l0 - l1 >= 0 adds that, the relative error of the area
    // (<= 4u P) and the final rounding (u (|2 area| + P_0 + P_1)). With
    // Q = sum_k (|x_k| + |x_k+1| + W) (|y_k| + |y_k+1| + H) >= sum_k P_k and
    // P = |x1 - x0| |y2 - y0| + |y1 - y0| |x2 - x0|, m = 16u (Q + P +
    // |2 area|) covers these and the block evaluation.
    {
        float q = 0.f;
        for (int k = 0; k < 3; k++) {
            const int k1 = (k + 1) % 3;
            q += (fabsf(sx[k]) + fabsf(sx[k1]) + W) * (fabsf(sy[k]) + fabsf(sy[k1]) + H);
        }
        const float pa = fabsf(sx[1] - sx[0]) * fabsf(sy[2] - sy[0]) +
                         fabsf(sy[1] - sy[0]) * fabsf(sx[2] - sx[0]);
        const float m = 0x1p-20f * (q + pa + fabsf(s_area));
        r->s_margin = (fabsf(s_area) > 0x1p-20f * pa && m < INFINITY) ? m : -1.f;
    }
    const float h_area = tri_area(hx[0], hy[0], hx[1], hy[1], hx[2], hy[2]);
    const bool area_ok = !(fabsf(h_area) < kDistEps);
    r->h_inv_area = area_ok ? 1.f / h_area : 0.f;
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
        // affine form of the edge function, cr = ex*py - ey*px + cc, used
        // only as a filter: |fma form - reference form| stays below
        // 2^-21 (|ex|(|py|+|ay|) + |ey|(|px|+|ax|)) on screen coordinates
        r->cc[k] = ht.ey[k] * ht.ax[k] - ht.ex[k] * ht.ay[k];
        // filter threshold: boundary_eps + that error, with the screen size
        // bounding |px|, |py| (positive for every finite edge)
        r->thr[k] = 0x1p-19f * (fabsf(ht.ex[k]) * fabsf(ht.ey[k]) +
                                fabsf(ht.ex[k]) * (H + 1.f + fabsf(ht.ay[k])) +
                                fabsf(ht.ey[k]) * (W + 1.f + fabsf(ht.ax[k])));
    }
    // thr[k] also bounds the rounding error of the reference's edge function
    // (8x margin), so a pixel centre its winding test puts inside has exact
    // barycentrics >= -m, m = max thr / |2 area|, and lies within the hard
    // bbox widened by 2 m max(bbox w, h). Unless that is < 0.51 px (|2 area|
    // > 4 thr w; the 4 also absorbs the rounding of h_area) the face is a
    // sliver and the resolver may not cull it by its hard bbox.
    const float thr_max = smax(smax(r->thr[0], r->thr[1]), r->thr[2]);
    const float wmax = smax(smax(smax(hx[0], hx[1]), hx[2]) - smin(smin(hx[0], hx[1]), hx[2]),
                            smax(smax(hy[0], hy[1]), hy[2]) - smin(smin(hy[0], hy[1]), hy[2]));
    // (|2 area| > 8 thr also rules out a winding test that calls a pixel
    // inside with the orientation opposite to the area's sign: the three
    // exact edge functions sum to 2 area)
    // (a hard area below the 1e-6 test leaves no orientation: also a sliver)
    const bool sliver = !area_ok || !(fabsf(h_area) > smax(4.f * thr_max * wmax, 8.f * thr_max)) ||
                        !(fabsf(h_area) < INFINITY);
    r->flags = (area_ok ? kRecHardArea : 0u) | (sliver ? kRecSliver : 0u) |
               (h_area > 0.f ? kRecPos : 0u);
    // Hard-branch margin. Non-slivers: 1 px (the bound above gives 0.51).
    // Slivers whose |2 area| exceeds 16 thr (the winding test cannot take the
    // opposite orientation) and whose computed area has the exact sign
    // (|2 area| > 2^-20 P, P the products of its corner differences): exact
    // barycentrics >= -m with m <= 2 thr / |2 area| (the computed area is
    // within a factor 2), so inside pixels lie within the bbox widened by
    // 2 m wmax. Other slivers: no bound.
    if (!sliver) {
        r->a_margin = 1.f;
    } else {
        const float pa = fabsf(hx[1] - hx[0]) * fabsf(hy[2] - hy[0]) +
                         fabsf(hy[1] - hy[0]) * fabsf(hx[2] - hx[0]);
        const float ah = fabsf(h_area);
        const float mg = 1.f + 4.f * thr_max * wmax / ah;
        r->a_margin = (area_ok && ah > 16.f * thr_max && ah > 0x1p-20f * pa && mg < 1e6f)
                              ? mg
                              : INFINITY;
    }
    // Depth floor of the hard branch (0.5 clamp(hard z), non-slivers; 0 for
    // the others, which the resolver never skips). Its pixels lie within the
    // hard bbox + 1 px, so each product of the barycentric formula is at
    // most (wmax + 2)^2 and the computed barycentrics are >= -eps, eps
    // covering the winding test's margin (thr) and their rounding (as the
    // soft margin, with that product bound) twice over. With
    // sum_k h_k = 1 +- 2.01u, hard z >= zmin - 2 eps (zmax - zmin) - 4u (1 +
    // 6 eps) max |z|; the floor takes twice these terms and one more
    // 2^-20 max |z|.
    r->zc = 0.f;
    if (!sliver) {
        const float zmin = smin(smin(r->hz[0], r->hz[1]), r->hz[2]);
        const float zmax = smax(smax(r->hz[0], r->hz[1]), r->hz[2]);
        const float zabs = smax(fabsf(zmin), fabsf(zmax));
        const float ah = fabsf(h_area);
        const float pa = fabsf(hx[1] - hx[0]) * fabsf(hy[2] - hy[0]) +
                         fabsf(hy[1] - hy[0]) * fabsf(hx[2] - hx[0]);
        const float ext = wmax + 2.f;
        const float eps =
                2.f * (thr_max + 0x1p-20f * (6.f * ext * ext + pa + ah)) / ah;
        const float zlb = zmin - 2.f * (2.f * eps * (zmax - zmin) +
                                        0x1p-22f * (1.f + 6.f * eps) * zabs) -
                          0x1p-20f * zabs;
        if (zlb > 0.f && zlb < INFINITY && eps < 1e6f) {
            r->zc = 0.5f * smin(zlb, 1.f) * (1.f - 0x1p-20f);
        }
    }
    pixel_bbox(sx[0], sx[1], sx[2], sy[0], sy[1], sy[2], (int)w, (int)h, &r->bx0, &r->by0,
               &r->bx1, &r->by1);
}

// Result of one pixel's fold: key + whether the winner is a hard-branch
// fragment (signed distance >= 0).
struct PixelBest {
    uint64_t key;
    bool hard;
};

__device__ __forceinline__ void fold(PixelBest& b, float depth, uint32_t f, bool hard) {
    const uint64_t key = depth_key(depth, f);
    if (key < b.key) {
        b.key = key;
        b.hard = hard;
    }
}

// Exact soft-coverage test of the reference (barycentrics >= 0, soft z in
// [0,1]); the pixel bbox test is done by the caller.
__device__ __forceinline__ bool soft_covers(const SoftRec& r, float p0, float p1) {
    float l0, l1, l2;
    barycentric(p0, p1, r.sx[0], r.sy[0], r.sx[1], r.sy[1], r.sx[2], r.sy[2], r.s_inv_area, &l0,
                &l1, &l2);
    if (l0 < 0.f || l1 < 0.f || l2 < 0.f) {
        return false;
    }
    const float soft_z = l0 * r.sz[0] + l1 * r.sz[1] + l2 * r.sz[2];
    return !(soft_z < 0.f || soft_z > 1.f);
}

__device__ __forceinline__ float hard_z_at(const SoftRec& r, float p0, float p1) {
    float hard_z = 0.5f;
    if (r.flags & kRecHardArea) {
        float h0, h1, h2;
        barycentric(p0, p1, r.hx[0], r.hy[0], r.hx[1], r.hy[1], r.hx[2], r.hy[2], r.h_inv_area,
                    &h0, &h1, &h2);
        hard_z = h0 * r.hz[0] + h1 * r.hz[1] + h2 * r.hz[2];
    }
    return hard_z;
}

// Fragment class w.r.t. the hard triangle: 0 = hard branch (dist >= 0),
// 1 = rim (dist < 0, and not -0), 2 = needs the full reference evaluation.
// Non-sliver faces: the winding test can only say inside with the area's
// orientation s, so every s * edge function clear above its threshold gives
// 0, and one clearly below -threshold gives 1 (the pixel is strictly
// outside, at least thr / |e| >= 2^-19 min(W, H) px from the edge line, far
// above the rounding of the distance, so d2 > 0). Slivers: all edge functions
// clear with one sign gives 0, with mixed signs 1; else the exact crosses
// decide, and a pixel within the boundary bound of an edge gives 2.
__device__ __forceinline__ int frag_class(const SoftRec& r, float p0, float p1) {
    float e[3];
#pragma unroll
    for (int k = 0; k < 3; k++) {
        e[k] = fmaf(r.ex[k], p1, fmaf(-r.ey[k], p0, r.cc[k]));
    }
    if (!(r.flags & kRecSliver)) {
        bool in = true, out = false;
        if (r.flags & kRecPos) {
#pragma unroll
            for (int k = 0; k < 3; k++) {
                in = in && e[k] > r.thr[k];
                out = out || e[k] < -r.thr[k];
            }
        } else {
#pragma unroll
            for (int k = 0; k < 3; k++) {
                in = in && e[k] < -r.thr[k];
                out = out || e[k] > r.thr[k];
            }
        }
        return in ? 0 : (out ? 1 : 2);
    }
    bool pos = true, neg = true, clear = true;
#pragma unroll
    for (int k = 0; k < 3; k++) {
        const bool big = fabsf(e[k]) > r.thr[k];
        clear = clear && big;
        pos = pos && e[k] > 0.f;
        neg = neg && e[k] < 0.f;
    }
    if (clear) {
        return (pos || neg) ? 0 : 1;
    }
    // exact reference crosses (cpu_raster.cpp:141-144) and boundary test
    int n_pos = 0, n_neg = 0;
    bool near = false;
#pragma unroll
    for (int k = 0; k < 3; k++) {
        const float cr = r.ex[k] * (p1 - r.hy[k]) - r.ey[k] * (p0 - r.hx[k]);
        n_pos += (cr >= 0.f);
        n_neg += (cr <= 0.f);
        near = near || fabsf(cr) <= boundary_eps(r.ex[k], r.ey[k], r.hx[k], r.hy[k], p0, p1);
    }
    if (n_pos == 3 || n_neg == 3) {
        return 0;
    }
    return near ? 2 : 1;
}

// Phase A fragment: hard branch and full-evaluation fragments. `inside`:
// the wave's block lies inside the soft bbox (no per-pixel bbox test).
__device__ __forceinline__ void frag_phase_a(const SoftRec& r, uint32_t f, int px, int py,
                                             bool inside, float radius, const float* prev,
                                             uint32_t width, PixelBest& b) {
    if (!inside && (px < r.bx0 || px > r.bx1 || py < r.by0 || py > r.by1)) {
        return;
    }
    const float p0 = (float)px + 0.5f;
    const float p1 = (float)py + 0.5f;
    const int cls = frag_class(r, p0, p1);
    if (cls == 1) {
        return;
    }
    float depth;
    bool hard;
    if (cls == 0) {
        depth = 0.5f * smin(smax(hard_z_at(r, p0, p1), 0.f), 1.f);
        hard = true;
    } else {
        const float dist = signed_dist(p0, p1, r.hx, r.hy, r.ex, r.ey, r.len2);
        depth = eq3_depth(dist, hard_z_at(r, p0, p1), radius);
        hard = dist >= 0.f;
    }
    if (prev && depth <= prev[(size_t)py * width + px] + 1e-4f) {
        return;
    }
    // the fragment exists only where the soft triangle covers the pixel;
    // testing that after the depth compare skips it for losing fragments
    const uint64_t key = depth_key(depth, f);
    if (key >= b.key || !soft_covers(r, p0, p1)) {
        return;
    }
    b.key = key;
    b.hard = hard;
}

// Phase B fragment (lanes whose best depth is >= 0.5): every fragment phase
// A did not fold. `in_a`: the face passed phase A's cull for this block (its
// class 0 / 2 fragments were folded there). `near`: the face's hard triangle
// is within r + a_margin px of the pixels phase B folds; otherwise every
// covered one of them is farther and its depth is exactly 1.0.
__device__ __forceinline__ void frag_phase_b(const SoftRec& r, uint32_t f, int px, int py,
                                             float radius, const float* prev, uint32_t width,
                                             bool near, bool in_a, PixelBest& b) {
    if (px < r.bx0 || px > r.bx1 || py < r.by0 || py > r.by1) {
        return;
    }
    const float p0 = (float)px + 0.5f;
    const float p1 = (float)py + 0.5f;
    float depth;
    bool hard = false;
    if (near) {
        if (in_a && frag_class(r, p0, p1) != 1) {
            return;  // folded in phase A
        }
        if (!soft_covers(r, p0, p1)) {
            return;
        }
        const float dist = signed_dist(p0, p1, r.hx, r.hy, r.ex, r.ey, r.len2);
        hard = dist >= 0.f;
        depth = eq3_depth(dist, hard ? hard_z_at(r, p0, p1) : 0.5f, radius);
    } else {
        if (depth_key(1.f, f) >= b.key) {
            return;  // cannot beat the current winner
        }
        if (!soft_covers(r, p0, p1)) {
            return;
        }
        depth = 1.f;
    }
    if (prev && depth <= prev[(size_t)py * width + px] + 1e-4f) {
        return;
    }
    fold(b, depth, f, hard);
}

// Per (view, face) cull record: the soft pixel bbox and the pixels whose
// centres may lie within the hard triangle's bbox +-1 px (all of the soft
// bbox for slivers or non-finite corners), inclusive ranges. 16 bytes.
struct CullRec {
    int16_t sx0, sy0, sx1, sy1;
    int16_t ax0, ay0, ax1, ay1;
};
static_assert(sizeof(CullRec) == 16, "CullRec layout");

__device__ __forceinline__ CullRec cull_setup(const SoftRec& r) {
    CullRec c;
    if (r.bx0 > r.bx1 || r.by0 > r.by1) {
        c.sx0 = c.sy0 = c.ax0 = c.ay0 = 1;
        c.sx1 = c.sy1 = c.ax1 = c.ay1 = 0;
        return c;
    }
    c.sx0 = (int16_t)r.bx0;
    c.sy0 = (int16_t)r.by0;
    c.sx1 = (int16_t)r.bx1;
    c.sy1 = (int16_t)r.by1;
    int ax0 = r.bx0, ay0 = r.by0, ax1 = r.bx1, ay1 = r.by1;
    if (r.a_margin < INFINITY) {
        // centre px + 0.5 in [min - a, max + a]  <=>  px in [min - a - 0.5,
        // max + a - 0.5]; one extra pixel each side absorbs the rounding.
        // fminf / fmaxf keep NaN corners conservative (the whole soft bbox).
        const float a = r.a_margin;
        const float mnx = smin(smin(r.hx[0], r.hx[1]), r.hx[2]);
        const float mxx = smax(smax(r.hx[0], r.hx[1]), r.hx[2]);
        const float mny = smin(smin(r.hy[0], r.hy[1]), r.hy[2]);
        const float mxy = smax(smax(r.hy[0], r.hy[1]), r.hy[2]);
        const int lx = (int)fmaxf(floorf(mnx - a - 0.5f), -4.f) - 1;
        const int hx = (int)fminf(ceilf(mxx + a - 0.5f), 32000.f) + 1;
        const int ly = (int)fmaxf(floorf(mny - a - 0.5f), -4.f) - 1;
        const int hy = (int)fminf(ceilf(mxy + a - 0.5f), 32000.f) + 1;
        ax0 = max(ax0, lx);
        ax1 = min(ax1, hx);
        ay0 = max(ay0, ly);
        ay1 = min(ay1, hy);
    }
    c.ax0 = (int16_t)ax0;
    c.ay0 = (int16_t)ay0;
    c.ax1 = (int16_t)ax1;
    c.ay1 = (int16_t)ay1;
    return c;
}

// Separating-axis test of a hard triangle with a finite a_margin (non-sliver
// or bounded sliver) against the 8x8 block
// along its three edge normals. A pixel centre the reference's winding test
// puts inside (or on the boundary) has, for the triangle's orientation s,
// s * (exact edge function) >= -thr[k] on every edge, and the filter form
// and this corner maximum add at most thr[k] / 4 of rounding: the block can
// hold such a pixel only if no edge's maximum over its pixel centres is below
// -2 thr[k]. `w` = the record's first 16 words.
__device__ __forceinline__ bool edges_reach_block(const float* w, int bx, int by) {
    if (!(w[15] < INFINITY)) {
        return true;  // no hard-branch bound (a_margin)
    }
    const float s = w[12] > 0.f ? 1.f : -1.f;  // orientation (sign of 1 / area)
    const float x0 = (float)bx + 0.5f, x1 = (float)bx + 7.5f;
    const float y0 = (float)by + 0.5f, y1 = (float)by + 7.5f;
    bool hit = true;
#pragma unroll
    for (int k = 0; k < 3; k++) {
        const float a = s * w[k];       // s * ex
        const float b = -s * w[3 + k];  // -s * ey
        const float m = s * w[6 + k] + smax(a * y0, a * y1) + smax(b * x0, b * x1);
        hit = hit && !(m < -2.f * w[9 + k]);
    }
    return hit;
}

// Separating-axis test of the soft triangle (corners x[k], y[k], orientation
// sign of s_inv_area) against the pixel centres of a rectangle of pixels
// [px0, px1] x [py0, py1] along its three edge normals, with the record's
// soft margin m: false only when no pixel centre of the rectangle can be
// covered (per lane, one face per lane).
__device__ __forceinline__ bool soft_reaches_rect(const float (&x)[3], const float (&y)[3],
                                                  float s_inv_area, float m, int px0, int py0,
                                                  int px1, int py1) {
    if (!(m >= 0.f)) {
        return true;
    }
    const float s = s_inv_area > 0.f ? 1.f : -1.f;
    const float x0 = (float)px0 + 0.5f, x1 = (float)px1 + 0.5f;
    const float y0 = (float)py0 + 0.5f, y1 = (float)py1 + 0.5f;
    bool hit = true;
#pragma unroll
    for (int k = 0; k < 3; k++) {
        const int k1 = (k + 1) % 3;
        const float ex = s * (x[k1] - x[k]);
        const float ey = s * (y[k1] - y[k]);
        // max over the block of s * (ex (py - y_k) - ey (px - x_k))
        const float g = smax(ex * (y0 - y[k]), ex * (y1 - y[k])) +
                        smax(-ey * (x0 - x[k]), -ey * (x1 - x[k]));
        hit = hit && !(g < -m);
    }
    return hit;
}

// Inclusive box [x0, x1] x [y0, y1] meets the 8x8 block at (bx, by).
__device__ __forceinline__ bool box_hits(int x0, int y0, int x1, int y1, int bx, int by) {
    return x0 <= bx + 7 && x1 >= bx && y0 <= by + 7 && y1 >= by;
}

// Pixel rectangle [x0, x1] x [y0, y1] of a block: the lanes of a wave mask
// (lane = 8 * row + column) span it; the whole block for a full mask.
struct PixRect {
    int x0, y0, x1, y1;
};
__device__ __forceinline__ PixRect lanes_rect(uint64_t m, int bx, int by) {
    uint32_t cols = 0u, rows = 0u;
#pragma unroll
    for (int r = 0; r < 8; r++) {
        const uint32_t row = (uint32_t)(m >> (8 * r)) & 0xffu;
        cols |= row;
        rows |= row ? 1u << r : 0u;
    }
    PixRect q;
    q.x0 = bx + (int)__builtin_ctz(cols | 0x100u);
    q.x1 = bx + 31 - (int)__builtin_clz(cols | 1u);
    q.y0 = by + (int)__builtin_ctz(rows | 0x100u);
    q.y1 = by + 31 - (int)__builtin_clz(rows | 1u);
    return q;
}

// What the block culls read of one face, loaded together (one round trip):
// the cull record, the record's first 16 words (edge functions, orientation,
// flags, hard-branch margin) and, for phase B, the soft triangle and its
// coverage margin.
struct CullLoad {
    CullRec c;
    float w[16];
    float zc;  // phase A
    float sx[3], sy[3], s_margin;
    float hx[3], hy[3];
};

template <bool kSoft>
__device__ __forceinline__ CullLoad load_cull(const SoftRec* recs, const CullRec* cull,
                                              uint32_t f) {
    CullLoad l;
    l.c = cull[f];
    const float4* q = (const float4*)(recs + f);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 v = q[i];
        l.w[4 * i + 0] = v.x;
        l.w[4 * i + 1] = v.y;
        l.w[4 * i + 2] = v.z;
        l.w[4 * i + 3] = v.w;
    }
    if (!kSoft) {
        l.zc = recs[f].zc;
    }
    if (kSoft) {
        const float4 a = *(const float4*)&recs[f].sx[0];  // sx0 sx1 sx2 sy0
        const float2 b = *(const float2*)&recs[f].sy[1];  // sy1 sy2
        l.sx[0] = a.x;
        l.sx[1] = a.y;
        l.sx[2] = a.z;
        l.sy[0] = a.w;
        l.sy[1] = b.x;
        l.sy[2] = b.y;
        l.s_margin = recs[f].s_margin;
        const float4 h = *(const float4*)&recs[f].hx[0];  // hx0 hx1 hx2 hy0
        const float2 g = *(const float2*)&recs[f].hy[1];  // hy1 hy2
        l.hx[0] = h.x;
        l.hx[1] = h.y;
        l.hx[2] = h.z;
        l.hy[0] = h.w;
        l.hy[1] = g.x;
        l.hy[2] = g.y;
    }
    return l;
}

// The face takes part in phase A for the block: its A-box (and, with
// `soft`, its soft bbox) meets the block and its edges do not separate it
// (per lane, one face per lane).
__device__ __forceinline__ bool cull_in_a(const CullLoad& l, int bx, int by, bool soft) {
    if (soft && !box_hits(l.c.sx0, l.c.sy0, l.c.sx1, l.c.sy1, bx, by)) {
        return false;
    }
    if (!box_hits(l.c.ax0, l.c.ay0, l.c.ax1, l.c.ay1, bx, by)) {
        return false;
    }
    return edges_reach_block(l.w, bx, by);
}

// Sign of 1 / (2 hard area) of a loaded face: the faces with a positive
// one are deferred by phase A.
__device__ __forceinline__ bool cull_pos(const CullLoad& l) { return l.w[12] > 0.f; }

// The soft triangle of a loaded face can cover a pixel centre of the
// rectangle.
__device__ __forceinline__ bool cull_soft(const CullLoad& l, const PixRect& q) {
    return l.c.sx0 <= q.x1 && l.c.sx1 >= q.x0 && l.c.sy0 <= q.y1 && l.c.sy1 >= q.y0 &&
           soft_reaches_rect(l.sx, l.sy, l.w[14], l.s_margin, q.x0, q.y0, q.x1, q.y1);
}

// Number of list entries of a bin and whether it overflowed (then every face
// of the view is walked; each face's own bbox keeps the result exact).
// `pre` = the list's entry at the calling lane (a bin has room for at least
// 64 entries), loaded together with the counter.
struct BinView {
    const uint32_t* list;
    uint32_t n;
    bool implicit;
    uint32_t pre;
    uint32_t count;  // the bin's counter
};

__device__ __forceinline__ BinView bin_view(const BinBuffers& b, uint32_t bin, uint32_t n_faces) {
    BinView v;
    v.list = b.list + (size_t)bin * b.cap;
    const uint32_t cnt = b.counts[bin];
    v.pre = v.list[threadIdx.x & 63u];
    v.implicit = cnt > b.cap;
    v.n = v.implicit ? n_faces : cnt;
    v.count = cnt;
    return v;
}

// 8x8 pixel block of a workgroup. Workgroups are dispatched to the 8 XCDs
// round robin (workgroup i runs on XCD i % 8): tiles are dealt to the XCDs
// round robin too, and the four blocks of a 16x16 tile run on one XCD.
struct BlockPos {
    uint32_t tile;
    int bx, by;
    bool valid;
};

inline uint32_t block_grid(const RasterGeom& g) { return 32u * ((g.n_tiles + 7u) / 8u); }

__device__ __forceinline__ BlockPos block_pos(uint32_t wg, const RasterGeom& g) {
    const uint32_t per = (g.n_tiles + 7u) / 8u;
    const uint32_t k = wg >> 3;
    BlockPos b;
    b.tile = (k >> 2) * 8u + (wg & 7u);
    const uint32_t q = k & 3u;
    const uint32_t trow = geom_div(b.tile, g.tiles_x, g.tiles_x_m);
    b.bx = (int)((b.tile - trow * g.tiles_x) * kTile + (q & 1u) * 8u);
    b.by = (int)(trow * kTile + (q >> 1) * 8u);
    b.valid = (k >> 2) < per && b.tile < g.n_tiles && b.bx < (int)g.width && b.by < (int)g.height;
    return b;
}

// The record's hard-triangle bbox widened by a_margin + `d` px overlaps the
// pixel-centre rectangle [cx0, cx1] x [cy0, cy1] (always true without a
// bound).
__device__ __forceinline__ bool hard_bbox_near(const float (&hx)[3], const float (&hy)[3],
                                               float a_margin, float cx0, float cx1, float cy0,
                                               float cy1, float d) {
    if (!(a_margin < INFINITY)) {
        return true;
    }
    d += a_margin;
    const float mnx = smin(smin(hx[0], hx[1]), hx[2]);
    const float mxx = smax(smax(hx[0], hx[1]), hx[2]);
    const float mny = smin(smin(hy[0], hy[1]), hy[2]);
    const float mxy = smax(smax(hy[0], hy[1]), hy[2]);
    return !(cx0 > mxx + d || cx1 < mnx - d || cy0 > mxy + d || cy1 < mny - d);
}

// Uniform record read: the face index is wave-uniform, so the record comes
// in through scalar loads (the constant address space) instead of LDS.
typedef const __attribute__((address_space(4))) uint32_t* UniformWordPtr;

__device__ __forceinline__ SoftRec load_rec_uniform(const SoftRec* recs, uint32_t f) {
    constexpr int kWords = (int)(sizeof(SoftRec) / 4);
    const UniformWordPtr src = (UniformWordPtr)(recs + f);
    union {
        SoftRec r;
        uint32_t w[kWords];
    } u;
#pragma unroll
    for (int i = 0; i < kWords; i++) {
        u.w[i] = src[i];
    }
    return u.r;
}

// LDS of one resolving wave: survivor records staged per batch and the
// deferred (back) faces of phase A.
constexpr int kStage = 16;
constexpr uint32_t kLaterCap = 512;
constexpr uint32_t kFarCap = 512;
struct ResolveLds {
    SoftRec rec[kStage];
    union {
        struct {
            uint32_t later[kLaterCap];  // phase A: deferred faces
            float later_zc[kLaterCap];  // and their depth floors
        };
        uint32_t far[kFarCap];  // phase B: far faces (as face + 1)
    };
};

// Orders the LDS accesses of one wave around an exchange between its lanes
// (a wave executes its LDS instructions in order).
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Sorts key[0 .. n) descending (bitonic network over the next power of two,
// padded with zeros, which sort last). One wave; n <= kFarCap.
__device__ __forceinline__ void sort_desc(uint32_t* key, uint32_t n) {
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t np = 2;
    while (np < n) {
        np <<= 1;
    }
    for (uint32_t i = n + lane; i < np; i += 64) {
        key[i] = 0u;
    }
    wave_lds_fence();
    for (uint32_t k = 2; k <= np; k <<= 1) {
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t i = lane; i < np; i += 64) {
                const uint32_t ixj = i ^ j;
                if (ixj > i) {
                    const uint32_t a = key[i], b = key[ixj];
                    // runs with (i & k) == 0 descend, the others ascend; the
                    // last merge (k = np) descends over the whole range
                    const bool desc = (i & k) == 0u;
                    if (desc ? a < b : a > b) {
                        key[i] = b;
                        key[ixj] = a;
                    }
                }
            }
            wave_lds_fence();
        }
    }
}

__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Visits the faces of the lanes set in `m` (lane j holds face f), in lane
// order. Their records are staged through LDS in batches of kStage: the
// batch's lanes copy their own record with vector loads (all in flight at
// once), then every lane reads each staged record (an LDS broadcast).
// `visit(rec, face, lane j)`. Single-wave workgroups only.
template <typename Visit>
__device__ __forceinline__ void visit_staged(const SoftRec* recs, uint32_t f, uint64_t m,
                                             ResolveLds& lds, Visit&& visit) {
    const int lane = threadIdx.x & 63;
    while (m) {
        const uint32_t rank = lanes_below(m);
        if (((m >> lane) & 1ull) && rank < (uint32_t)kStage) {
            const float4* src = (const float4*)(recs + f);
            float4* dst = (float4*)&lds.rec[rank];
#pragma unroll
            for (int i = 0; i < (int)(sizeof(SoftRec) / 16); i++) {
                dst[i] = src[i];
            }
        }
        __syncthreads();
        for (int slot = 0; slot < kStage && m; slot++) {
            const int j = __builtin_ctzll(m);
            m &= m - 1;
            const uint32_t fj = (uint32_t)__builtin_amdgcn_readlane((int)f, j);
            const SoftRec r = lds.rec[slot];
            visit(r, fj, j);
        }
        __syncthreads();
    }
}

// Phase B of one 8x8 block (lane = pixel): for the lanes with `need` (best
// depth >= 0.5 after phase A), the fragments phase A did not fold.
__device__ __forceinline__ void phase_b(const SoftRec* recs, const CullRec* cull, const BinView& bv,
                                        int bx, int by, float radius, const float* prev,
                                        uint32_t width, bool need, ResolveLds& lds,
                                        PixelBest& best) {
    const int lane = threadIdx.x & 63;
    const int px = bx + (lane & 7);
    const int py = by + (lane >> 3);
    const float near_d = radius;  // + the face's a_margin
    // Only the lanes with `need` fold here, so the culls and the near / far
    // split below take the rectangle those lanes span (at the limb often a
    // few pixels of the block): a face that cannot cover it, or whose hard
    // triangle lies more than r + a_margin from it, changes no such lane.
    const PixRect nr = lanes_rect(__ballot(need), bx, by);
    const float cx0 = (float)nr.x0 + 0.5f, cx1 = (float)nr.x1 + 0.5f;
    const float cy0 = (float)nr.y0 + 0.5f, cy1 = (float)nr.y1 + 0.5f;
    // Near faces (the hard triangle within r + a_margin of the block, or
    // folded in phase A) are folded as they come. Far faces give depth
    // exactly 1.0 at every pixel they cover, so among them the highest face
    // index wins: they are collected (up to kFarCap; the rest fold at once),
    // sorted by descending index and folded until no pixel that needs
    // phase B can still take a later (lower) one.
    uint32_t n_far = 0;
    for (uint32_t base = 0; base < bv.n; base += 64) {
        const uint32_t e = base + (uint32_t)lane;
        uint32_t f = 0;
        bool keep = false, in_a = false, near = false;
        if (e < bv.n) {
            f = bv.implicit ? e : (base == 0 ? bv.pre : bv.list[e]);
            const CullLoad l = load_cull<true>(recs, cull, f);
            keep = cull_soft(l, nr);
            in_a = keep && cull_in_a(l, bx, by, false);
            near = in_a || hard_bbox_near(l.hx, l.hy, l.w[15], cx0, cx1, cy0, cy1, near_d);
        }
        bool far = keep && !near;
        const uint64_t mf0 = __ballot(far);
        far = far && n_far + lanes_below(mf0) < kFarCap;
        const uint64_t mf = __ballot(far);
        if (far) {
            lds.far[n_far + lanes_below(mf)] = f + 1u;
        }
        n_far += (uint32_t)__popcll(mf);
        const uint64_t ma = __ballot(in_a);
        const uint64_t mn = __ballot(near);
        visit_staged(recs, f, __ballot(keep && !far), lds, [&](const SoftRec& r, uint32_t fj, int j) {
            if (need) {
                frag_phase_b(r, fj, px, py, radius, prev, width, (mn >> j) & 1ull,
                             (ma >> j) & 1ull, best);
            }
        });
    }
    if (n_far) {
        __syncthreads();
        sort_desc(lds.far, n_far);
        for (uint32_t b0 = 0; b0 < n_far; b0 += (uint32_t)kStage) {
            // the batch's first face has the highest index left
            const uint32_t f0 = lds.far[b0] - 1u;
            if (!__any(need && best.key > depth_key(1.f, f0))) {
                break;
            }
            const uint32_t cnt = min((uint32_t)kStage, n_far - b0);
            uint32_t f = 0;
            if ((uint32_t)lane < cnt) {
                f = lds.far[b0 + lane] - 1u;
                const float4* src = (const float4*)(recs + f);
                float4* dst = (float4*)&lds.rec[lane];
#pragma unroll
                for (int i = 0; i < (int)(sizeof(SoftRec) / 16); i++) {
                    dst[i] = src[i];
                }
            }
            __syncthreads();
            for (uint32_t j = 0; j < cnt; j++) {
                const uint32_t fj = (uint32_t)__builtin_amdgcn_readlane((int)f, (int)j);
                const SoftRec r = lds.rec[j];
                if (need) {
                    frag_phase_b(r, fj, px, py, radius, prev, width, false, false, best);
                }
            }
            __syncthreads();
        }
    }
}

// Resolves the winner of every pixel of one 8x8 block (lane = pixel, one
// wave, no cross-wave synchronisation). `recs` / `cull` point at the view's
// records. Phase A folds the class 0 / 2 fragments of faces whose A-box
// meets the block; phase B, run only if some lane's best depth is >= 0.5,
// folds the rest for those lanes. Every hard-branch fragment (depth <= 0.5)
// lies within its face's A-box, so lanes whose best is < 0.5 after phase A
// are final.
__device__ __forceinline__ PixelBest resolve_block(const SoftRec* recs, const CullRec* cull,
                                                   const BinView& bv, int bx, int by,
                                                   float radius, const float* prev,
                                                   uint32_t width, ResolveLds& lds) {
    const int lane = threadIdx.x & 63;
    const int px = bx + (lane & 7);
    const int py = by + (lane >> 3);
    PixelBest best;
    best.key = kEmptyKey;
    best.hard = false;
    auto fold_a = [&](const SoftRec& r, uint32_t fj, int) {
        const bool inside = r.bx0 <= bx && r.bx1 >= bx + 7 && r.by0 <= by && r.by1 >= by + 7;
        frag_phase_a(r, fj, px, py, inside, radius, prev, width, best);
    };
    // Phase A folds faces whose hard area is negative (the front faces of a
    // closed mesh under this projection) first and keeps the others in LDS
    // (up to kLaterCap; the rest are folded at once): the key minimum does
    // not depend on the fold order, and a kept face whose depth floor zc
    // lies above every lane's depth after the first pass can win no pixel --
    // its hard fragments are deeper and its rim fragments are >= 0.5 > zc --
    // nor can phase B need it (every lane's depth is then < 0.5).
    const bool defer = !bv.implicit;
    uint32_t n_later = 0;
    for (uint32_t base = 0; base < bv.n; base += 64) {
        const uint32_t e = base + (uint32_t)lane;
        uint32_t f = 0;
        bool keep = false, pos = false;
        float zc = 0.f;
        if (e < bv.n) {
            f = bv.implicit ? e : (base == 0 ? bv.pre : bv.list[e]);
            const CullLoad l = load_cull<false>(recs, cull, f);
            keep = cull_in_a(l, bx, by, true);
            pos = cull_pos(l);
            zc = l.zc;
        }
        bool hold = defer && keep && pos;
        const uint64_t mh0 = __ballot(hold);
        hold = hold && n_later + lanes_below(mh0) < kLaterCap;
        const uint64_t mh = __ballot(hold);
        if (hold) {
            lds.later[n_later + lanes_below(mh)] = f;
            lds.later_zc[n_later + lanes_below(mh)] = zc;
        }
        n_later += (uint32_t)__popcll(mh);
        visit_staged(recs, f, __ballot(keep && !hold), lds, fold_a);
    }
    if (n_later) {
        __syncthreads();
        // the deepest lane depth (an empty lane: all ones, nothing is skipped)
        uint32_t zmax = (uint32_t)(best.key >> 32);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            const uint32_t other = (uint32_t)__shfl_xor((int)zmax, o);
            zmax = other > zmax ? other : zmax;
        }
        for (uint32_t base = 0; base < n_later; base += 64) {
            const uint32_t i = base + (uint32_t)lane;
            uint32_t f = 0;
            bool keep = false;
            if (i < n_later) {
                f = lds.later[i];
                // zc >= 0: bit order is value order
                keep = __float_as_uint(lds.later_zc[i]) <= zmax;
            }
            visit_staged(recs, f, __ballot(keep), lds, fold_a);
        }
    }
    const bool need = (uint32_t)(best.key >> 32) >= 0x3f000000u;  // best depth >= 0.5
    if (!__any(need)) {
        return best;
    }
    phase_b(recs, cull, bv, bx, by, radius, prev, width, need, lds, best);
    return best;
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

// Walks the faces binned to one (view, tile) of the hard rasterizer (scan
// based bins): chunks of up to 256 records are staged through LDS and every
// lane folds each record via `frag(rec, f)`. When the bin's list overflowed
// the capacity the walk covers all faces.
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

// ---------------------------------------------------------------------------
// Fixed-capacity soft bins, appended from the setup kernels. A face goes to
// the tiles of its pixel bbox that its triangle reaches (the separating-axis
// test of the block culls, with the record's margin; every tile of the bbox
// when it has none), walked row by row over the columns the triangle can
// reach (tri_row_span: the thin, tilted soft triangles of edge-on faces have
// bboxes of hundreds of tiles but touch a band of them). A thread walks the
// tiles of its own face when its bbox holds at most kBinBig; the tile rows of
// larger faces are dealt to all threads of the workgroup (a scan of their
// row counts, a binary search per row), so the lanes of a wave share the
// work evenly whatever the faces' sizes (a face spanning many tiles would
// otherwise hold its wave). Pairs
// in the workgroup's LDS window of tiles are counted in LDS (one global
// atomic per touched window tile), then written; the others (outside the
// window, or a workgroup spanning two views) append with direct atomics. All
// threads of the workgroup (blockDim.x a multiple of 64, <= kBinThreads)
// must call it.
// ---------------------------------------------------------------------------
constexpr int kBinWin = 32;  // LDS window of 32 x 32 tiles
constexpr int kBinThreads = 256;
constexpr int kBinBig = 2;
// Dealt rows whose face slot a lookup table holds (beyond it: a binary
// search over the row scan).
constexpr uint32_t kBinRowCap = 2048;
static_assert(kBinThreads <= 256, "face slots fit a byte");

// Triangle of the tile test: screen corners, orientation sign of its area
// and the edge-function margin (< 0: bbox only).
struct BinTri {
    float x[3], y[3];
    float s, m;
};

struct BinLds {
    uint32_t cnt[kBinWin * kBinWin];
    uint32_t base[kBinWin * kBinWin];
    int win[4];                     // tx0, ty0, view0, mixed-view flag
    uint32_t off[kBinThreads + 1];  // exclusive scan of the threads' tile counts
    uint32_t f[kBinThreads], view[kBinThreads];
    int tx0[kBinThreads], ty0[kBinThreads], tx1[kBinThreads];
    BinTri tri[kBinThreads];
    uint8_t row_face[kBinRowCap];  // face slot of dealt row p (p < kBinRowCap)
};

// Whether triangle t can cover a pixel centre of tile (tx, ty): on every
// edge the best corner of the tile's centre rectangle is not below -m.
__device__ __forceinline__ bool tri_reaches_tile(const BinTri& t, int tx, int ty) {
    if (!(t.m >= 0.f)) {
        return true;
    }
    const float x0 = (float)(tx * kTile) + 0.5f, x1 = x0 + (float)(kTile - 1);
    const float y0 = (float)(ty * kTile) + 0.5f, y1 = y0 + (float)(kTile - 1);
    bool hit = true;
#pragma unroll
    for (int k = 0; k < 3; k++) {
        const int k1 = (k + 1) % 3;
        const float ex = t.s * (t.x[k1] - t.x[k]);
        const float ey = t.s * (t.y[k1] - t.y[k]);
        const float gk = smax(ex * (y0 - t.y[k]), ex * (y1 - t.y[k])) +
                         smax(-ey * (x0 - t.x[k]), -ey * (x1 - t.x[k]));
        hit = hit && !(gk < -t.m);
    }
    return hit;
}

// The tiles [*a, *b] of tile row ty (within [tx0, tx1]) that triangle t can
// reach: along a row of tiles each edge's test in tri_reaches_tile is
// monotone in the tile column, so every edge bounds the columns on one side;
// the bounds are widened by one tile (rounding) and the tiles in the range
// still take the exact test. Non-finite bounds leave the side open.
__device__ __forceinline__ void tri_row_span(const BinTri& t, int ty, int tx0, int tx1, int* a,
                                             int* b) {
    *a = tx0;
    *b = tx1;
    if (!(t.m >= 0.f)) {
        return;
    }
    const float y0 = (float)(ty * kTile) + 0.5f, y1 = y0 + (float)(kTile - 1);
#pragma unroll
    for (int k = 0; k < 3; k++) {
        const int k1 = (k + 1) % 3;
        const float ex = t.s * (t.x[k1] - t.x[k]);
        const float ey = t.s * (t.y[k1] - t.y[k]);
        const float A = smax(ex * (y0 - t.y[k]), ex * (y1 - t.y[k]));
        if (ey > 0.f) {
            // the test's best column is the tile's first: x0 <= x_k + (A + m) / ey
            const float c = ((t.x[k] + (A + t.m) / ey) - 0.5f) / (float)kTile;
            if (c >= -1e6f && c <= 1e6f) {
                *b = min(*b, (int)floorf(c) + 1);
            }
        } else if (ey < 0.f) {
            // the tile's last column: x1 >= x_k + (A + m) / ey
            const float c = ((t.x[k] + (A + t.m) / ey) - (float)kTile + 0.5f) / (float)kTile;
            if (c >= -1e6f && c <= 1e6f) {
                *a = max(*a, (int)ceilf(c) - 1);
            }
        } else if (A < -t.m) {
            *a = tx1 + 1;  // the row is outside this edge
        }
    }
}

// Tile-test triangle of a soft record: the soft triangle (every fragment
// needs its coverage) with its coverage margin.
__device__ __forceinline__ BinTri soft_bin_tri(const SoftRec& r) {
    BinTri t;
#pragma unroll
    for (int k = 0; k < 3; k++) {
        t.x[k] = r.sx[k];
        t.y[k] = r.sy[k];
    }
    t.s = r.s_inv_area > 0.f ? 1.f : -1.f;
    t.m = r.s_margin;
    return t;
}

// Heavy bins (at least HeavyList::min_count entries: the silhouette's limb,
// where the soft triangles of edge-on faces pile up) take many times longer
// to resolve than the rest, so the raster dispatches them first. The append
// that takes a bin's count across min_count lists it: in segment
// heavy_seg(bin) (a counter each, so no single counter takes every atomic;
// a multiplicative hash spreads the limb's runs of neighbouring bins), at
// the returned slot, which is also kept per bin. A bin past its segment's
// capacity stays with the others. The consumer clears the segment counters
// with the bin counters.
constexpr uint32_t kHeavySegs = 64;
constexpr uint32_t kHeavySegCap = 96;
constexpr uint32_t kHeavyCap = kHeavySegs * kHeavySegCap;
struct HeavyList {
    uint32_t* count;  // [kHeavySegs]
    uint32_t* list;   // [kHeavySegs][kHeavySegCap] bins
    uint32_t* slot;   // [n_bins] slot of a bin whose count reached min_count
    uint32_t cap;     // slots per segment the consumer takes (<= kHeavySegCap)
    uint32_t min_count;
};

// The entry count that makes a bin heavy, for a problem of n_bins bins. A
// short raster (few bins) ends on the tail of its longest blocks, so more of
// them go first; in a long one the first-dispatched bins lose the tile
// order's cache locality, so only the longest do (measured: 512 x 512 x 4
// views, 4 096 bins: 48 entries; 2048 x 2048 x 4 views, 65 536 bins: 96).
inline uint32_t heavy_min_count(uint32_t n_bins) { return n_bins <= 16384u ? 48u : 96u; }

// Slots per segment for a problem of n_bins bins: at most a quarter of the
// bins go first (the rest of a segment stays with the others).
inline uint32_t heavy_seg_cap(uint32_t n_bins) {
    const uint32_t c = n_bins / (4u * kHeavySegs);
    return c < 1u ? 1u : (c > kHeavySegCap ? kHeavySegCap : c);
}

__device__ __forceinline__ uint32_t heavy_seg(uint32_t bin) {
    return (bin * 2654435761u) >> 26;  // top 6 bits: kHeavySegs = 64
}

__device__ __forceinline__ void heavy_note(const HeavyList* h, uint32_t bin, uint32_t old,
                                           uint32_t add) {
    if (h && old < h->min_count && old + add >= h->min_count) {
        const uint32_t seg = heavy_seg(bin);
        const uint32_t s = atomicAdd(&h->count[seg], 1u);
        h->slot[bin] = s;
        if (s < kHeavySegCap) {
            h->list[seg * kHeavySegCap + s] = bin;
        }
    }
}

// The bin is listed (resolved by the heavy part of the raster's grid).
__device__ __forceinline__ bool heavy_listed(const HeavyList& h, uint32_t count, uint32_t bin) {
    return count >= h.min_count && h.slot[bin] < h.cap;
}

// One (face, tile) pair that the tile test passed, in bin_append's pass (0:
// count window pairs in LDS and append the others, 1: write window pairs
// from their bases).
__device__ __forceinline__ void bin_put(const BinBuffers& b, const RasterGeom& g, BinLds& lds,
                                        int pass, bool mixed, int wx0, int wy0, uint32_t f,
                                        uint32_t view, int tx, int ty, const HeavyList* heavy) {
    const bool local = !mixed && tx - wx0 < kBinWin && ty - wy0 < kBinWin;
    if (pass == 1 && !local) {
        return;
    }
    const uint32_t bin = view * g.n_tiles + ty * g.tiles_x + tx;
    uint32_t slot;
    if (local) {
        const int li = (ty - wy0) * kBinWin + (tx - wx0);
        const uint32_t k = atomicAdd(&lds.cnt[li], 1u);
        if (pass == 0) {
            return;
        }
        slot = lds.base[li] + k;
    } else {
        slot = atomicAdd(&b.counts[bin], 1u);
        heavy_note(heavy, bin, slot, 1u);
    }
    if (slot < b.cap) {
        b.list[(size_t)bin * b.cap + slot] = f;
    }
}

// The same for a pair the tile test has not seen yet.
__device__ __forceinline__ void bin_pair(const BinBuffers& b, const RasterGeom& g, BinLds& lds,
                                         int pass, bool mixed, int wx0, int wy0, uint32_t f,
                                         uint32_t view, const BinTri& tri, int tx, int ty,
                                         const HeavyList* heavy) {
    if ((pass == 1 && (mixed || tx - wx0 >= kBinWin || ty - wy0 >= kBinWin)) ||
        !tri_reaches_tile(tri, tx, ty)) {
        return;
    }
    bin_put(b, g, lds, pass, mixed, wx0, wy0, f, view, tx, ty, heavy);
}

// Face slot q of the workgroup's dealt rows with off[q] <= p < off[q + 1].
__device__ __forceinline__ int dealt_face(const BinLds& lds, uint32_t p, int nthr) {
    if (p < kBinRowCap) {
        return lds.row_face[p];
    }
    int lo = 0, hi = nthr - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (lds.off[mid] <= p) {
            lo = mid;
        } else {
            hi = mid - 1;
        }
    }
    return lo;
}

__device__ __forceinline__ void bin_append(const BinBuffers& b, const RasterGeom& g, bool valid,
                                           uint32_t view, uint32_t f, int bx0, int by0, int bx1,
                                           int by1, const BinTri& tri, BinLds& lds,
                                           const HeavyList* heavy = nullptr) {
    const int tid = (int)threadIdx.x;
    const int nthr = (int)blockDim.x;
    const int tx0 = bx0 / kTile, tx1 = bx1 / kTile, ty0 = by0 / kTile, ty1 = by1 / kTile;
    const uint32_t nt = valid ? (uint32_t)((tx1 - tx0 + 1) * (ty1 - ty0 + 1)) : 0u;
    const bool big = nt > (uint32_t)kBinBig;
    if (tid == 0) {
        lds.win[0] = 0x7fffffff;
        lds.win[1] = 0x7fffffff;
        lds.win[2] = -1;
        lds.win[3] = 0;
    }
    for (int i = tid; i < kBinWin * kBinWin; i += nthr) {
        lds.cnt[i] = 0;
    }
    if (big) {
        lds.f[tid] = f;
        lds.view[tid] = view;
        lds.tx0[tid] = tx0;
        lds.ty0[tid] = ty0;
        lds.tx1[tid] = tx1;
        lds.tri[tid] = tri;
    }
    // inclusive scan of the large faces' tile-row counts: within each wave,
    // then across waves
    uint32_t incl = big ? (uint32_t)(ty1 - ty0 + 1) : 0u;
    const int lane = tid & 63;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = (uint32_t)__shfl_up((int)incl, o);
        incl += lane >= o ? v : 0u;
    }
    lds.off[tid + 1] = incl;
    // the window's corner and the last view: reduced per wave, then one LDS
    // atomic per wave
    int wtx = valid ? tx0 : 0x7fffffff, wty = valid ? ty0 : 0x7fffffff;
    int wview = valid ? (int)view : -1;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        wtx = min(wtx, __shfl_xor(wtx, o));
        wty = min(wty, __shfl_xor(wty, o));
        wview = max(wview, __shfl_xor(wview, o));
    }
    __syncthreads();
    if (lane == 0) {
        atomicMin(&lds.win[0], wtx);
        atomicMin(&lds.win[1], wty);
        atomicMax(&lds.win[2], wview);
    }
    uint32_t wave_base = 0;
    for (int wv = 0; wv < (tid >> 6); wv++) {
        wave_base += lds.off[wv * 64 + 64];
    }
    __syncthreads();
    lds.off[tid + 1] = wave_base + incl;
    if (tid == 0) {
        lds.off[0] = 0;
    }
    if (valid && (int)view != lds.win[2]) {
        lds.win[3] = 1;
    }
    __syncthreads();
    const uint32_t total = lds.off[nthr];
    // the row -> face table of the first kBinRowCap dealt rows
    if (big) {
        const uint32_t r1 = min(lds.off[tid + 1], kBinRowCap);
        for (uint32_t r = lds.off[tid]; r < r1; r++) {
            lds.row_face[r] = (uint8_t)tid;
        }
    }
    __syncthreads();
    const int wx0 = lds.win[0], wy0 = lds.win[1];
    const bool mixed = lds.win[3] != 0;
    // the first kKeepRows dealt rows of each thread: pass 0 keeps the face
    // slot, row, first column and a mask of the columns whose test passed
    // (spans of at most 32 tiles), so pass 1 repeats neither the search nor
    // the tests
    constexpr int kKeepRows = 8;
    int keep_lo[kKeepRows], keep_ty[kKeepRows], keep_ta[kKeepRows];
    uint32_t keep_mask[kKeepRows];
    bool keep_ok[kKeepRows];
#pragma unroll
    for (int it = 0; it < kKeepRows; it++) {
        keep_lo[it] = keep_ty[it] = keep_ta[it] = 0;
        keep_mask[it] = 0u;
        keep_ok[it] = false;
    }
    for (int pass = 0; pass < 2; pass++) {
        if (valid && !big) {
            // up to 2 x 2 tiles the test rarely rejects one: bbox only
            BinTri t = tri;
            t.m = nt <= 4u ? -1.f : t.m;
            for (int ty = ty0; ty <= ty1; ty++) {
                // small bboxes: the per-tile test alone is cheaper
                int ta = tx0, tb = tx1;
                if (nt > 16u) {
                    tri_row_span(t, ty, tx0, tx1, &ta, &tb);
                }
                for (int tx = ta; tx <= tb; tx++) {
                    bin_pair(b, g, lds, pass, mixed, wx0, wy0, f, view, t, tx, ty, heavy);
                }
            }
        }
#pragma unroll
        for (int it = 0; it < kKeepRows; it++) {
            const uint32_t p = (uint32_t)tid + (uint32_t)(it * nthr);
            if (p >= total) {
                break;
            }
            if (pass == 1 && keep_ok[it]) {
                const int lo = keep_lo[it];
                const uint32_t fq = lds.f[lo], vq = lds.view[lo];
                for (uint32_t m = keep_mask[it]; m; m &= m - 1u) {
                    bin_put(b, g, lds, 1, mixed, wx0, wy0, fq, vq,
                            keep_ta[it] + (int)__builtin_ctz(m), keep_ty[it], heavy);
                }
                continue;
            }
            // the face q with off[q] <= p < off[q + 1], and its tile row
            const int lo = dealt_face(lds, p, nthr);
            const int ty = lds.ty0[lo] + (int)(p - lds.off[lo]);
            const BinTri t = lds.tri[lo];
            int ta, tb;
            tri_row_span(t, ty, lds.tx0[lo], lds.tx1[lo], &ta, &tb);
            uint32_t mask = 0u;
            for (int tx = ta; tx <= tb; tx++) {
                if (!tri_reaches_tile(t, tx, ty)) {
                    continue;
                }
                mask |= tx - ta < 32 ? 1u << (tx - ta) : 0u;
                bin_put(b, g, lds, pass, mixed, wx0, wy0, lds.f[lo], lds.view[lo], tx, ty,
                        heavy);
            }
            if (pass == 0) {
                keep_lo[it] = lo;
                keep_ty[it] = ty;
                keep_ta[it] = ta;
                keep_mask[it] = mask;
                keep_ok[it] = tb - ta < 32;
            }
        }
        for (uint32_t p = (uint32_t)(tid + kKeepRows * nthr); p < total; p += (uint32_t)nthr) {
            const int lo = dealt_face(lds, p, nthr);
            const int ty = lds.ty0[lo] + (int)(p - lds.off[lo]);
            const BinTri t = lds.tri[lo];
            int ta, tb;
            tri_row_span(t, ty, lds.tx0[lo], lds.tx1[lo], &ta, &tb);
            for (int tx = ta; tx <= tb; tx++) {
                bin_pair(b, g, lds, pass, mixed, wx0, wy0, lds.f[lo], lds.view[lo], t, tx, ty,
                         heavy);
            }
        }
        if (pass == 0) {
            __syncthreads();
            const uint32_t view0 = (uint32_t)max(lds.win[2], 0);
            for (int i = tid; i < kBinWin * kBinWin; i += nthr) {
                const uint32_t c = lds.cnt[i];
                if (c) {
                    const int tx = wx0 + i % kBinWin, ty = wy0 + i / kBinWin;
                    const uint32_t bin = view0 * g.n_tiles + ty * g.tiles_x + tx;
                    const uint32_t old = atomicAdd(&b.counts[bin], c);
                    heavy_note(heavy, bin, old, c);
                    lds.base[i] = old;
                    lds.cnt[i] = 0;
                }
            }
            __syncthreads();
        }
    }
}

}  // namespace dressi
