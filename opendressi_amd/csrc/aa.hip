// aa.hip -- screen-space antialiasing (the reference's technique "aa",
// Dr.Hair-style AA): the per-op AntiAlias / AntiAliasBwdImg /
// AntiAliasBwdVtx / ColSum entry points and the kernels of the fused AA
// silhouette iteration (hard raster -> AntiAlias -> L2 -> stochastic vertex
// gather -> ColSum -> clip->pos -> Adam).
#include "plan.h"

namespace dressi {

namespace {

__device__ __forceinline__ uint32_t tri_id(const float* tri, size_t o) {
    return (uint32_t)(int)(tri[o] + 0.5f);  // int(tri + 0.5f) (cpu_raster.cpp:374-375)
}

// Reference-layout accessors of the per-op kernels: faces as float ids
// (int64(v + 0.5f), cpu_raster.cpp:395), clip {V,1} VEC4.
struct FloatFaces {
    const float* faces;
    __device__ uint32_t operator()(uint32_t f, int k) const {
        return (uint32_t)(int64_t)(faces[(size_t)f * 3 + k] + 0.5f);
    }
};

// Owner triangles of the fused iteration: vertex ids from the int32 faces,
// screen corners from the view's setup records (the same ProjectClipToScreen
// values). Owners come from the face-id buffer, so every one of them won a
// pixel and has all corners in front of the camera.
struct TriFromRecs {
    const int32_t* faces;
    const AaRec* recs;
    __device__ bool operator()(uint32_t f, uint32_t vi[3], float qx[3], float qy[3]) const {
        const AaRec& r = recs[f];
        for (int k = 0; k < 3; k++) {
            vi[k] = (uint32_t)faces[f * 3 + k];
            qx[k] = r.x[k];
            qy[k] = r.y[k];
        }
        return true;
    }
};

// kAaOffX / kAaOffY as compile-time constants (register-array indices)
constexpr int kAaOffXh[8] = {-1, 0, 1, -1, 1, -1, 0, 1};
constexpr int kAaOffYh[8] = {-1, -1, -1, 0, 0, 1, 1, 1};

}  // namespace

// ---------------------------------------------------------------------------
// Per-op kernels (reference layouts: float face-id image, float faces)
// ---------------------------------------------------------------------------

// Batched per-op kernels: blockIdx.y is the item; images are [item][H][W]
// (x n_comp), clips [item][V] when `clip_per_item`, else shared.
struct AaItem {
    uint32_t item;
    size_t npx;
    __device__ AaItem(uint32_t w, uint32_t h) : item(blockIdx.y), npx((size_t)w * h) {}
    template <typename T>
    __device__ T* img(T* p, uint32_t n_comp) const { return p + item * npx * n_comp; }
    __device__ const float4* clip(const float4* p, uint32_t n_verts, int per_item) const {
        return per_item ? p + (size_t)item * n_verts : p;
    }
};

// AntiAlias forward (f_ops.cpp:2544-2576), one thread per pixel.
__global__ __launch_bounds__(256) void k_antialias_op(const float* img, uint32_t n_comp,
                                                      const float* tri, const float4* clip,
                                                      uint32_t n_verts, int clip_per_item,
                                                      const float* faces, uint32_t n_faces,
                                                      uint32_t w, uint32_t h, float* out) {
    const uint32_t p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= w * h) {
        return;
    }
    const AaItem it(w, h);
    img = it.img(img, n_comp);
    tri = it.img(tri, 1);
    out = it.img(out, n_comp);
    clip = it.clip(clip, n_verts, clip_per_item);
    const int x = (int)(p % w), y = (int)(p / w);
    const float W = (float)w, H = (float)h;
    const size_t so = (size_t)p * n_comp;
    float dst[4];
    for (uint32_t c = 0; c < n_comp; c++) {
        dst[c] = img[so + c];
    }
    const uint32_t its = tri_id(tri, p);
    for (int k = 0; k < 8; k++) {
        const int nx = x + kAaOffX[k], ny = y + kAaOffY[k];
        AaPair pr;
        const bool in = !(nx < 0 || ny < 0 || nx >= (int)w || ny >= (int)h);
        if (!in || !eval_aa_pair(its, tri_id(tri, (size_t)ny * w + nx), x, y, nx, ny, n_faces,
                                 TriFromClip{faces, clip, n_verts, W, H}, &pr)) {
            for (uint32_t c = 0; c < n_comp; c++) {
                dst[c] += img[so + c];
            }
            continue;
        }
        const size_t no = ((size_t)ny * w + nx) * n_comp;
        for (uint32_t c = 0; c < n_comp; c++) {
            dst[c] += pr.r * img[so + c] + (1.f - pr.r) * img[no + c];
        }
    }
    for (uint32_t c = 0; c < n_comp; c++) {
        out[so + c] = dst[c] / 9.f;
    }
}

// AntiAliasBwdImg (f_ops.cpp:2231-2275), one thread per pixel.
__global__ __launch_bounds__(256) void k_antialias_bwd_img_op(const float* gy, uint32_t n_comp,
                                                              const float* tri, const float4* clip,
                                                              uint32_t n_verts, int clip_per_item,
                                                              const float* faces,
                                                              uint32_t n_faces, uint32_t w,
                                                              uint32_t h, float* out) {
    const uint32_t p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= w * h) {
        return;
    }
    const AaItem it(w, h);
    gy = it.img(gy, n_comp);
    tri = it.img(tri, 1);
    out = it.img(out, n_comp);
    clip = it.clip(clip, n_verts, clip_per_item);
    const int x = (int)(p % w), y = (int)(p / w);
    const float W = (float)w, H = (float)h;
    const size_t so = (size_t)p * n_comp;
    float dst[4] = {0.f, 0.f, 0.f, 0.f};
    float alpha_sum = 0.f;
    const uint32_t its = tri_id(tri, p);
    for (int k = 0; k < 8; k++) {
        const int nx = x + kAaOffX[k], ny = y + kAaOffY[k];
        if (nx < 0 || ny < 0 || nx >= (int)w || ny >= (int)h) {
            alpha_sum += 1.f;
            continue;
        }
        const uint32_t itn = tri_id(tri, (size_t)ny * w + nx);
        AaPair pr;
        alpha_sum += eval_aa_pair(its, itn, x, y, nx, ny, n_faces,
                                  TriFromClip{faces, clip, n_verts, W, H}, &pr)
                             ? pr.r
                             : 1.f;
        AaPair pr2;
        if (eval_aa_pair(itn, its, nx, ny, x, y, n_faces, TriFromClip{faces, clip, n_verts, W, H},
                         &pr2)) {
            const size_t no = ((size_t)ny * w + nx) * n_comp;
            for (uint32_t c = 0; c < n_comp; c++) {
                dst[c] += (1.f - pr2.r) * gy[no + c];
            }
        }
    }
    for (uint32_t c = 0; c < n_comp; c++) {
        dst[c] += gy[so + c] * (1.f + alpha_sum);
        out[so + c] = dst[c] / 9.f;
    }
}

// One active pair's contribution to vertex v's row (f_ops.cpp:2345-2386,
// only_v): gr = dot(gy(s), c(s) - c(n)) / 9, then each endpoint equal to v.
__device__ __forceinline__ void aa_accumulate_v(const float* gy, const float* img,
                                                uint32_t n_comp, const float4* clip, float W,
                                                float H, uint32_t w, uint32_t v, int x, int y,
                                                int nx, int ny, const AaPair& pr, float4* dst) {
    const size_t so = ((size_t)y * w + x) * n_comp;
    const size_t no = ((size_t)ny * w + nx) * n_comp;
    float gr = 0.f;
    for (uint32_t c = 0; c < n_comp; c++) {
        gr += gy[so + c] * (img[so + c] - img[no + c]);
    }
    gr /= 9.f;
    if (gr == 0.f) {
        return;
    }
    float dqa[2], dqb[2];
    aa_pair_dq(pr, x, y, dqa, dqb);
    if (pr.ia == v) {
        aa_add_endpoint(gr, dqa, clip[pr.ia], W, H, dst);
    }
    if (pr.ib == v) {
        aa_add_endpoint(gr, dqb, clip[pr.ib], W, H, dst);
    }
}

// AntiAliasBwdVtx, n_samples > 0 (f_ops.cpp:2410-2472): one 8-lane group per
// (vertex, slot) row when `wide` (out {V, deg} VEC4, row d * V + v), else
// per vertex accumulating its slots in order (out {V,1}). The group walks
// the row's faces and samples together; at each sample lane k evaluates the
// pair with neighbour k and the term it gives v (at most one: an edge's two
// endpoints differ), then the group adds the eight terms in neighbour order,
// so the row sums its terms in the reference's (slot, sample, neighbour)
// order.
__global__ __launch_bounds__(256) void k_antialias_bwd_vtx_op(
        const float* gy, const float* img, uint32_t n_comp, const float* tri, const float4* clip,
        uint32_t n_verts, int clip_per_item, const float* faces, uint32_t n_faces,
        const float* vtx_faces, uint32_t max_deg, const float* seed, uint32_t n_samples, int wide,
        uint32_t w, uint32_t h, float4* out) {
    const uint32_t i = (blockIdx.x * blockDim.x + threadIdx.x) >> 3;
    const int k = (int)(threadIdx.x & 7u);
    const int gbase = (int)(threadIdx.x & 56u);  // the group's first lane in the wave
    const uint32_t rows = wide ? max_deg : 1u;
    if (i >= n_verts * rows) {
        return;  // the whole group: its lanes share i
    }
    const AaItem it(w, h);
    gy = it.img(gy, n_comp);
    img = it.img(img, n_comp);
    tri = it.img(tri, 1);
    clip = it.clip(clip, n_verts, clip_per_item);
    seed += it.item;
    out += (size_t)it.item * rows * n_verts;
    const uint32_t v = wide ? i % n_verts : i;
    const uint32_t d0 = wide ? i / n_verts : 0u;
    const uint32_t d1 = wide ? d0 + 1 : max_deg;
    const float W = (float)w, H = (float)h;
    const uint32_t seed_u = (uint32_t)(int64_t)(*seed + 0.5f);
    float4 dst = make_float4(0.f, 0.f, 0.f, 0.f);
    for (uint32_t d = d0; d < d1; d++) {
        const float fv = vtx_faces[(size_t)d * n_verts + v];
        if (fv < -0.5f) {
            continue;
        }
        const uint32_t f = (uint32_t)(int64_t)(fv + 0.5f);
        if (f >= n_faces) {
            continue;
        }
        float4 c[3];
        bool ok = true;
        for (int q = 0; q < 3; q++) {
            const uint32_t vi = FloatFaces{faces}(f, q);
            if (vi >= n_verts) {
                ok = false;
                break;
            }
            c[q] = clip[vi];
        }
        float s3x[3], s3y[3];
        if (!ok || !aa_face_screen(c, W, H, s3x, s3y)) {
            continue;
        }
        for (uint32_t smp = 0; smp < n_samples; smp++) {
            int x, y;
            if (!aa_sample_px(s3x, s3y, f, smp, seed_u, &x, &y) || x < 0 || y < 0 ||
                x >= (int)w || y >= (int)h) {
                continue;
            }
            // lane k: neighbour k's terms for v, endpoint a then endpoint b
            // (both only for an edge whose two endpoints are v: a face that
            // repeats a vertex)
            float ta[3] = {0.f, 0.f, 0.f}, tb[3] = {0.f, 0.f, 0.f};
            int has = 0;
            const int nx = x + kAaOffX[k], ny = y + kAaOffY[k];
            if (!(nx < 0 || ny < 0 || nx >= (int)w || ny >= (int)h)) {
                const uint32_t its = tri_id(tri, (size_t)y * w + x);
                AaPair pr;
                if (eval_aa_pair(its, tri_id(tri, (size_t)ny * w + nx), x, y, nx, ny, n_faces,
                                 TriFromClip{faces, clip, n_verts, W, H}, &pr) &&
                    pr.r < 1.f && (pr.ia == v || pr.ib == v)) {
                    const size_t so = ((size_t)y * w + x) * n_comp;
                    const size_t no = ((size_t)ny * w + nx) * n_comp;
                    float gr = 0.f;
                    for (uint32_t cc = 0; cc < n_comp; cc++) {
                        gr += gy[so + cc] * (img[so + cc] - img[no + cc]);
                    }
                    gr /= 9.f;
                    if (gr != 0.f) {
                        float dqa[2], dqb[2];
                        aa_pair_dq(pr, x, y, dqa, dqb);
                        const auto term = [&](const float dq[2], float4 ce, float* t) {
                            const float gqx = gr * dq[0];
                            const float gqy = gr * dq[1];
                            t[0] = gqx * 0.5f * W / ce.w;
                            t[1] = gqy * 0.5f * H / ce.w;
                            t[2] = -(gqx * 0.5f * W * ce.x + gqy * 0.5f * H * ce.y) /
                                   (ce.w * ce.w);
                        };
                        if (pr.ia == v) {
                            term(dqa, clip[pr.ia], ta);
                            has |= 1;
                        }
                        if (pr.ib == v) {
                            term(dqb, clip[pr.ib], tb);
                            has |= 2;
                        }
                    }
                }
            }
            for (int kk = 0; kk < 8; kk++) {
                const int src = gbase + kk;
                const int fl = __shfl(has, src, 64);
                if (fl & 1) {
                    dst.x += __shfl(ta[0], src, 64);
                    dst.y += __shfl(ta[1], src, 64);
                    dst.w += __shfl(ta[2], src, 64);
                }
                if (fl & 2) {
                    dst.x += __shfl(tb[0], src, 64);
                    dst.y += __shfl(tb[1], src, 64);
                    dst.w += __shfl(tb[2], src, 64);
                }
            }
        }
    }
    if (k == 0) {
        out[i] = dst;
    }
}

// AntiAliasBwdVtx, n_samples = 0 (f_ops.cpp:2389-2407): the exact scatter
// over every active pair, restated as a gather per vertex that visits the
// pixels of its incident faces' bboxes (+-1 px) in the scatter's raster order,
// so every vertex's sum has the reference's order. An active pair's edge
// belongs to a face covering s or its neighbour, so no pair of v's lies
// outside those pixels.
__global__ __launch_bounds__(128) void k_antialias_bwd_vtx_exact_op(
        const float* gy, const float* img, uint32_t n_comp, const float* tri, const float4* clip,
        uint32_t n_verts, int clip_per_item, const float* faces, uint32_t n_faces,
        const float* vtx_faces, uint32_t max_deg, uint32_t w, uint32_t h, float4* out) {
    const uint32_t v = blockIdx.x * blockDim.x + threadIdx.x;
    if (v >= n_verts) {
        return;
    }
    const AaItem it(w, h);
    gy = it.img(gy, n_comp);
    img = it.img(img, n_comp);
    tri = it.img(tri, 1);
    clip = it.clip(clip, n_verts, clip_per_item);
    out += (size_t)it.item * n_verts;
    const float W = (float)w, H = (float)h;
    int bx0 = (int)w, by0 = (int)h, bx1 = -1, by1 = -1;
    for (uint32_t d = 0; d < max_deg; d++) {
        const float fv = vtx_faces[(size_t)d * n_verts + v];
        if (fv < -0.5f) {
            continue;
        }
        const uint32_t f = (uint32_t)(int64_t)(fv + 0.5f);
        if (f >= n_faces) {
            continue;
        }
        float qx[3], qy[3];
        bool ok = true;
        for (int k = 0; k < 3 && ok; k++) {
            const uint32_t vi = FloatFaces{faces}(f, k);
            ok = vi < n_verts && clip_w_valid(clip[vi].w);
            if (ok) {
                const float4 c = clip[vi];
                const ScreenVert s = project_to_screen(c.x, c.y, c.z, c.w, W, H);
                qx[k] = s.x;
                qy[k] = s.y;
            }
        }
        if (!ok) {
            continue;  // never an owner (EvalAaPair skips it)
        }
        int fx0, fy0, fx1, fy1;
        pixel_bbox(qx[0], qx[1], qx[2], qy[0], qy[1], qy[2], (int)w, (int)h, &fx0, &fy0, &fx1,
                   &fy1);
        bx0 = min(bx0, fx0 - 1);
        by0 = min(by0, fy0 - 1);
        bx1 = max(bx1, fx1 + 1);
        by1 = max(by1, fy1 + 1);
    }
    bx0 = max(bx0, 0);
    by0 = max(by0, 0);
    bx1 = min(bx1, (int)w - 1);
    by1 = min(by1, (int)h - 1);
    float4 dst = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int y = by0; y <= by1; y++) {
        for (int x = bx0; x <= bx1; x++) {
            const uint32_t its = tri_id(tri, (size_t)y * w + x);
            for (int k = 0; k < 8; k++) {
                const int nx = x + kAaOffX[k], ny = y + kAaOffY[k];
                if (nx < 0 || ny < 0 || nx >= (int)w || ny >= (int)h) {
                    continue;
                }
                AaPair pr;
                if (!eval_aa_pair(its, tri_id(tri, (size_t)ny * w + nx), x, y, nx, ny, n_faces,
                                  TriFromClip{faces, clip, n_verts, W, H}, &pr) ||
                    pr.r >= 1.f || (pr.ia != v && pr.ib != v)) {
                    continue;
                }
                aa_accumulate_v(gy, img, n_comp, clip, W, H, w, v, x, y, nx, ny, pr, &dst);
            }
        }
    }
    out[v] = dst;
}

// ColSum (f_ops.cpp:1227-1244): rows summed in order per column and component.
// blockIdx.y: the item of a batch ([item][H][W] -> [item][W]).
__global__ __launch_bounds__(256) void k_col_sum_op(const float* x, uint32_t n_comp, uint32_t w,
                                                    uint32_t h, float* out) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= w * n_comp) {
        return;
    }
    x += (size_t)blockIdx.y * h * w * n_comp;
    out += (size_t)blockIdx.y * w * n_comp;
    float acc = 0.f;
    for (uint32_t r = 0; r < h; r++) {
        acc += x[(size_t)r * w * n_comp + i];
    }
    out[i] = acc;
}

// ---------------------------------------------------------------------------
// Fused AA iteration
// ---------------------------------------------------------------------------

// Per-view clip positions: TransformToClipVar of every vertex.
__global__ __launch_bounds__(256) void k_aa_clip(HsrDev d) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i == 0 && d.aa_count) {
        *d.aa_count = 0u;  // the face scan of this iteration appends from 0
    }
    if (i >= d.g.n_views * d.n_verts) {
        return;
    }
    const uint32_t view = i / d.n_verts;
    const uint32_t v = i - view * d.n_verts;
    d.clip[i] = mvp_transform(d.mvps + view * 16, d.pos[v * 3 + 0], d.pos[v * 3 + 1],
                              d.pos[v * 3 + 2]);
}

// Hard raster setup per (view, face) (RasterizeCore, cpu_raster.cpp:42-94)
// with the coverage margin of the block cull, appended to the tile bins.
__global__ __launch_bounds__(256) void k_aa_setup(HsrDev d) {
    __shared__ BinLds blds;
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    const bool live = i < d.g.n_views * d.g.n_faces;
    const uint32_t view = live ? i / d.g.n_faces : 0;
    const uint32_t f = live ? i - view * d.g.n_faces : 0;
    AaRec r;
    r.bx0 = 1;
    r.bx1 = 0;
    r.by0 = 1;
    r.by1 = 0;
    r.margin = -1.f;
    r.zcull = 0.f;
    if (live) {
        const float W = (float)d.g.width, H = (float)d.g.height;
        bool ok = true;
        float iw[3];
#pragma unroll
        for (int k = 0; k < 3; k++) {
            const float4 c = d.clip[(size_t)view * d.n_verts + d.faces[f * 3 + k]];
            iw[k] = 1.f / c.w;
            ok = ok && !(fabsf(c.w) <= kWEps || c.w < 0.f);
            const ScreenVert s = project_to_screen(c.x, c.y, c.z, c.w, W, H);
            r.x[k] = s.x;
            r.y[k] = s.y;
            r.z[k] = s.z;
        }
        if (ok) {
            const float area = tri_area(r.x[0], r.y[0], r.x[1], r.y[1], r.x[2], r.y[2]);
            if (!(fabsf(area) < kDistEps)) {
                r.inv_area = 1.f / area;
                // coverage margin: the soft raster's bound for the same
                // barycentric formula (raster_core.h, soft_setup)
                float q = 0.f;
                for (int k = 0; k < 3; k++) {
                    const int k1 = (k + 1) % 3;
                    q += (fabsf(r.x[k]) + fabsf(r.x[k1]) + W) *
                         (fabsf(r.y[k]) + fabsf(r.y[k1]) + H);
                }
                const float pa = fabsf(r.x[1] - r.x[0]) * fabsf(r.y[2] - r.y[0]) +
                                 fabsf(r.y[1] - r.y[0]) * fabsf(r.x[2] - r.x[0]);
                const float m = 0x1p-20f * (q + pa + fabsf(area));
                r.margin = (fabsf(area) > 0x1p-20f * pa && m < INFINITY) ? m : -1.f;
                pixel_bbox(r.x[0], r.x[1], r.x[2], r.y[0], r.y[1], r.y[2], (int)d.g.width,
                           (int)d.g.height, &r.bx0, &r.by0, &r.bx1, &r.by1);
                // At a covered pixel l0, l1, l2 >= 0 and l2 = (1 - l0) - l1
                // make l0 + l1 + l2 >= 1 - 2.01u (u = 2^-24), so with all z
                // positive the interpolated z (three roundings) is at least
                // zmin (1 - 5.1u), and fl(zmin (1 - 2^-20)) < zmin (1 - 15u)
                // lies strictly below it.
                const float zmin = smin(smin(r.z[0], r.z[1]), r.z[2]);
                r.zcull = zmin > 0.f ? zmin * (1.f - 0x1p-20f) : 0.f;
            }
        }
        d.arecs[i] = r;
        if (d.tface) {
            const float2 a0 = d.tf_uv[d.faces[f * 3 + 0]];
            const float2 a1 = d.tf_uv[d.faces[f * 3 + 1]];
            const float2 a2 = d.tf_uv[d.faces[f * 3 + 2]];
            float4* tf = d.tface + (size_t)i * 3;
            tf[0] = make_float4(iw[0], iw[1], iw[2], 0.f);
            tf[1] = make_float4(a0.x, a0.y, a1.x, a1.y);
            tf[2] = make_float4(a2.x, a2.y, 0.f, 0.f);
        }
    }
    const bool valid = live && r.bx0 <= r.bx1 && r.by0 <= r.by1;
    BinTri t;
#pragma unroll
    for (int k = 0; k < 3; k++) {
        t.x[k] = r.x[k];
        t.y[k] = r.y[k];
    }
    t.s = r.inv_area > 0.f ? 1.f : -1.f;
    t.m = r.margin;
    bin_append(d.bins, d.g, valid, view, f, r.bx0, r.by0, r.bx1, r.by1, t, blds);
}

// Separating-axis test of a hard triangle's coverage region (its
// barycentrics >= 0 up to the record's margin) against the 8x8 block.
__device__ __forceinline__ bool aa_tri_reaches_block(const AaRec* rec, int bx, int by,
                                                     bool* neg) {
    const float4 a = *(const float4*)&rec->x[0];  // x0 x1 x2 y0
    const float4 b = *(const float4*)&rec->y[1];  // y1 y2 inv_area margin
    *neg = b.z < 0.f;
    const float m = b.w;
    if (!(m >= 0.f)) {
        return true;
    }
    const float x[3] = {a.x, a.y, a.z};
    const float y[3] = {a.w, b.x, b.y};
    const float s = b.z > 0.f ? 1.f : -1.f;
    const float x0 = (float)bx + 0.5f, x1 = (float)bx + 7.5f;
    const float y0 = (float)by + 0.5f, y1 = (float)by + 7.5f;
    bool hit = true;
#pragma unroll
    for (int k = 0; k < 3; k++) {
        const int k1 = (k + 1) % 3;
        const float ex = s * (x[k1] - x[k]);
        const float ey = s * (y[k1] - y[k]);
        const float g = smax(ex * (y0 - y[k]), ex * (y1 - y[k])) +
                        smax(-ey * (x0 - x[k]), -ey * (x1 - x[k]));
        hit = hit && !(g < -m);
    }
    return hit;
}

typedef const __attribute__((address_space(4))) uint32_t* AaUniformWordPtr;

__device__ __forceinline__ AaRec load_aa_rec_uniform(const AaRec* recs, uint32_t f) {
    const AaUniformWordPtr src = (AaUniformWordPtr)(recs + f);
    union {
        AaRec r;
        uint32_t w[16];
    } u;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        u.w[i] = src[i];
    }
    return u.r;
}

// Folds face fj (its record r) into the lane's depth key: coverage by the
// reference's inclusive barycentrics, NDC z in [0, 1], smaller key wins.
__device__ __forceinline__ void aa_fold_face(const AaRec& r, uint32_t fj, int px, int py,
                                             uint64_t* best) {
    if (px < r.bx0 || px > r.bx1 || py < r.by0 || py > r.by1) {
        return;
    }
    const float p0 = (float)px + 0.5f, p1 = (float)py + 0.5f;
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
    const uint64_t key = depth_key(z, fj);
    *best = key < *best ? key : *best;
}

// Visibility of the hard raster: one single-wave workgroup per (view, 8x8
// block) folds (z | ~face) keys of the faces binned to its tile (coverage by
// the reference's inclusive barycentrics, NDC z in [0,1], LessOrEqual: the
// later face wins ties) and writes face + 1 (0 = background). The key
// minimum does not depend on the order the faces are folded in, so faces
// with negative screen area (the front faces of a closed mesh in this
// projection) go first and the others are kept in LDS; those whose zcull
// lies above every lane's depth after the first pass cannot win a pixel and
// are skipped. Tiles are dealt to the XCDs round robin, the four blocks of a
// tile on one XCD.
__global__ __launch_bounds__(64) void k_aa_raster(HsrDev d) {
    __shared__ uint32_t later[kSoftBinCap];
    const uint32_t per = (d.g.n_tiles + 7u) / 8u;
    const uint32_t k = blockIdx.x >> 3;
    const uint32_t q = k & 3u;
    const uint32_t lt = geom_div(k >> 2, d.g.n_views, d.g.views_m);
    const uint32_t view = (k >> 2) - lt * d.g.n_views;
    const uint32_t tile = lt * 8u + (blockIdx.x & 7u);
    const uint32_t trow = geom_div(tile, d.g.tiles_x, d.g.tiles_x_m);
    const int bx = (int)((tile - trow * d.g.tiles_x) * kTile + (q & 1u) * 8u);
    const int by = (int)(trow * kTile + (q >> 1) * 8u);
    if (lt >= per || tile >= d.g.n_tiles || bx >= (int)d.g.width || by >= (int)d.g.height) {
        return;
    }
    const int lane = threadIdx.x & 63;
    const int px = bx + (lane & 7);
    const int py = by + (lane >> 3);
    const AaRec* recs = d.arecs + (size_t)view * d.g.n_faces;
    const BinView bv = bin_view(d.bins, view * d.g.n_tiles + tile, d.g.n_faces);
    // an overflowed bin (every face) is walked in one pass
    const bool defer = !bv.implicit && bv.n <= kSoftBinCap;
    uint32_t n_later = 0;
    uint64_t best = kEmptyKey;
    for (uint32_t base = 0; base < bv.n; base += 64) {
        const uint32_t e = base + (uint32_t)lane;
        uint32_t f = 0;
        bool keep = false, neg = false;
        if (e < bv.n) {
            f = bv.implicit ? e : bv.list[e];
            const int4 bb = *(const int4*)&recs[f].bx0;
            keep = bb.x <= bx + 7 && bb.z >= bx && bb.y <= by + 7 && bb.w >= by &&
                   aa_tri_reaches_block(recs + f, bx, by, &neg);
        }
        const bool hold = defer && keep && !neg;
        const uint64_t mh = __ballot(hold);
        if (hold) {
            const uint32_t below = __builtin_amdgcn_mbcnt_hi(
                    (uint32_t)(mh >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mh, 0u));
            later[n_later + below] = f;
        }
        n_later += (uint32_t)__popcll(mh);
        uint64_t m = __ballot(keep && !hold);
        while (m) {
            const int j = __builtin_ctzll(m);
            m &= m - 1;
            const uint32_t fj = (uint32_t)__builtin_amdgcn_readlane((int)f, j);
            aa_fold_face(load_aa_rec_uniform(recs, fj), fj, px, py, &best);
        }
    }
    if (n_later) {
        __syncthreads();
        // the deepest lane depth (an empty lane: all ones, nothing is skipped)
        uint32_t zmax = (uint32_t)(best >> 32);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            const uint32_t other = (uint32_t)__shfl_xor((int)zmax, o);
            zmax = other > zmax ? other : zmax;
        }
        zmax = (uint32_t)__builtin_amdgcn_readfirstlane((int)zmax);
        for (uint32_t i = 0; i < n_later; i++) {
            const uint32_t fj = (uint32_t)__builtin_amdgcn_readfirstlane((int)later[i]);
            const AaRec r = load_aa_rec_uniform(recs, fj);
            if (__float_as_uint(r.zcull) > zmax) {
                continue;  // zcull >= 0: bit order is value order
            }
            aa_fold_face(r, fj, px, py, &best);
        }
    }
    if (px < (int)d.g.width && py < (int)d.g.height) {
        d.ids[(size_t)view * d.g.width * d.g.height + (size_t)py * d.g.width + px] =
                best == kEmptyKey ? 0u : key_face(best) + 1;
    }
}

// Orders the LDS accesses of one wave around an exchange between its lanes
// (a wave executes its LDS instructions in order).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Mask bits (1 = covered) of ids columns x0 .. x0+3 of one row.
__device__ __forceinline__ uint32_t fg_bits4(uint32_t a, uint32_t b, uint32_t c, uint32_t e) {
    return (a != 0u ? 1u : 0u) | (b != 0u ? 2u : 0u) | (c != 0u ? 4u : 0u) | (e != 0u ? 8u : 0u);
}

// AntiAlias of the mask (Rasterize(clip, 1): 1 exactly where covered) and the
// L2 loss (f_ops.cpp:2544-2576 with one channel). A lane covers 4
// consecutive pixels of a row in one view, a wave 256 pixels, the NV waves of
// a workgroup the NV views of the same pixels, their SumPixelWise reduced
// through LDS. With c_s = c_n in {0, 1} an active pair adds r c + (1 - r) c,
// which rounds to exactly c (1 - r is within half an ulp of its exact value
// and r + fl(1 - r) rounds back to 1), so a pixel whose in-screen neighbours
// all share its mask value sums 9 c exactly (pred = c); those are found from
// 3x3 windows of mask bits (an off-screen neighbour counts as agreeing; it is
// filled with a copy of an in-screen value of the same window). The other
// pixels (the silhouette) are queued in LDS and evaluated 8 at a time, one
// 8-lane group each, lane k taking neighbour k, the group then summing the
// nine terms in the reference's order. pred is kept for the face backward.
// VEC: the row width is a multiple of 4 (16-byte loads and stores).
template <int NV, bool VEC>
__global__ __launch_bounds__(64 * NV) void k_aa_fwd(HsrDev d) {
    __shared__ float4 lv[NV][64];
    __shared__ uint32_t queue[NV][256];
    __shared__ float epred[NV][256];
    const uint32_t view = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int w = (int)d.g.width, h = (int)d.g.height;
    const int xw = (int)blockIdx.x * 256;
    const int x0 = xw + lane * 4;
    const int y = (int)blockIdx.y;
    const size_t npx = (size_t)w * h;
    const size_t o = (size_t)y * w + x0;
    const uint32_t* ids = d.ids + view * npx;
    const bool any = x0 < w;
    // rows y-1, y, y+1: 6-bit masks, bit i = column x0 - 1 + i
    uint32_t row[3];
    uint32_t fg4 = 0;
#pragma unroll
    for (int ry = 0; ry < 3; ry++) {
        const int yy = y + ry - 1;
        const bool row_ok = any && yy >= 0 && yy < h;
        const uint32_t* rp = ids + (size_t)(row_ok ? yy : 0) * w;
        uint32_t m;
        if (VEC) {
            const uint4 q = row_ok ? *reinterpret_cast<const uint4*>(rp + x0) : uint4{0, 0, 0, 0};
            m = fg_bits4(q.x, q.y, q.z, q.w);
        } else {
            uint32_t v[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                v[c] = row_ok && x0 + c < w ? rp[x0 + c] : 0u;
            }
            m = fg_bits4(v[0], v[1], v[2], v[3]);
        }
        // the wave's outer lanes read the columns beyond it
        uint32_t lcol = 0, rcol = 0;
        if (lane == 0 && row_ok && x0 > 0) {
            lcol = rp[x0 - 1] != 0u ? 1u : 0u;
        }
        if (lane == 63 && row_ok && x0 + 4 < w) {
            rcol = rp[x0 + 4] != 0u ? 1u : 0u;
        }
        row[ry] = m;
        fg4 |= (lcol | rcol << 1) << (2 * ry);  // lane 0 / 63 only
    }
    float tg[4];
    const float* tgt = d.targets + view * npx;
    if (VEC) {
        const float4 q = any ? *reinterpret_cast<const float4*>(tgt + o) : float4{0, 0, 0, 0};
        tg[0] = q.x;
        tg[1] = q.y;
        tg[2] = q.z;
        tg[3] = q.w;
    } else {
#pragma unroll
        for (int c = 0; c < 4; c++) {
            tg[c] = any && x0 + c < w ? tgt[o + c] : 0.f;
        }
    }
    // neighbouring lanes' edge columns (12 bits: 4 per row)
    const uint32_t own = row[0] | row[1] << 4 | row[2] << 8;
    const uint32_t from_left = (uint32_t)__shfl_up((int)own, 1);
    const uint32_t from_right = (uint32_t)__shfl_down((int)own, 1);
    // columns in screen: x0 - 1 + i < w for i < ncol (>= 2 where any)
    const int ncol = w - x0 + 1 < 6 ? w - x0 + 1 : 6;
    uint32_t edge = 0;
    float pred[4];
    if (any) {
#pragma unroll
        for (int ry = 0; ry < 3; ry++) {
            const uint32_t l = lane == 0 ? (fg4 >> (2 * ry)) & 1u : (from_left >> (4 * ry + 3)) & 1u;
            const uint32_t r = lane == 63 ? (fg4 >> (2 * ry + 1)) & 1u : (from_right >> (4 * ry)) & 1u;
            uint32_t m = l | row[ry] << 1 | r << 5;
            if (x0 == 0) {
                m = (m & ~1u) | ((m >> 1) & 1u);
            }
            if (ncol < 6) {
                const uint32_t keep = (1u << ncol) - 1u;
                m = (m & keep) | (((m >> (ncol - 1)) & 1u) ? (0x3fu & ~keep) : 0u);
            }
            row[ry] = m;
        }
        if (y == 0) {
            row[0] = row[1];
        }
        if (y == h - 1) {
            row[2] = row[1];
        }
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t win = ((row[0] >> c) & 7u) | ((row[1] >> c) & 7u) << 3 |
                                 ((row[2] >> c) & 7u) << 6;
            edge |= (win != 0u && win != 0x1ffu && x0 + c < w) ? 1u << c : 0u;
            // nine equal terms: 9 c / 9 = c
            pred[c] = (row[1] >> (c + 1)) & 1u ? 1.f : 0.f;
        }
    }
    if (__ballot(edge != 0u)) {
        // queue the silhouette pixels of the wave as lane * 4 + c
        uint32_t* qv = queue[view];
        uint32_t n_q = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const bool e = (edge >> c) & 1u;
            const uint64_t m = __ballot(e);
            if (e) {
                const uint32_t below = __builtin_amdgcn_mbcnt_hi(
                        (uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
                qv[n_q + below] = (uint32_t)lane * 4u + (uint32_t)c;
            }
            n_q += (uint32_t)__popcll(m);
        }
        wave_lds_sync();
        const TriFromRecs tris{d.faces, d.arecs + (size_t)view * d.g.n_faces};
        const int k = lane & 7;
        for (uint32_t q0 = 0; q0 < n_q; q0 += 8) {
            const uint32_t qi = q0 + (uint32_t)(lane >> 3);
            const bool ok = qi < n_q;
            uint32_t slot = 0;
            float cs = 0.f, term = 0.f;
            if (ok) {
                slot = qv[qi];
                const int x = xw + (int)slot;
                const uint32_t its = ids[(size_t)y * w + x];
                cs = its ? 1.f : 0.f;
                term = cs;
                const int nx = x + kAaOffXh[k], ny = y + kAaOffYh[k];
                if (!(nx < 0 || ny < 0 || nx >= w || ny >= h)) {
                    const uint32_t itn = ids[(size_t)ny * w + nx];
                    AaPair pr;
                    if ((its == 0u) != (itn == 0u) &&
                        eval_aa_pair(its, itn, x, y, nx, ny, d.g.n_faces, tris, &pr)) {
                        const float cn = itn ? 1.f : 0.f;
                        term = pr.r * cs + (1.f - pr.r) * cn;
                    }
                }
            }
            // c_s, then the eight neighbours' terms in order
            float dst = cs;
#pragma unroll
            for (int kk = 0; kk < 8; kk++) {
                dst += __shfl(term, (lane & 56) + kk);
            }
            if (ok && k == 0) {
                epred[view][slot] = dst / 9.f;
            }
        }
        wave_lds_sync();
#pragma unroll
        for (int c = 0; c < 4; c++) {
            if ((edge >> c) & 1u) {
                pred[c] = epred[view][lane * 4 + c];
            }
        }
    }
    float l[4] = {0.f, 0.f, 0.f, 0.f};
    bool gnz = false;  // a pixel of the lane has the face scan's gy != 0
    if (any) {
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float diff = tg[c] - pred[c];
            l[c] = diff * diff * d.inv_px;
            const float cd = d.inv_px * diff;
            gnz = gnz || (x0 + c < w && -(cd + cd) != 0.f);
        }
        float* pd = d.pred + view * npx;
        if (VEC) {
            *reinterpret_cast<float4*>(pd + o) = make_float4(pred[0], pred[1], pred[2], pred[3]);
        } else {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                if (x0 + c < w) {
                    pd[o + c] = pred[c];
                }
            }
        }
    }
    const bool seg_nz = __ballot(gnz) != 0ull;
    lv[view][lane] = make_float4(l[0], l[1], l[2], l[3]);
    __syncthreads();
    if (view == 0 && any) {
        float out[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            float in[NV][1];
#pragma unroll
            for (int v = 0; v < NV; v++) {
                const float4 q = lv[v][lane];
                in[v][0] = c == 0 ? q.x : c == 1 ? q.y : c == 2 ? q.z : q.w;
            }
            float one[1];
            Tree<NV, 1>::run(in, one);
            out[c] = one[0];
        }
        if (VEC) {
            *reinterpret_cast<float4*>(d.loss + o) = make_float4(out[0], out[1], out[2], out[3]);
        } else {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                if (x0 + c < w) {
                    d.loss[o + c] = out[c];
                }
            }
        }
    }
    if (lane == 0 && d.gflag) {
        d.gflag[((size_t)view * h + y) * gridDim.x + blockIdx.x] = seg_nz ? 1u : 0u;
    }
}

// Lanes (8-lane group) g + src of a wave: lane-group shuffle.
__device__ __forceinline__ float grp_shfl(float v, int src) { return __shfl(v, src, 64); }
__device__ __forceinline__ int grp_shfl(int v, int src) { return __shfl(v, src, 64); }

// OR of the 8-bit fields of a wave ballot: the group slots (samples or
// neighbours) that are set in at least one group.
__device__ __forceinline__ uint32_t fold_groups(uint64_t m) {
    m |= m >> 32;
    m |= m >> 16;
    m |= m >> 8;
    return (uint32_t)m & 0xffu;
}

// AntiAliasBwdVtx (stochastic, wide) fused per (view, face) on an 8-lane
// group: the face's n samples (salts 2 and 3, seed = t) are shared by its
// three corner slots. Lane j computes sample s0 + j of each batch of 8; then,
// sample by sample in order, lane k evaluates the pair of neighbour k and the
// corner terms it adds, and the group adds them into its accumulators in
// neighbour order -- per corner the same (sample, neighbour, endpoint)
// sequence of additions as the reference's (vertex, slot) row. Pairs whose
// two pixels have the same mask value carry gr = 0 and are skipped before the
// pair evaluation. Every lane of a wave runs every shuffle (no early exit).
// Also clears the bin counters.
__device__ __forceinline__ void aa_face_bwd_item(const HsrDev& d, uint32_t item, bool valid,
                                                 int j, int gbase) {
    const uint32_t view = valid ? item / d.g.n_faces : 0u;
    const uint32_t f = valid ? item - view * d.g.n_faces : 0u;
    const int w = (int)d.g.width, h = (int)d.g.height;
    const float W = (float)w, H = (float)h;
    const size_t npx = (size_t)w * h;
    const uint32_t* ids = d.ids + view * npx;
    const float* pred = d.pred + view * npx;
    const float* tgt = d.targets + view * npx;
    const float4* clip = d.clip + (size_t)view * d.n_verts;
    const TriFromRecs tris{d.faces, d.arecs + (size_t)view * d.g.n_faces};
    uint32_t vc[3];
    float4 c[3];
    float4 acc[3];
#pragma unroll
    for (int k = 0; k < 3; k++) {
        vc[k] = valid ? (uint32_t)d.faces[f * 3 + k] : 0u;
        c[k] = valid ? clip[vc[k]] : make_float4(0.f, 0.f, 0.f, 1.f);
        acc[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float s3x[3], s3y[3];
    const bool face_ok = valid && d.n_samples > 0 && aa_face_screen(c, W, H, s3x, s3y);
    const uint32_t seed_u = (uint32_t)(int64_t)(*d.t + 0.5f);
    for (uint32_t s0 = 0; s0 < d.n_samples; s0 += 8) {
        // lane j: sample s0 + j and d loss / d pred there,
        // diff = target - pred, -(c diff + c diff); gy = 0 zeroes every gr
        int sx = -1, sy = -1;
        float gy = 0.f;
        if (face_ok && s0 + j < d.n_samples &&
            aa_sample_px(s3x, s3y, f, s0 + j, seed_u, &sx, &sy) && sx >= 0 && sy >= 0 &&
            sx < w && sy < h) {
            const size_t so = (size_t)sy * w + sx;
            const float diff = tgt[so] - pred[so];
            const float cd = d.inv_px * diff;
            gy = -(cd + cd);
        }
        const bool act = sx >= 0 && sy >= 0 && sx < w && sy < h && gy != 0.f;
        uint32_t bmask = fold_groups(__ballot(act));
        while (bmask) {
            const int b = __builtin_ctz(bmask);
            bmask &= bmask - 1;
            const int x = grp_shfl(sx, gbase + b);
            const int y = grp_shfl(sy, gbase + b);
            const float gyb = grp_shfl(gy, gbase + b);
            const bool on = grp_shfl((int)act, gbase + b) != 0;
            // lane k = j: the pair with neighbour k and its corner terms
            uint32_t tflag = 0;
            float tx[3] = {0.f, 0.f, 0.f}, ty[3] = {0.f, 0.f, 0.f}, tw[3] = {0.f, 0.f, 0.f};
            if (on) {
                const int nx = x + kAaOffX[j], ny = y + kAaOffY[j];
                if (!(nx < 0 || ny < 0 || nx >= w || ny >= h)) {
                    const uint32_t its = ids[(size_t)y * w + x];
                    const uint32_t itn = ids[(size_t)ny * w + nx];
                    const float ms = its ? 1.f : 0.f;
                    const float mn = itn ? 1.f : 0.f;
                    float gr = 0.f;
                    gr += gyb * (ms - mn);
                    gr /= 9.f;
                    AaPair pr;
                    if (gr != 0.f && eval_aa_pair(its, itn, x, y, nx, ny, d.g.n_faces, tris, &pr) &&
                        pr.r < 1.f) {
                        float dqa[2], dqb[2];
                        aa_pair_dq(pr, x, y, dqa, dqb);
                        // an endpoint that is corner kc of this face has clip
                        // c[kc]; an active edge has two distinct endpoints
#pragma unroll
                        for (int kc = 0; kc < 3; kc++) {
                            const bool ea = pr.ia == vc[kc];
                            if (ea || pr.ib == vc[kc]) {
                                const float* dq = ea ? dqa : dqb;
                                const float gqx = gr * dq[0];
                                const float gqy = gr * dq[1];
                                tx[kc] = gqx * 0.5f * W / c[kc].w;
                                ty[kc] = gqy * 0.5f * H / c[kc].w;
                                tw[kc] = -(gqx * 0.5f * W * c[kc].x + gqy * 0.5f * H * c[kc].y) /
                                         (c[kc].w * c[kc].w);
                                tflag |= 1u << kc;
                            }
                        }
                    }
                }
            }
            // the group adds neighbour k's terms for k = 0..7 in order
            uint32_t kmask = fold_groups(__ballot(tflag != 0));
            while (kmask) {
                const int k = __builtin_ctz(kmask);
                kmask &= kmask - 1;
                const int src = gbase + k;
                const uint32_t fl = (uint32_t)grp_shfl((int)tflag, src);
#pragma unroll
                for (int kc = 0; kc < 3; kc++) {
                    const float vx = grp_shfl(tx[kc], src);
                    const float vy = grp_shfl(ty[kc], src);
                    const float vw = grp_shfl(tw[kc], src);
                    if (fl >> kc & 1u) {
                        acc[kc].x += vx;
                        acc[kc].y += vy;
                        acc[kc].w += vw;
                    }
                }
            }
        }
    }
    if (valid && j < 3) {
        float4* dst = d.gtri + (size_t)view * 3 * d.g.n_faces;
        dst[(size_t)j * d.g.n_faces + f] = j == 0 ? acc[0] : j == 1 ? acc[1] : acc[2];
    }
}

// Faces whose samples all carry gy = 0 (pred = target at every sample; most
// faces, away from both silhouettes) add nothing: they get their zero
// corner gradients here, one 8-lane group per (view, face) with the sample
// positions and gy of aa_face_bwd_item, and the others are listed (per
// workgroup in LDS, one global append per workgroup) for k_aa_face_bwd.
// Also clears the bin counters and publishes t + 1.
__global__ __launch_bounds__(256) void k_aa_face_scan(HsrDev d) {
    __shared__ uint32_t queue[32];
    __shared__ uint32_t n_q, base_q;
    const uint32_t gi = blockIdx.x * blockDim.x + threadIdx.x;
    publish_t_next(d, gi);
    for (uint32_t b = gi; b < d.bins.n_bins; b += gridDim.x * blockDim.x) {
        const uint32_t c = d.bins.counts[b];
        if (c > d.bins.cap && d.bin_over_max) {
            atomicMax(d.bin_over_max, c);  // rare: the host grows the bins before the next step
        }
        d.bins.counts[b] = 0;
    }
    if (threadIdx.x == 0) {
        n_q = 0;
    }
    __syncthreads();
    const uint32_t nvf = d.g.n_views * d.g.n_faces;
    const uint32_t item = gi >> 3;
    const bool valid = item < nvf;
    const int j = (int)(threadIdx.x & 7u);
    const uint32_t view = valid ? item / d.g.n_faces : 0u;
    const uint32_t f = valid ? item - view * d.g.n_faces : 0u;
    const int w = (int)d.g.width, h = (int)d.g.height;
    const size_t npx = (size_t)w * h;
    bool act = false;
    if (valid && d.n_samples > 0) {
        const float4* clip = d.clip + (size_t)view * d.n_verts;
        float4 c[3];
#pragma unroll
        for (int k = 0; k < 3; k++) {
            c[k] = clip[(uint32_t)d.faces[f * 3 + k]];
        }
        float s3x[3], s3y[3];
        if (aa_face_screen(c, (float)w, (float)h, s3x, s3y)) {
            const uint32_t seed_u = (uint32_t)(int64_t)(*d.t + 0.5f);
            const float* pred = d.pred + view * npx;
            const float* tgt = d.targets + view * npx;
            for (uint32_t smp = (uint32_t)j; smp < d.n_samples && !act; smp += 8) {
                int sx = -1, sy = -1;
                if (aa_sample_px(s3x, s3y, f, smp, seed_u, &sx, &sy) && sx >= 0 && sy >= 0 &&
                    sx < w && sy < h &&
                    (!d.gflag ||
                     d.gflag[((size_t)view * h + sy) * (uint32_t)((w + 255) / 256) + sx / 256])) {
                    // a segment without the flag has gy = 0 at every pixel
                    const size_t so = (size_t)sy * w + sx;
                    const float diff = tgt[so] - pred[so];
                    const float cd = d.inv_px * diff;
                    act = -(cd + cd) != 0.f;
                }
            }
        }
    }
    // the group's verdict on its first lane
    const uint64_t m = __ballot(act);
    const bool any = ((m >> (threadIdx.x & 56u)) & 0xffull) != 0ull;
    if (valid && j == 0) {
        if (any) {
            queue[atomicAdd(&n_q, 1u)] = item;
        } else {
            float4* dst = d.gtri + (size_t)view * 3 * d.g.n_faces;
#pragma unroll
            for (int k = 0; k < 3; k++) {
                dst[(size_t)k * d.g.n_faces + f] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
    }
    __syncthreads();
    if (threadIdx.x == 0 && n_q) {
        base_q = atomicAdd(d.aa_count, n_q);
    }
    __syncthreads();
    if (threadIdx.x < n_q) {
        d.aa_list[base_q + threadIdx.x] = queue[threadIdx.x];
    }
}

// AntiAliasBwdVtx (stochastic, wide) of the listed faces: 8-lane groups walk
// the list (aa_face_bwd_item on each).
constexpr uint32_t kAaFaceBwdGrid = 2048;
__global__ __launch_bounds__(256) void k_aa_face_bwd(HsrDev d) {
    const uint32_t n = *d.aa_count;
    const uint32_t n_groups = gridDim.x * blockDim.x / 8u;
    const int j = (int)(threadIdx.x & 7u);
    const int gbase = (int)(threadIdx.x & 56u);
    for (uint32_t li = (blockIdx.x * blockDim.x + threadIdx.x) >> 3; li < n; li += n_groups) {
        aa_face_bwd_item(d, d.aa_list[li], true, j, gbase);
    }
}

// ColSum of the (vertex, slot) rows per view -- the row of slot d is the
// accumulator of face vf[d][v] at the corner holding v; padding rows are
// zero -- then the shared clip->pos chain and Adam: one lane per (vertex,
// view) for the ColSum, the vertex's first lane for the rest; the last
// workgroup advances t.
template <int NV>
__global__ __launch_bounds__(256) void k_aa_vertex_adam(HsrDev d) {
    publish_bin_over(d);
    vertex_views_adam<NV>(d, [&](uint32_t vtx, uint32_t view, float (&g4)[4]) {
        const float4* gt = d.gtri + (size_t)view * 3 * d.g.n_faces;
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        for (uint32_t d0 = 0; d0 < d.max_deg; d0 += kDegBatch) {
            AdjBatch ab;
            load_adjacency(d, vtx, d0, ab);
            float4 gg[kDegBatch];
#pragma unroll
            for (int i = 0; i < kDegBatch; i++) {
                gg[i] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (ab.f[i] >= 0) {
                    gg[i] = gt[(size_t)first_corner(ab.mask[i]) * d.g.n_faces + ab.f[i]];
                }
            }
            // in slot order; a padding row is zero (adding +0 leaves the sum
            // unchanged, so it is skipped)
#pragma unroll
            for (int i = 0; i < kDegBatch; i++) {
                if (ab.f[i] >= 0) {
                    acc[0] += gg[i].x;
                    acc[1] += gg[i].y;
                    acc[2] += gg[i].z;
                    acc[3] += gg[i].w;
                }
            }
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            g4[r] = acc[r];
        }
    });
}

const char* const kAaKernelNames[kAaKernels] = {"k_aa_setup", "k_aa_raster", "k_aa_fwd",
                                                "k_aa_face_bwd", "k_aa_vertex_adam"};

int launch_aa_setup(const HsrDev& d, hipStream_t s) {
    hipLaunchKernelGGL(k_aa_setup, dim3(div_up(d.g.n_views * d.g.n_faces, 256)), dim3(256), 0, s,
                       d);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int launch_aa_raster(const HsrDev& d, hipStream_t s) {
    hipLaunchKernelGGL(k_aa_raster, dim3(32u * d.g.n_views * div_up(d.g.n_tiles, 8)), dim3(64),
                       0, s, d);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int launch_aa_kernel(const HsrDev& d, hipStream_t s, int k) {
    const RasterGeom& g = d.g;
    const uint32_t nvf = g.n_views * g.n_faces;
    switch (k) {
        case 0:
            hipLaunchKernelGGL(k_aa_clip, dim3(div_up(g.n_views * d.n_verts, 256)), dim3(256), 0,
                               s, d);
            DRESSI_CHECK_LAUNCH();
            return launch_aa_setup(d, s);
        case 1:
            return launch_aa_raster(d, s);
        case 2:
        case 4: {
            const dim3 grid = dim3(div_up(g.width, 256), g.height);
            const bool vec = (g.width & 3u) == 0;
            switch (g.n_views) {
#define DRESSI_NV(N)                                                                      \
    case N:                                                                               \
        if (k == 2) {                                                                     \
            if (vec) {                                                                    \
                hipLaunchKernelGGL((k_aa_fwd<N, true>), grid, dim3(64 * N), 0, s, d);     \
            } else {                                                                      \
                hipLaunchKernelGGL((k_aa_fwd<N, false>), grid, dim3(64 * N), 0, s, d);    \
            }                                                                             \
        } else {                                                                          \
            hipLaunchKernelGGL(k_aa_vertex_adam<N>, dim3(vertex_grid<N>(d.n_verts)),       \
                               dim3(256), 0, s, d);                                        \
        }                                                                                 \
        break;
                DRESSI_NV(1) DRESSI_NV(2) DRESSI_NV(3) DRESSI_NV(4)
                DRESSI_NV(5) DRESSI_NV(6) DRESSI_NV(7) DRESSI_NV(8)
#undef DRESSI_NV
                default:
                    set_error("n_views %u unsupported", g.n_views);
                    return DRESSI_ERR_UNSUPPORTED;
            }
            break;
        }
        default:
            hipLaunchKernelGGL(k_aa_face_scan, dim3(div_up(nvf, 32)), dim3(256), 0, s, d);
            DRESSI_CHECK_LAUNCH();
            hipLaunchKernelGGL(k_aa_face_bwd, dim3(std::min(div_up(nvf, 32), kAaFaceBwdGrid)),
                               dim3(256), 0, s, d);
            break;
    }
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

}  // namespace dressi

using namespace dressi;

namespace {

int check_aa_args(dressi_ctx* ctx, uint32_t n_comp, uint32_t w, uint32_t h) {
    DRESSI_REQUIRE(ctx, "NULL context");
    DRESSI_REQUIRE(n_comp >= 1 && n_comp <= 4, "AntiAlias: n_comp must be 1..4");
    DRESSI_REQUIRE(w > 0 && h > 0, "AntiAlias: empty image");
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    return DRESSI_OK;
}

}  // namespace

namespace dressi {

int aa_render_target(dressi_ctx* ctx, const float* tgt_clip_dev, uint32_t n_tverts,
                     const float* tgt_faces_dev, uint32_t n_tfaces, uint32_t w, uint32_t h,
                     float* out) {
    // mask = Rasterize(tgt, ones), tri = RasterizeFaceId(tgt) into context
    // scratch (slots 4 .. 6), then the AntiAlias forward
    void *ones = nullptr, *mask = nullptr, *tri = nullptr;
    const size_t npx = (size_t)w * h;
    if (int rc = ctx_workspace(ctx, 4, sizeof(float) * (n_tverts ? n_tverts : 1), &ones)) return rc;
    if (int rc = ctx_workspace(ctx, 5, sizeof(float) * npx, &mask)) return rc;
    if (int rc = ctx_workspace(ctx, 6, sizeof(float) * npx, &tri)) return rc;
    std::vector<float> host_ones(n_tverts ? n_tverts : 1, 1.f);
    DRESSI_TRY_HIP(hipMemcpyAsync(ones, host_ones.data(), sizeof(float) * host_ones.size(),
                                  hipMemcpyHostToDevice, ctx->stream));
    if (int rc = dressi_rasterize(ctx, tgt_clip_dev, n_tverts, (const float*)ones, 1,
                                  tgt_faces_dev, n_tfaces, w, h, (float*)mask)) return rc;
    if (int rc = dressi_rasterize_face_id(ctx, tgt_clip_dev, n_tverts, tgt_faces_dev, n_tfaces,
                                          w, h, (float*)tri)) return rc;
    if (int rc = dressi_antialias(ctx, (const float*)mask, 1, (const float*)tri, tgt_clip_dev,
                                  n_tverts, tgt_faces_dev, n_tfaces, w, h, out)) return rc;
    // the host vector must outlive the async copy
    DRESSI_TRY_HIP(hipStreamSynchronize(ctx->stream));
    return DRESSI_OK;
}

}  // namespace dressi

extern "C" {

int dressi_antialias_batch(dressi_ctx* ctx, const float* img, uint32_t n_comp, const float* tri,
                           const float* clip, uint32_t n_verts, int clip_per_item,
                           const float* faces, uint32_t n_faces, uint32_t width, uint32_t height,
                           uint32_t n_items, float* out) {
    if (int rc = check_aa_args(ctx, n_comp, width, height)) return rc;
    DRESSI_REQUIRE(img && tri && clip && (faces || n_faces == 0) && out,
                   "dressi_antialias: NULL buffer");
    DRESSI_REQUIRE(n_items <= kMaxBatchItems, "batch of %u items exceeds %u", n_items,
                   kMaxBatchItems);
    if (n_items == 0) {
        return DRESSI_OK;
    }
    const uint32_t npx = width * height;
    hipLaunchKernelGGL(k_antialias_op, dim3(div_up(npx, 256), n_items), dim3(256), 0,
                       ctx->stream, img, n_comp, tri, (const float4*)clip, n_verts, clip_per_item,
                       faces, n_faces, width, height, out);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int dressi_antialias(dressi_ctx* ctx, const float* img, uint32_t n_comp, const float* tri,
                     const float* clip, uint32_t n_verts, const float* faces, uint32_t n_faces,
                     uint32_t width, uint32_t height, float* out) {
    return dressi_antialias_batch(ctx, img, n_comp, tri, clip, n_verts, 0, faces, n_faces, width,
                                  height, 1, out);
}

int dressi_antialias_bwd_img_batch(dressi_ctx* ctx, const float* gy, uint32_t n_comp,
                                   const float* tri, const float* clip, uint32_t n_verts,
                                   int clip_per_item, const float* faces, uint32_t n_faces,
                                   uint32_t width, uint32_t height, uint32_t n_items, float* out) {
    if (int rc = check_aa_args(ctx, n_comp, width, height)) return rc;
    DRESSI_REQUIRE(gy && tri && clip && (faces || n_faces == 0) && out,
                   "dressi_antialias_bwd_img: NULL buffer");
    DRESSI_REQUIRE(n_items <= kMaxBatchItems, "batch of %u items exceeds %u", n_items,
                   kMaxBatchItems);
    if (n_items == 0) {
        return DRESSI_OK;
    }
    const uint32_t npx = width * height;
    hipLaunchKernelGGL(k_antialias_bwd_img_op, dim3(div_up(npx, 256), n_items), dim3(256), 0,
                       ctx->stream, gy, n_comp, tri, (const float4*)clip, n_verts, clip_per_item,
                       faces, n_faces, width, height, out);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int dressi_antialias_bwd_img(dressi_ctx* ctx, const float* gy, uint32_t n_comp, const float* tri,
                             const float* clip, uint32_t n_verts, const float* faces,
                             uint32_t n_faces, uint32_t width, uint32_t height, float* out) {
    return dressi_antialias_bwd_img_batch(ctx, gy, n_comp, tri, clip, n_verts, 0, faces, n_faces,
                                          width, height, 1, out);
}

int dressi_antialias_bwd_vtx_batch(dressi_ctx* ctx, const float* gy, const float* img,
                                   uint32_t n_comp, const float* tri, const float* clip,
                                   uint32_t n_verts, int clip_per_item, const float* faces,
                                   uint32_t n_faces, const float* vtx_faces, uint32_t max_deg,
                                   const float* seeds, uint32_t n_samples, int wide,
                                   uint32_t width, uint32_t height, uint32_t n_items, float* out) {
    if (int rc = check_aa_args(ctx, n_comp, width, height)) return rc;
    DRESSI_REQUIRE(gy && img && tri && clip && (faces || n_faces == 0) && vtx_faces && out,
                   "dressi_antialias_bwd_vtx: NULL buffer");
    DRESSI_REQUIRE(!wide || n_samples > 0, "AntiAliasBwdVtx: wide requires stochastic samples");
    DRESSI_REQUIRE(n_samples == 0 || seeds, "AntiAliasBwdVtx: NULL seed");
    DRESSI_REQUIRE(n_items <= kMaxBatchItems, "batch of %u items exceeds %u", n_items,
                   kMaxBatchItems);
    if (n_verts == 0 || n_items == 0) {
        return DRESSI_OK;
    }
    if (n_samples == 0) {
        hipLaunchKernelGGL(k_antialias_bwd_vtx_exact_op, dim3(div_up(n_verts, 128), n_items),
                           dim3(128), 0, ctx->stream, gy, img, n_comp, tri, (const float4*)clip,
                           n_verts, clip_per_item, faces, n_faces, vtx_faces, max_deg, width,
                           height, (float4*)out);
    } else {
        const uint32_t rows = wide ? max_deg : 1u;
        DRESSI_REQUIRE((uint64_t)n_verts * rows * 8 < (1ull << 32), "AntiAliasBwdVtx: too many rows");
        hipLaunchKernelGGL(k_antialias_bwd_vtx_op, dim3(div_up(n_verts * rows * 8, 256), n_items),
                           dim3(256), 0, ctx->stream, gy, img, n_comp, tri, (const float4*)clip,
                           n_verts, clip_per_item, faces, n_faces, vtx_faces, max_deg, seeds,
                           n_samples, wide, width, height, (float4*)out);
    }
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int dressi_antialias_bwd_vtx(dressi_ctx* ctx, const float* gy, const float* img, uint32_t n_comp,
                             const float* tri, const float* clip, uint32_t n_verts,
                             const float* faces, uint32_t n_faces, const float* vtx_faces,
                             uint32_t max_deg, const float* seed, uint32_t n_samples, int wide,
                             uint32_t width, uint32_t height, float* out) {
    return dressi_antialias_bwd_vtx_batch(ctx, gy, img, n_comp, tri, clip, n_verts, 0, faces,
                                          n_faces, vtx_faces, max_deg, seed, n_samples, wide,
                                          width, height, 1, out);
}

int dressi_col_sum_batch(dressi_ctx* ctx, const float* x, uint32_t n_comp, uint32_t width,
                         uint32_t height, uint32_t n_items, float* out) {
    DRESSI_REQUIRE(ctx && x && out, "dressi_col_sum: NULL buffer");
    DRESSI_REQUIRE(n_comp >= 1 && n_comp <= 4, "ColSum: n_comp must be 1..4");
    DRESSI_REQUIRE(n_items <= kMaxBatchItems, "batch of %u items exceeds %u", n_items,
                   kMaxBatchItems);
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    if (width == 0 || n_items == 0) {
        return DRESSI_OK;
    }
    hipLaunchKernelGGL(k_col_sum_op, dim3(div_up(width * n_comp, 256), n_items), dim3(256), 0,
                       ctx->stream, x, n_comp, width, height, out);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int dressi_col_sum(dressi_ctx* ctx, const float* x, uint32_t n_comp, uint32_t width,
                   uint32_t height, float* out) {
    return dressi_col_sum_batch(ctx, x, n_comp, width, height, 1, out);
}

}  // extern "C"
