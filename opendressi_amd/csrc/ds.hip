// ds.hip -- GatherDistGrad (src/core/f_ops.cpp:1248-1358): the exact
// backward of RasterizeSoft's dist channel w.r.t. the hard clip positions
// (the backward RasterizeSoft builds, f_ops.cpp:1448-1455, and what
// dressi.torch.rasterize_soft's VJP runs).
#include <cstdint>

#include "internal.h"
#include "soft_clip.h"

namespace dressi {
namespace {

// cpu_raster.cpp:114-151 (SignedDistToTri) with the argmin edge and its
// clamped parameter.
struct TriDistE {
    float dist;
    int edge;
    float t;
};

__device__ __forceinline__ TriDistE signed_dist_edge(float px, float py, const float sx[3],
                                                     const float sy[3]) {
    TriDistE best;
    best.dist = 0.f;
    best.edge = 0;
    best.t = 0.f;
    float best_d2 = -1.f;
    int n_pos = 0, n_neg = 0;
#pragma unroll
    for (int k = 0; k < 3; k++) {
        const int k1 = (k + 1) % 3;
        const float ex = sx[k1] - sx[k];
        const float ey = sy[k1] - sy[k];
        const float len2 = ex * ex + ey * ey;
        float t = 0.f;
        if (len2 > kDistEps * kDistEps) {
            t = ((px - sx[k]) * ex + (py - sy[k]) * ey) / len2;
            t = smin(smax(t, 0.f), 1.f);
        }
        const float qx = sx[k] + t * ex;
        const float qy = sy[k] + t * ey;
        const float dx = px - qx;
        const float dy = py - qy;
        const float d2 = dx * dx + dy * dy;
        if (best_d2 < 0.f || d2 < best_d2) {
            best_d2 = d2;
            best.edge = k;
            best.t = t;
        }
        const float cr = ex * (py - sy[k]) - ey * (px - sx[k]);
        n_pos += (cr >= 0.f);
        n_neg += (cr <= 0.f);
    }
    const float sgn = (n_pos == 3 || n_neg == 3) ? 1.f : -1.f;
    best.dist = sgn * sqrtf(smax(best_d2, 0.f));
    return best;
}

// cpu_raster.cpp:153-175 (SignedDistGradToTri): d dist / d corner k, the
// argmin edge and t held fixed (envelope theorem); 0 on the boundary.
__device__ __forceinline__ void signed_dist_grad_k(float px, float py, const float sx[3],
                                                   const float sy[3], const TriDistE& td, int k,
                                                   float* gx, float* gy) {
    *gx = 0.f;
    *gy = 0.f;
    const float d = fabsf(td.dist);
    if (d < kDistEps) {
        return;
    }
    const int ia = td.edge;
    const int ib = (td.edge + 1) % 3;
    if (k != ia && k != ib) {
        return;
    }
    const float qx = sx[ia] + td.t * (sx[ib] - sx[ia]);
    const float qy = sy[ia] + td.t * (sy[ib] - sy[ia]);
    const float sgn = td.dist >= 0.f ? 1.f : -1.f;
    const float nx = (px - qx) / d;
    const float ny = (py - qy) / d;
    if (k == ia) {
        *gx = -sgn * (1.f - td.t) * nx;
        *gy = -sgn * (1.f - td.t) * ny;
    } else {
        *gx = -sgn * td.t * nx;
        *gy = -sgn * td.t * ny;
    }
}

// A face's corners: vertex ids, hard clips and projected screen positions;
// false when a corner is not projectable (the reference skips its pixels).
struct FaceCorners {
    uint32_t idx[3];
    float4 c[3];
    float sx[3], sy[3];
};

__device__ __forceinline__ bool load_face(const float* faces, const float4* clip, uint32_t n_verts,
                                          uint32_t f, float W, float H, FaceCorners* fc,
                                          uint32_t* err) {
#pragma unroll
    for (int k = 0; k < 3; k++) {
        fc->idx[k] = (uint32_t)(int64_t)(faces[(size_t)f * 3 + k] + 0.5f);
        if (fc->idx[k] >= n_verts) {
            atomicOr(err, 2u);
            return false;
        }
        fc->c[k] = clip[fc->idx[k]];
    }
#pragma unroll
    for (int k = 0; k < 3; k++) {
        if (!clip_w_valid(fc->c[k].w)) {
            return false;
        }
        const ScreenVert v = project_to_screen(fc->c[k].x, fc->c[k].y, fc->c[k].z, fc->c[k].w, W, H);
        fc->sx[k] = v.x;
        fc->sy[k] = v.y;
    }
    return true;
}

// The pixel bbox of a face's soft triangle (SoftClip of its hard clips, as
// the soft raster's setup): every pixel whose RasterizeSoft winner is the
// face lies in it. False when the face produces no fragment.
__device__ __forceinline__ bool soft_bbox(const FaceCorners& fc, uint32_t w, uint32_t h,
                                          float radius, int* bx0, int* by0, int* bx1, int* by1) {
    float4 sc[3];
    soft_clip_face(fc.c, w, h, radius, sc);
    float x[3], y[3];
#pragma unroll
    for (int k = 0; k < 3; k++) {
        if (!clip_w_valid(sc[k].w)) {
            return false;
        }
        const ScreenVert v = project_to_screen(sc[k].x, sc[k].y, sc[k].z, sc[k].w, (float)w, (float)h);
        x[k] = v.x;
        y[k] = v.y;
    }
    if (fabsf(tri_area(x[0], y[0], x[1], y[1], x[2], y[2])) < kDistEps) {
        return false;
    }
    pixel_bbox(x[0], x[1], x[2], y[0], y[1], y[2], (int)w, (int)h, bx0, by0, bx1, by1);
    return *bx0 <= *bx1 && *by0 <= *by1;
}

// Adds pixel (x, y)'s contribution to corner k of `fc` into acc (the
// screen -> clip Jacobian of f_ops.cpp:1342-1350).
__device__ __forceinline__ void add_corner(const FaceCorners& fc, const TriDistE& td, float px,
                                           float py, int k, float g, float W, float H,
                                           float4* acc) {
    float gsx0, gsy0;
    signed_dist_grad_k(px, py, fc.sx, fc.sy, td, k, &gsx0, &gsy0);
    const float gsx = g * gsx0;
    const float gsy = g * gsy0;
    if (gsx == 0.f && gsy == 0.f) {
        return;
    }
    const float4 c = fc.c[k];
    acc->x += gsx * 0.5f * W / c.w;
    acc->y += gsy * 0.5f * H / c.w;
    acc->w += -(gsx * 0.5f * W * c.x + gsy * 0.5f * H * c.y) / (c.w * c.w);
}

// Wide layout, one thread per (adjacency row d, vertex u): face f =
// vtx_faces[d][u]'s pixels in raster order (its soft bbox, face-id guard),
// the corners that are u. Only the first row holding f for u receives
// (the reference's row_of).
__global__ __launch_bounds__(128) void k_gather_dist_grad_wide(
        const float4* gy, const float4* rs, const float4* clip, uint32_t n_verts,
        const float* faces, uint32_t n_faces, const float* vf, uint32_t max_deg, float radius,
        uint32_t w, uint32_t h, uint32_t* err, float4* out) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= max_deg * n_verts) {
        return;
    }
    const uint32_t d = i / n_verts, u = i - d * n_verts;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    const float fv = vf[i];
    if (fv >= -0.5f) {
        const uint32_t f = (uint32_t)(int64_t)(fv + 0.5f);
        bool first = true;
        for (uint32_t e = 0; e < d; e++) {
            const float fe = vf[(size_t)e * n_verts + u];
            first = first && !(fe >= -0.5f && (uint32_t)(int64_t)(fe + 0.5f) == f);
        }
        const float W = (float)w, H = (float)h;
        FaceCorners fc;
        int bx0, by0, bx1, by1;
        if (f >= n_faces) {
            atomicOr(err, 2u);
        } else if (first && load_face(faces, clip, n_verts, f, W, H, &fc, err) &&
                   soft_bbox(fc, w, h, radius, &bx0, &by0, &bx1, &by1)) {
            for (int y = by0; y <= by1; y++) {
                for (int x = bx0; x <= bx1; x++) {
                    const size_t o = (size_t)y * w + x;
                    const float4 r = rs[o];
                    if (r.w < 0.5f || (uint32_t)(int64_t)(r.y + 0.5f) != f) {
                        continue;
                    }
                    const float g = gy[o].x;
                    if (g == 0.f) {
                        continue;
                    }
                    const float px = (float)x + 0.5f, py = (float)y + 0.5f;
                    const TriDistE td = signed_dist_edge(px, py, fc.sx, fc.sy);
#pragma unroll
                    for (int k = 0; k < 3; k++) {
                        if (fc.idx[k] == u) {
                            add_corner(fc, td, px, py, k, g, W, H, &acc);
                        }
                    }
                }
            }
        }
    }
    out[i] = acc;
}

// {V,1} layout, one thread per vertex: the union of its incident faces'
// soft bboxes in raster order, pixels whose face is incident to it.
__global__ __launch_bounds__(128) void k_gather_dist_grad_vtx(
        const float4* gy, const float4* rs, const float4* clip, uint32_t n_verts,
        const float* faces, uint32_t n_faces, const float* vf, uint32_t max_deg, float radius,
        uint32_t w, uint32_t h, uint32_t* err, float4* out) {
    const uint32_t u = blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= n_verts) {
        return;
    }
    const float W = (float)w, H = (float)h;
    int ux0 = (int)w, uy0 = (int)h, ux1 = -1, uy1 = -1;
    for (uint32_t d = 0; d < max_deg; d++) {
        const float fv = vf[(size_t)d * n_verts + u];
        if (fv < -0.5f) {
            continue;
        }
        const uint32_t f = (uint32_t)(int64_t)(fv + 0.5f);
        FaceCorners fc;
        int bx0, by0, bx1, by1;
        if (f >= n_faces) {
            atomicOr(err, 2u);
        } else if (load_face(faces, clip, n_verts, f, W, H, &fc, err) &&
                   soft_bbox(fc, w, h, radius, &bx0, &by0, &bx1, &by1)) {
            ux0 = min(ux0, bx0);
            uy0 = min(uy0, by0);
            ux1 = max(ux1, bx1);
            uy1 = max(uy1, by1);
        }
    }
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int y = uy0; y <= uy1; y++) {
        for (int x = ux0; x <= ux1; x++) {
            const size_t o = (size_t)y * w + x;
            const float4 r = rs[o];
            if (r.w < 0.5f) {
                continue;
            }
            const float g = gy[o].x;
            if (g == 0.f) {
                continue;
            }
            const uint32_t f = (uint32_t)(int64_t)(r.y + 0.5f);
            bool inc = false;
            for (uint32_t d = 0; d < max_deg && !inc; d++) {
                const float fv = vf[(size_t)d * n_verts + u];
                inc = fv >= -0.5f && (uint32_t)(int64_t)(fv + 0.5f) == f;
            }
            FaceCorners fc;
            if (!inc || f >= n_faces || !load_face(faces, clip, n_verts, f, W, H, &fc, err)) {
                continue;
            }
            const float px = (float)x + 0.5f, py = (float)y + 0.5f;
            const TriDistE td = signed_dist_edge(px, py, fc.sx, fc.sy);
#pragma unroll
            for (int k = 0; k < 3; k++) {
                if (fc.idx[k] == u) {
                    add_corner(fc, td, px, py, k, g, W, H, &acc);
                }
            }
        }
    }
    out[u] = acc;
}

}  // namespace
}  // namespace dressi

using namespace dressi;

extern "C" int dressi_gather_dist_grad(dressi_ctx* ctx, const float* gy, const float* rs,
                                       const float* clip, uint32_t n_verts, const float* faces,
                                       uint32_t n_faces, const float* vtx_faces, uint32_t max_deg,
                                       float radius_px, int wide, uint32_t width, uint32_t height,
                                       float* out) {
    DRESSI_REQUIRE(ctx && gy && rs && clip && faces && vtx_faces && out, "bad arguments");
    DRESSI_REQUIRE(radius_px > 0.f, "radius_px must be > 0");
    DRESSI_REQUIRE(max_deg >= 1, "max_deg must be >= 1");
    DRESSI_REQUIRE((uint64_t)max_deg * n_verts < (1ull << 31), "adjacency too large");
    if (!n_verts) return DRESSI_OK;
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    if (wide) {
        hipLaunchKernelGGL(k_gather_dist_grad_wide, dim3(div_up(max_deg * n_verts, 128)),
                           dim3(128), 0, ctx->stream, (const float4*)gy, (const float4*)rs,
                           (const float4*)clip, n_verts, faces, n_faces, vtx_faces, max_deg,
                           radius_px, width, height, ctx->d_err, (float4*)out);
    } else {
        hipLaunchKernelGGL(k_gather_dist_grad_vtx, dim3(div_up(n_verts, 128)), dim3(128), 0,
                           ctx->stream, (const float4*)gy, (const float4*)rs, (const float4*)clip,
                           n_verts, faces, n_faces, vtx_faces, max_deg, radius_px, width, height,
                           ctx->d_err, (float4*)out);
    }
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}
