// hsr.hip -- the fused silhouette-fit plan (forward + backward + Adam as one
// hipGraph; technique HardSoftRas here, the AA technique's kernels in aa.hip)
// and the per-op LookupFaces / FaceFetch kernels.
#include <cstring>
#include <vector>

#include "hsr_chain.h"
#include "plan.h"
#include "soft_clip.h"

namespace dressi {

// SoftClip + RasterizeSoft setup per (view, face), appended to the soft bins.
__global__ __launch_bounds__(256) void k_hsr_setup(HsrDev d) {
    __shared__ BinLds blds;
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    const bool live = i < d.g.n_views * d.g.n_faces;
    const uint32_t view = live ? i / d.g.n_faces : 0;
    const uint32_t f = live ? i - view * d.g.n_faces : 0;
    SoftRec r;
    r.bx0 = 1;
    r.bx1 = 0;
    r.by0 = 1;
    r.by1 = 0;
    if (live) {
        float4 hc[3], sc[3];
        face_clips(d, view, f, hc);
        soft_clip_face(hc, d.g.width, d.g.height, d.radius, sc);
        soft_setup(sc, hc, (float)f, d.g.width, d.g.height, &r);
        d.recs[i] = r;
        d.cull[i] = cull_setup(r);
        float cs[3][2];
        chain_screen(hc, (float)d.g.width, (float)d.g.height, cs);
        d.fscr[(size_t)i * 2] = make_float4(cs[0][0], cs[0][1], cs[1][0], cs[1][1]);
        d.fscr[(size_t)i * 2 + 1] = make_float4(cs[2][0], cs[2][1], 0.f, 0.f);
    }
    const bool valid = live && r.bx0 <= r.bx1 && r.by0 <= r.by1;
    bin_append(d.bins, d.g, valid, view, f, r.bx0, r.by0, r.bx1, r.by1, soft_bin_tri(r), blds,
               &d.heavy);
}

// Visibility: one single-wave workgroup per (view, 8x8 block) resolves the
// RasterizeSoft winner of every pixel and writes the face-id buffer (face +
// 1, bit 31 for rim winners, 0 for background). The first 4 kHeavySegs
// heavy.cap workgroups take the four blocks of each listed heavy bin
// (slot-major over the segments); the others walk every (view, tile, block)
// and skip the listed bins. Workgroup w runs on
// XCD w % 8: tiles are dealt to the XCDs round robin (neighbouring tiles,
// and so the costly silhouette bands, spread over all of them), and the
// four blocks of a tile of a view are consecutive on one XCD.
__global__ __launch_bounds__(64) void k_hsr_raster(HsrDev d) {
    uint32_t view, tile, q;
    BinView bv;
    const uint32_t n_first = 4u * kHeavySegs * d.heavy.cap;
    if (blockIdx.x < n_first) {
        const uint32_t k = blockIdx.x >> 3;
        q = k & 3u;
        const uint32_t j = (k >> 2) * 8u + (blockIdx.x & 7u);
        const uint32_t seg = j % kHeavySegs, slot = j / kHeavySegs;
        if (slot >= d.heavy.count[seg]) {
            return;
        }
        const uint32_t bin = d.heavy.list[seg * kHeavySegCap + slot];
        view = geom_div(bin, d.g.n_tiles, d.g.tiles_m);
        tile = bin - view * d.g.n_tiles;
        bv = bin_view(d.bins, bin, d.g.n_faces);
    } else {
        const uint32_t b = blockIdx.x - n_first;
        const uint32_t per = (d.g.n_tiles + 7u) / 8u;
        const uint32_t k = b >> 3;
        q = k & 3u;
        const uint32_t lt = geom_div(k >> 2, d.g.n_views, d.g.views_m);
        view = (k >> 2) - lt * d.g.n_views;
        tile = lt * 8u + (b & 7u);
        if (lt >= per || tile >= d.g.n_tiles) {
            return;
        }
        const uint32_t bin = view * d.g.n_tiles + tile;
        // the counter and this lane's list entry in one round trip, before
        // the heavy-list test that reads the counter
        bv = bin_view(d.bins, bin, d.g.n_faces);
        if (heavy_listed(d.heavy, bv.count, bin)) {
            return;
        }
    }
    const uint32_t trow = geom_div(tile, d.g.tiles_x, d.g.tiles_x_m);
    const int bx = (int)((tile - trow * d.g.tiles_x) * kTile + (q & 1u) * 8u);
    const int by = (int)(trow * kTile + (q >> 1) * 8u);
    if (bx >= (int)d.g.width || by >= (int)d.g.height) {
        return;
    }
    const int lane = threadIdx.x & 63;
    const int px = bx + (lane & 7);
    const int py = by + (lane >> 3);
    const size_t vf = (size_t)view * d.g.n_faces;
    __shared__ ResolveLds lds;
    const PixelBest best = resolve_block(d.recs + vf, d.cull + vf, bv, bx, by, d.radius, nullptr,
                                         d.g.width, lds);
    if (px < (int)d.g.width && py < (int)d.g.height) {
        uint32_t id = 0;
        if (best.key != kEmptyKey) {
            id = (key_face(best.key) + 1) | (best.hard ? 0u : kRimFlag);
            if (!best.hard) {
                d.rimf[vf + key_face(best.key)] = 1;
            }
        }
        d.ids[(size_t)view * d.g.width * d.g.height + (size_t)py * d.g.width + px] = id;
    }
}

// Forward tail per pixel: pred of every view from its face-id entry
// (background 0; a hard-branch winner gives cov * step(0, dist) = 1 >= the
// soft silhouette, so max(hard, soft) = 1; a rim winner evaluates the pixel
// chain), the L2 loss per view and their SumPixelWise over views. A lane
// takes P pixels of a row (width % P == 0): the face ids of every view as
// one P-word load, the targets as P bytes (0 / 1 targets) or P floats, pred
// and loss as P-word stores.
template <int P>
struct LossVec;
template <>
struct LossVec<1> {
    static __device__ __forceinline__ void ids(const uint32_t* p, uint32_t (&v)[1]) { v[0] = *p; }
    static __device__ __forceinline__ void bytes(const uint8_t* p, float (&v)[1]) {
        v[0] = (float)*p;
    }
    static __device__ __forceinline__ void floats(const float* p, float (&v)[1]) { v[0] = *p; }
    static __device__ __forceinline__ void store(float* p, const float (&v)[1]) { *p = v[0]; }
};
template <>
struct LossVec<4> {
    static __device__ __forceinline__ void ids(const uint32_t* p, uint32_t (&v)[4]) {
        const uint4 q = *reinterpret_cast<const uint4*>(p);
        v[0] = q.x;
        v[1] = q.y;
        v[2] = q.z;
        v[3] = q.w;
    }
    static __device__ __forceinline__ void bytes(const uint8_t* p, float (&v)[4]) {
        const uint32_t q = *reinterpret_cast<const uint32_t*>(p);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            v[c] = (float)((q >> (8 * c)) & 0xffu);
        }
    }
    static __device__ __forceinline__ void floats(const float* p, float (&v)[4]) {
        const float4 q = *reinterpret_cast<const float4*>(p);
        v[0] = q.x;
        v[1] = q.y;
        v[2] = q.z;
        v[3] = q.w;
    }
    static __device__ __forceinline__ void store(float* p, const float (&v)[4]) {
        *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    }
};

template <int NV, int P>
__device__ __forceinline__ void loss_block(const HsrDev& d, uint32_t bkx, uint32_t bky) {
    static_assert(NV * P <= 32, "rim bits");
    const uint32_t lane = threadIdx.x & 63u, wv = threadIdx.x >> 6;
    const uint32_t x0 = (bkx * 64 + lane) * P;
    const uint32_t y = bky * 4 + wv;
    // lanes past the edge stay for the wave's exchanges (no rim, no stores)
    const bool valid = x0 < d.g.width && y < d.g.height;
    const size_t npx = (size_t)d.g.width * d.g.height;
    const size_t o = valid ? (size_t)y * d.g.width + x0 : 0;
    uint32_t id[NV][P];
    float tg[NV][P];
    // the loads of every view issued together (invalid lanes read pixel 0)
#pragma unroll
    for (int view = 0; view < NV; view++) {
        LossVec<P>::ids(d.ids + view * npx + o, id[view]);
    }
    if (d.tgt8) {
#pragma unroll
        for (int view = 0; view < NV; view++) {
            LossVec<P>::bytes(d.tgt8 + view * npx + o, tg[view]);
        }
    } else {
#pragma unroll
        for (int view = 0; view < NV; view++) {
            LossVec<P>::floats(d.targets + view * npx + o, tg[view]);
        }
    }
#pragma unroll
    for (int view = 0; view < NV; view++) {
#pragma unroll
        for (int c = 0; c < P; c++) {
            id[view][c] = valid ? id[view][c] : 0u;
        }
    }
    // hard-branch winners and background directly; the rim winners (a few
    // per silhouette crossing) are dealt out one per lane, 64 per round, so a
    // wave evaluates its rim pixels side by side instead of one after another
    __shared__ uint2 s_item[4][64];  // (face id, lane | c << 6 | view << 8)
    __shared__ float s_pred[4][64];
    float pred[NV][P];
    uint32_t rim = 0;  // bit view * P + c
#pragma unroll
    for (int view = 0; view < NV; view++) {
#pragma unroll
        for (int c = 0; c < P; c++) {
            pred[view][c] = id[view][c] ? 1.f : 0.f;
            rim |= (id[view][c] >> 31) << (view * P + c);
        }
    }
    if (__ballot(rim != 0)) {
        // exclusive prefix of the lanes' rim counts
        const uint32_t cnt = __popc(rim);
        uint32_t incl = cnt;
#pragma unroll
        for (int k = 1; k < 64; k <<= 1) {
            const uint32_t t = (uint32_t)__shfl_up((int)incl, k);
            incl += lane >= (uint32_t)k ? t : 0u;
        }
        const uint32_t first = incl - cnt;
        const uint32_t total = (uint32_t)__shfl((int)incl, 63);
        for (uint32_t base = 0; base < total; base += 64) {
            uint32_t k = first;
#pragma unroll
            for (int view = 0; view < NV; view++) {
#pragma unroll
                for (int c = 0; c < P; c++) {
                    if ((rim >> (view * P + c)) & 1u) {
                        if (k - base < 64u) {
                            s_item[wv][k - base] = make_uint2(
                                id[view][c], lane | (uint32_t)c << 6 | (uint32_t)view << 8);
                        }
                        k++;
                    }
                }
            }
            wave_lds_fence();
            if (base + lane < total) {
                const uint2 it = s_item[wv][lane];
                const uint32_t view = it.y >> 8, c = (it.y >> 6) & 3u, owner = it.y & 63u;
                const size_t fi = (size_t)view * d.g.n_faces + (it.x & ~kRimFlag) - 1;
                const float4 a = d.fscr[fi * 2];
                const float4 b = d.fscr[fi * 2 + 1];
                PixelFw st;
                st.s[0][0] = a.x;
                st.s[0][1] = a.y;
                st.s[1][0] = a.z;
                st.s[1][1] = a.w;
                st.s[2][0] = b.x;
                st.s[2][1] = b.y;
                const uint32_t px = (bkx * 64 + owner) * P + c;
                pixel_fw_screen(1.f, -1.f, 1.f, (float)px + 0.5f, (float)y + 0.5f,
                                d.sigma_scale, st);
                s_pred[wv][lane] = st.pred;
            }
            wave_lds_fence();
            k = first;
#pragma unroll
            for (int view = 0; view < NV; view++) {
#pragma unroll
                for (int c = 0; c < P; c++) {
                    if ((rim >> (view * P + c)) & 1u) {
                        if (k - base < 64u) {
                            pred[view][c] = s_pred[wv][k - base];
                        }
                        k++;
                    }
                }
            }
            wave_lds_fence();
        }
    }
    if (!valid) {
        return;
    }
    if (d.pred) {
#pragma unroll
        for (int view = 0; view < NV; view++) {
            LossVec<P>::store(d.pred + view * npx + o, pred[view]);
        }
    }
    float outp[P];
#pragma unroll
    for (int c = 0; c < P; c++) {
        float lv[NV][1];
#pragma unroll
        for (int view = 0; view < NV; view++) {
            const float diff = tg[view][c] - pred[view][c];
            lv[view][0] = diff * diff * d.inv_px;
        }
        float out[1];
        Tree<NV, 1>::run(lv, out);
        outp[c] = out[0];
    }
    LossVec<P>::store(d.loss + o, outp);
}

template <int NV, int P>
__global__ __launch_bounds__(256) void k_hsr_loss(HsrDev d) {
    loss_block<NV, P>(d, blockIdx.x, blockIdx.y);
}

// FaceFetchBwd (stochastic, n samples, seed = t) fused with the pixel
// chain's backward at each accepted sample: per (view, face) the three
// corner-clip gradients (src/core/f_ops.cpp:1646-1729, 1700-1727). Samples
// on pixels whose winner is a hard-branch fragment contribute exactly zero
// (pred = max(1, soft) passes no gradient to soft) and are skipped, so a
// face that won no rim pixel (rimf = 0; most faces) has no sample that
// counts: one lane per (view, face) writes its zero gradient, and the
// workgroup queues its rim faces in LDS. A group of kSampleLanes lanes then
// takes each queued face: lane j evaluates samples j, j + kSampleLanes, ...,
// and the group's first lane adds the lanes' gradients in sample order
// (lanes without an accepted sample add +0, which leaves the sum unchanged:
// it starts at +0 and never becomes -0).
constexpr int kSampleLanes = 8;
// (view, face) items above which the face backward queues its rim faces
// (measured: 2048 x 2048 x 4 views, 327 680 items: 36 -> 26 us; 512 x 512 x 4
// views, 20 480 items: 11 -> 20 us, so the form with a group per item stays)
constexpr uint32_t kFaceBwdQueueMin = 131072;

// One queued rim face (item = view * F + face) on the kSampleLanes lanes of
// a group (lane j of the group; gbase: the group's first lane in the wave).
__device__ __forceinline__ void face_bwd_item(const HsrDev& d, uint32_t item, int j, int gbase) {
    const uint32_t view = item / d.g.n_faces;
    const uint32_t f = item - view * d.g.n_faces;
    const float W = (float)d.g.width, H = (float)d.g.height;
    float4 c[3];
    face_clips(d, view, f, c);
    float4 acc[3];
#pragma unroll
    for (int k = 0; k < 3; k++) {
        acc[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const bool ok = c[0].w > 1e-6f && c[1].w > 1e-6f && c[2].w > 1e-6f;
    float s[3][2];
#pragma unroll
    for (int k = 0; k < 3; k++) {
        s[k][0] = (c[k].x / c[k].w * 0.5f + 0.5f) * W;
        s[k][1] = (c[k].y / c[k].w * 0.5f + 0.5f) * H;
    }
    const uint32_t seed_u = (uint32_t)(int64_t)(*d.t + 0.5f);
    const size_t npx = (size_t)d.g.width * d.g.height;
    const uint32_t* ids = d.ids + view * npx;
    const float* tgt = d.targets + view * npx;
    const uint8_t* tgt8 = d.tgt8 ? d.tgt8 + view * npx : nullptr;
    const uint32_t want = (f + 1) | kRimFlag;
    for (uint32_t s0 = 0; s0 < d.n_samples && __any(ok); s0 += kSampleLanes) {
        const uint32_t smp = s0 + (uint32_t)j;
        int64_t pix = -1;
        if (ok && smp < d.n_samples) {
            const int e = (int)(smp % 3);
            const float* a = s[e];
            const float* b = s[(e + 1) % 3];
            const float ex = b[0] - a[0];
            const float ey = b[1] - a[1];
            const float len = sqrtf(ex * ex + ey * ey);
            if (!(len < 1e-6f)) {
                const float u = hash_to_unit(f, smp, seed_u, 0);
                const float off = (hash_to_unit(f, smp, seed_u, 1) * 2.f - 1.f) * d.radius;
                const float spx = a[0] + u * ex - off * (ey / len);
                const float spy = a[1] + u * ey + off * (ex / len);
                const int ix = (int)floorf(spx);
                const int iy = (int)floorf(spy);
                if (ix >= 0 && iy >= 0 && ix < (int)d.g.width && iy < (int)d.g.height) {
                    pix = (int64_t)iy * d.g.width + ix;
                }
            }
        }
        // other faces and hard-branch winners (zero gradient) are skipped
        const bool hit = pix >= 0 && ids[pix] == want;
        float4 g[3];
#pragma unroll
        for (int k = 0; k < 3; k++) {
            g[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if (hit) {
            const int ix = (int)(pix % d.g.width), iy = (int)(pix / d.g.width);
            const float pcx = (float)ix + 0.5f, pcy = (float)iy + 0.5f;
            PixelFw st;
            pixel_fw(c, 1.f, -1.f, 1.f, pcx, pcy, W, H, d.sigma_scale, st);
            pixel_bw(st, c, 1.f, tgt8 ? (float)tgt8[pix] : tgt[pix], d.inv_px, W, H,
                     d.sigma_scale, g);
        }
        if (__any(hit)) {
            // the group's first lane adds the samples in order
#pragma unroll
            for (int q = 0; q < kSampleLanes; q++) {
#pragma unroll
                for (int k = 0; k < 3; k++) {
                    const float gx = __shfl(g[k].x, gbase + q);
                    const float gy = __shfl(g[k].y, gbase + q);
                    const float gz = __shfl(g[k].z, gbase + q);
                    const float gw = __shfl(g[k].w, gbase + q);
                    acc[k].x += gx;
                    acc[k].y += gy;
                    acc[k].z += gz;
                    acc[k].w += gw;
                }
            }
        }
    }
    if (j == 0) {
        d.rimf[item] = 0;
        float4* dst = d.gtri + (size_t)view * 3 * d.g.n_faces;
#pragma unroll
        for (int k = 0; k < 3; k++) {
            dst[(size_t)k * d.g.n_faces + f] = acc[k];
        }
    }
}

__global__ __launch_bounds__(256) void k_hsr_face_bwd(HsrDev d) {
    __shared__ uint32_t queue[256];
    __shared__ uint32_t wave_n[4];
    const uint32_t gi = blockIdx.x * blockDim.x + threadIdx.x;
    publish_t_next(d, gi);
    // the raster is done with this iteration's bins: clear their counters
    for (uint32_t b = gi; b < d.bins.n_bins; b += gridDim.x * blockDim.x) {
        const uint32_t c = d.bins.counts[b];
        if (c > d.bins.cap && d.bin_over_max) {
            atomicMax(d.bin_over_max, c);  // rare: the host grows the bins before the next step
        }
        d.bins.counts[b] = 0;
    }
    if (d.heavy.count && gi < kHeavySegs) {
        d.heavy.count[gi] = 0;
    }
    const uint32_t F = d.g.n_faces;
    const bool valid = gi < d.g.n_views * F;
    const bool rim = valid && d.rimf[gi] != 0;
    if (valid && !rim) {
        const uint32_t view = gi / F, f = gi - view * F;
        float4* dst = d.gtri + (size_t)view * 3 * F;
#pragma unroll
        for (int k = 0; k < 3; k++) {
            dst[(size_t)k * F + f] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    // the workgroup's rim faces, in item order
    const uint32_t lane = threadIdx.x & 63u, wv = threadIdx.x >> 6;
    const uint64_t m = __ballot(rim);
    if (lane == 0) {
        wave_n[wv] = (uint32_t)__popcll(m);
    }
    __syncthreads();
    uint32_t before = 0, n = 0;
    for (uint32_t w = 0; w < blockDim.x / 64; w++) {
        before += w < wv ? wave_n[w] : 0u;
        n += wave_n[w];
    }
    if (rim) {
        queue[before + lanes_below(m)] = gi;
    }
    __syncthreads();
    const int j = (int)(threadIdx.x % kSampleLanes);
    const int gbase = (int)lane - j;
    for (uint32_t qi = threadIdx.x / kSampleLanes; qi < n; qi += blockDim.x / kSampleLanes) {
        face_bwd_item(d, queue[qi], j, gbase);
    }
}

// The same with a group of kSampleLanes lanes for every (view, face), rim
// or not (each group reads its face's flag): the form for small problems,
// whose few workgroups would otherwise take their queued faces in turn.
__device__ __forceinline__ void face_bwd_all_block(const HsrDev& d, uint32_t blk,
                                                   uint32_t n_blk) {
    const uint32_t gi = blk * blockDim.x + threadIdx.x;
    publish_t_next(d, gi);
    // the raster is done with this iteration's bins: clear their counters
    for (uint32_t b = gi; b < d.bins.n_bins; b += n_blk * blockDim.x) {
        const uint32_t c = d.bins.counts[b];
        if (c > d.bins.cap && d.bin_over_max) {
            atomicMax(d.bin_over_max, c);  // rare: the host grows the bins before the next step
        }
        d.bins.counts[b] = 0;
    }
    if (d.heavy.count && gi < kHeavySegs) {
        d.heavy.count[gi] = 0;
    }
    const uint32_t item = gi / kSampleLanes;
    const uint32_t F = d.g.n_faces;
    if (item >= d.g.n_views * F) {
        return;  // the whole group
    }
    const int j = (int)(threadIdx.x % kSampleLanes);
    const int gbase = (int)(threadIdx.x & 63u) - j;
    if (d.rimf[item] != 0) {
        face_bwd_item(d, item, j, gbase);
    } else if (j == 0) {
        const uint32_t view = item / F, f = item - view * F;
        float4* dst = d.gtri + (size_t)view * 3 * F;
#pragma unroll
        for (int k = 0; k < 3; k++) {
            dst[(size_t)k * F + f] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
}

__global__ __launch_bounds__(256) void k_hsr_face_bwd_all(HsrDev d) {
    face_bwd_all_block(d, blockIdx.x, gridDim.x);
}

// Small problems: the loss (one pixel per lane) and the group-per-face
// backward in one launch -- they read the raster's output and write disjoint
// buffers -- the first n_loss workgroups taking the loss's blocks, the rest
// the backward's (one kernel boundary less in a latency-bound iteration).
template <int NV>
__global__ __launch_bounds__(256) void k_hsr_loss_face_bwd(HsrDev d, uint32_t loss_gx,
                                                           uint32_t n_loss) {
    if (blockIdx.x < n_loss) {
        loss_block<NV, 1>(d, blockIdx.x % loss_gx, blockIdx.x / loss_gx);
    } else {
        face_bwd_all_block(d, blockIdx.x - n_loss, gridDim.x - n_loss);
    }
}

// LookupFacesBwd x3 + clip->pos chain over all views + Adam: one lane per
// (vertex, view) gathers that view's corner gradients (the adjacency rows of
// a batch of kDegBatch slots loaded together, then their gradients), the
// vertex's first lane sums the views and steps Adam. The last workgroup to
// finish advances t (all reads of t precede every workgroup's arrival on the
// counter).
template <int NV>
__global__ __launch_bounds__(256) void k_hsr_vertex_adam(HsrDev d) {
    publish_bin_over(d);
    vertex_views_adam<NV>(d, [&](uint32_t vtx, uint32_t view, float (&g4)[4]) {
        const float4* gt = d.gtri + (size_t)view * 3 * d.g.n_faces;
        float lfb[3][4];
#pragma unroll
        for (int k = 0; k < 3; k++) {
            lfb[k][0] = lfb[k][1] = lfb[k][2] = lfb[k][3] = 0.f;
        }
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
#pragma unroll
            for (int i = 0; i < kDegBatch; i++) {
                if (ab.f[i] < 0) {
                    continue;
                }
                const int k0 = first_corner(ab.mask[i]);
#pragma unroll
                for (int k = 0; k < 3; k++) {
                    if (ab.mask[i] & (1u << k)) {
                        // a face holding the vertex at two corners (degenerate)
                        // reloads the other corner's gradient
                        const float4 g = k == k0 ? gg[i] : gt[(size_t)k * d.g.n_faces + ab.f[i]];
                        lfb[k][0] += g.x;
                        lfb[k][1] += g.y;
                        lfb[k][2] += g.z;
                        lfb[k][3] += g.w;
                    }
                }
            }
        }
        // clip_v gradient: LookupFaces 2, 1, 0 (newest first), one 3-ary sum
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float acc = 0.f;
            acc += lfb[2][r];
            acc += lfb[1][r];
            acc += lfb[0][r];
            g4[r] = acc;
        }
    });
}

// Per-op kernels ------------------------------------------------------------

// The per-op kernels below take a batch on the grid's y dimension: item
// blockIdx.y reads and writes at the given per-item strides (in elements; a
// stride of 0 shares the buffer among the items).
__global__ void k_lookup_faces(const float* attr, uint32_t n_comp, const float* faces,
                               uint32_t n_faces, uint32_t n_attr, uint32_t corner, uint32_t* err,
                               float* out, size_t attr_stride) {
    const uint32_t f = blockIdx.x * blockDim.x + threadIdx.x;
    if (f >= n_faces) {
        return;
    }
    attr += blockIdx.y * attr_stride;
    out += (size_t)blockIdx.y * n_faces * n_comp;
    const uint32_t vi = fid_u(faces[(size_t)f * 3 + corner]);
    if (vi >= n_attr) {
        atomicOr(err, 32u);
        return;
    }
    for (uint32_t c = 0; c < n_comp; c++) {
        out[(size_t)f * n_comp + c] = attr[(size_t)vi * n_comp + c];
    }
}

__global__ void k_lookup_faces_bwd(const float* gy, uint32_t n_comp, const float* faces,
                                   uint32_t n_faces, const float* vtx_faces, uint32_t n_verts,
                                   uint32_t max_deg, uint32_t corner, uint32_t* err,
                                   float* out) {
    const uint32_t v = blockIdx.x * blockDim.x + threadIdx.x;
    if (v >= n_verts) {
        return;
    }
    gy += (size_t)blockIdx.y * n_faces * n_comp;
    out += (size_t)blockIdx.y * n_verts * n_comp;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t dd = 0; dd < max_deg; dd++) {
        const float fv = vtx_faces[(size_t)dd * n_verts + v];
        if (fv < -0.5f) {
            continue;
        }
        const uint32_t f = fid_u(fv);
        if (f >= n_faces) {
            atomicOr(err, 64u);
            continue;
        }
        if (fid_u(faces[(size_t)f * 3 + corner]) != v) {
            continue;
        }
        for (uint32_t c = 0; c < n_comp; c++) {
            acc[c] += gy[(size_t)f * n_comp + c];
        }
    }
    for (uint32_t c = 0; c < n_comp; c++) {
        out[(size_t)v * n_comp + c] = acc[c];
    }
}

__global__ void k_face_fetch(const float* attr, uint32_t n_comp, uint32_t n_faces,
                             const float* idx, size_t npx, float* out, size_t attr_stride) {
    const size_t p = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= npx) {
        return;
    }
    attr += blockIdx.y * attr_stride;
    idx += blockIdx.y * npx;
    out += blockIdx.y * npx * n_comp;
    const int f = (int)(idx[p] + 0.5f) - 1;
    const bool ok = f >= 0 && (uint32_t)f < n_faces;
    for (uint32_t c = 0; c < n_comp; c++) {
        out[p * n_comp + c] = ok ? attr[(size_t)f * n_comp + c] : 0.f;
    }
}

__global__ void k_face_fetch_bwd(const float* gy, uint32_t n_comp, const float* idx, uint32_t w,
                                 uint32_t h, const float4* prj0, const float4* prj1,
                                 const float4* prj2, uint32_t n_faces, const float* seed,
                                 float radius, uint32_t n_samples, float* out, size_t prj_stride) {
    const uint32_t f = blockIdx.x * blockDim.x + threadIdx.x;
    if (f >= n_faces) {
        return;
    }
    const size_t npx = (size_t)w * h;
    gy += blockIdx.y * npx * n_comp;
    idx += blockIdx.y * npx;
    prj0 += blockIdx.y * prj_stride;
    prj1 += blockIdx.y * prj_stride;
    prj2 += blockIdx.y * prj_stride;
    seed += blockIdx.y;
    out += (size_t)blockIdx.y * n_faces * n_comp;
    const float4 c[3] = {prj0[f], prj1[f], prj2[f]};
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    bool ok = c[0].w > 1e-6f && c[1].w > 1e-6f && c[2].w > 1e-6f;
    if (ok) {
        float s[3][2];
        for (int k = 0; k < 3; k++) {
            s[k][0] = (c[k].x / c[k].w * 0.5f + 0.5f) * (float)w;
            s[k][1] = (c[k].y / c[k].w * 0.5f + 0.5f) * (float)h;
        }
        if (n_samples == 0) {
            int x0 = (int)floorf(smin(smin(s[0][0], s[1][0]), s[2][0]) - 1.f);
            int x1 = (int)ceilf(smax(smax(s[0][0], s[1][0]), s[2][0]) + 1.f);
            int y0 = (int)floorf(smin(smin(s[0][1], s[1][1]), s[2][1]) - 1.f);
            int y1 = (int)ceilf(smax(smax(s[0][1], s[1][1]), s[2][1]) + 1.f);
            x0 = x0 > 0 ? x0 : 0;
            y0 = y0 > 0 ? y0 : 0;
            x1 = x1 < (int)w - 1 ? x1 : (int)w - 1;
            y1 = y1 < (int)h - 1 ? y1 : (int)h - 1;
            for (int iy = y0; iy <= y1; iy++) {
                for (int ix = x0; ix <= x1; ix++) {
                    const size_t p = (size_t)iy * w + ix;
                    if (fid_u(idx[p]) != f + 1) {
                        continue;
                    }
                    for (uint32_t q = 0; q < n_comp; q++) {
                        acc[q] += gy[p * n_comp + q];
                    }
                }
            }
        } else {
            const uint32_t seed_u = (uint32_t)(int64_t)(*seed + 0.5f);
            for (uint32_t smp = 0; smp < n_samples; smp++) {
                const int e = (int)(smp % 3);
                const float* a = s[e];
                const float* b = s[(e + 1) % 3];
                const float ex = b[0] - a[0];
                const float ey = b[1] - a[1];
                const float len = sqrtf(ex * ex + ey * ey);
                if (len < 1e-6f) {
                    continue;
                }
                const float u = hash_to_unit(f, smp, seed_u, 0);
                const float off = (hash_to_unit(f, smp, seed_u, 1) * 2.f - 1.f) * radius;
                const float spx = a[0] + u * ex - off * (ey / len);
                const float spy = a[1] + u * ey + off * (ex / len);
                const int ix = (int)floorf(spx);
                const int iy = (int)floorf(spy);
                if (ix < 0 || iy < 0 || ix >= (int)w || iy >= (int)h) {
                    continue;
                }
                const size_t p = (size_t)iy * w + ix;
                if (fid_u(idx[p]) != f + 1) {
                    continue;
                }
                for (uint32_t q = 0; q < n_comp; q++) {
                    acc[q] += gy[p * n_comp + q];
                }
            }
        }
    }
    for (uint32_t q = 0; q < n_comp; q++) {
        out[(size_t)f * n_comp + q] = acc[q];
    }
}

}  // namespace dressi

// ---------------------------------------------------------------------------
// The plan
// ---------------------------------------------------------------------------
using namespace dressi;

struct dressi_hsr_plan {
    dressi_ctx* ctx = nullptr;
    dressi_hsr_desc desc{};
    HsrDev d{};
    std::vector<void*> allocs;
    void* bin_mem = nullptr;     // the soft bins (resized by grow_bins)
    uint32_t* over_host = nullptr;  // host-mapped: d.bin_over
    uint8_t* tgt_bytes = nullptr;   // HardSoftRas: d.tgt8 when the targets are all 0 / 1
    uint32_t* nonbinary = nullptr;  // set by k_target_bytes on a target other than 0 / 1
    bool mesh_set = false, targets_set = false, state_set = false;
    hipGraph_t graph = nullptr;  // one iteration
    hipGraphExec_t exec = nullptr;
    hipGraph_t graph_batch = nullptr;  // kGraphBatch iterations back to back
    hipGraphExec_t exec_batch = nullptr;
    hipStream_t graph_stream = nullptr;  // stream the execs were instantiated for
};

namespace {

template <typename T>
int plan_alloc(dressi_hsr_plan* p, T** out, size_t count) {
    void* ptr = nullptr;
    DRESSI_TRY_HIP(hipMalloc(&ptr, sizeof(T) * (count ? count : 1)));
    p->allocs.push_back(ptr);
    *out = (T*)ptr;
    return DRESSI_OK;
}

// Byte copy of the targets for the loss and face backward: out[i] = t[i]
// (0 or 1); any other bit pattern (-0, fractions, NaN) sets *nonbinary and
// the plan keeps reading the float targets.
__global__ __launch_bounds__(256) void k_target_bytes(const float* t, size_t n, uint8_t* out,
                                                      uint32_t* nonbinary) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) {
        return;
    }
    const uint32_t u = __float_as_uint(t[i]);
    out[i] = u == 0x3f800000u ? 1u : 0u;
    if (u != 0u && u != 0x3f800000u) {
        *nonbinary = 1u;
    }
}

// Iterations per replay of the batched graph (dressi_hsr_step launches it
// for every full batch of its count: fewer launch gaps between iterations).
constexpr uint32_t kGraphBatch = 8;

// Kernel k of one iteration: 0 setup + binning, 1 visibility raster,
// 2 pred + loss, 3 face backward, 4 vertex backward + Adam.
constexpr int kIterKernels = 5;
const char* const kIterKernelNames[kIterKernels] = {"k_hsr_setup", "k_hsr_raster", "k_hsr_loss",
                                                    "k_hsr_face_bwd", "k_hsr_vertex_adam"};

// Screen pixels from which the captured graph runs the loss on a branch.
constexpr uint64_t kForkLossMinPixels = 1ull << 20;

// The loss takes four pixels per lane where its grid still fills the chip.
bool loss_vec(const RasterGeom& g) {
    return g.width % 4 == 0 && (size_t)div_up(g.width, 256) * div_up(g.height, 4) >= 2048;
}

// Small problems run the loss and the face backward as one launch (kernel 2;
// kernel 3 is then empty). Measured at 512 x 512 x 4 views.
bool fused_loss_bwd(const RasterGeom& g) {
    return !loss_vec(g) && g.n_views * g.n_faces <= kFaceBwdQueueMin &&
           (uint64_t)g.width * g.height < kForkLossMinPixels;
}

int launch_iter_kernel(const HsrDev& d, hipStream_t s, int k) {
    if (d.technique == 1) {
        return launch_aa_kernel(d, s, k);
    }
    const RasterGeom& g = d.g;
    const uint32_t nvf = g.n_views * g.n_faces;
    const bool fused = fused_loss_bwd(g);
    switch (k) {
        case 0:
            hipLaunchKernelGGL(k_hsr_setup, dim3(div_up(nvf, 256)), dim3(256), 0, s, d);
            break;
        case 1:
            hipLaunchKernelGGL(k_hsr_raster,
                               dim3(4u * kHeavySegs * d.heavy.cap + block_grid(g) * g.n_views),
                               dim3(64), 0, s, d);
            break;
        case 2: {
            const bool vec = loss_vec(g);
            const dim3 grid(div_up(g.width, vec ? 256 : 64), div_up(g.height, 4));
            const uint32_t n_loss = grid.x * grid.y;
            const uint32_t n_bwd = div_up(nvf, 256 / kSampleLanes);
            switch (g.n_views) {
#define DRESSI_NV(N)                                                                          \
    case N:                                                                                   \
        if (fused) {                                                                          \
            hipLaunchKernelGGL((k_hsr_loss_face_bwd<N>), dim3(n_loss + n_bwd), dim3(256), 0,  \
                               s, d, grid.x, n_loss);                                         \
        } else if (vec) {                                                                     \
            hipLaunchKernelGGL((k_hsr_loss<N, 4>), grid, dim3(256), 0, s, d);                 \
        } else {                                                                              \
            hipLaunchKernelGGL((k_hsr_loss<N, 1>), grid, dim3(256), 0, s, d);                 \
        }                                                                                     \
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
        case 3:
            if (fused) {
                return DRESSI_OK;  // ran with the loss
            }
            if (nvf > kFaceBwdQueueMin) {
                hipLaunchKernelGGL(k_hsr_face_bwd, dim3(div_up(nvf, 256)), dim3(256), 0, s, d);
            } else {
                hipLaunchKernelGGL(k_hsr_face_bwd_all, dim3(div_up(nvf, 256 / kSampleLanes)),
                                   dim3(256), 0, s, d);
            }
            break;
        default:
            switch (g.n_views) {
#define DRESSI_NV(N)                                                                          \
    case N:                                                                                   \
        hipLaunchKernelGGL(k_hsr_vertex_adam<N>, dim3(vertex_grid<N>(d.n_verts)), dim3(256),  \
                           0, s, d);                                                          \
        break;
                DRESSI_NV(1) DRESSI_NV(2) DRESSI_NV(3) DRESSI_NV(4)
                DRESSI_NV(5) DRESSI_NV(6) DRESSI_NV(7) DRESSI_NV(8)
#undef DRESSI_NV
            }
            break;
    }
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int enqueue_iteration(dressi_hsr_plan* p, hipStream_t s) {
    for (int k = 0; k < kIterKernels; k++) {
        if (int rc = launch_iter_kernel(p->d, s, k)) return rc;
    }
    return DRESSI_OK;
}

// `reps` iterations for graph capture on `s`, the loss of each on `side`
// (HardSoftRas: the loss reads the face ids, targets and the setup's screen
// corners and writes only pred and the loss image, which the face backward,
// the vertex kernel and the next setup never read): it overlaps the face
// backward, the vertex kernel and the next setup, and joins before the next
// raster rewrites the face ids, and at the end. `ev` holds 2 * reps events.
int enqueue_iterations_forked(dressi_hsr_plan* p, hipStream_t s, hipStream_t side,
                              uint32_t reps, hipEvent_t* ev) {
    hipEvent_t joined = nullptr;
    for (uint32_t r = 0; r < reps; r++) {
        if (int rc = launch_iter_kernel(p->d, s, 0)) return rc;  // setup
        if (joined) DRESSI_TRY_HIP(hipStreamWaitEvent(s, joined, 0));
        if (int rc = launch_iter_kernel(p->d, s, 1)) return rc;  // raster
        DRESSI_TRY_HIP(hipEventRecord(ev[2 * r], s));
        DRESSI_TRY_HIP(hipStreamWaitEvent(side, ev[2 * r], 0));
        if (int rc = launch_iter_kernel(p->d, side, 2)) return rc;  // loss
        DRESSI_TRY_HIP(hipEventRecord(ev[2 * r + 1], side));
        joined = ev[2 * r + 1];
        for (int k = 3; k < kIterKernels; k++) {
            if (int rc = launch_iter_kernel(p->d, s, k)) return rc;
        }
    }
    if (joined) DRESSI_TRY_HIP(hipStreamWaitEvent(s, joined, 0));
    return DRESSI_OK;
}

int ready(dressi_hsr_plan* p) {
    DRESSI_REQUIRE(p, "NULL plan");
    DRESSI_REQUIRE(p->mesh_set, "dressi_hsr_set_mesh() must be called before stepping");
    DRESSI_REQUIRE(p->targets_set, "targets must be set (set_targets / render_targets)");
    DRESSI_REQUIRE(p->state_set, "dressi_hsr_set_state() must be called before stepping");
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    return DRESSI_OK;
}

void drop_graph(dressi_hsr_plan* p) {
    for (hipGraphExec_t* e : {&p->exec, &p->exec_batch}) {
        if (*e) {
            hipGraphExecDestroy(*e);
            *e = nullptr;
        }
    }
    for (hipGraph_t* g : {&p->graph, &p->graph_batch}) {
        if (*g) {
            hipGraphDestroy(*g);
            *g = nullptr;
        }
    }
}

// A bin overflowed in an earlier iteration (its raster walked every face of
// the view: exact but slow): the bins grow to the next power of two that
// holds the reported count (at most kSoftBinCapMax entries), so the
// following iterations walk lists again. The report is read without waiting
// for the stream; a grow waits for it before swapping the memory.
int grow_bins(dressi_hsr_plan* p) {
    if (!p->over_host) {
        return DRESSI_OK;
    }
    const uint32_t need = __atomic_load_n(p->over_host, __ATOMIC_ACQUIRE);
    if (need <= p->d.bins.cap || p->d.bins.cap >= kSoftBinCapMax) {
        return DRESSI_OK;
    }
    uint32_t cap = p->d.bins.cap;
    while (cap < need && cap < kSoftBinCapMax) {
        cap *= 2;
    }
    hipStream_t s = p->ctx->stream;
    DRESSI_TRY_HIP(hipStreamSynchronize(s));
    const uint32_t n_bins = p->d.bins.n_bins;
    const size_t bytes = fixed_bin_bytes(n_bins, cap);
    void* mem = nullptr;
    if (hipMalloc(&mem, bytes) != hipSuccess) {
        // keep the current bins (overflowed bins stay exact, walking every face)
        (void)hipGetLastError();
        *p->over_host = 0;
        return DRESSI_OK;
    }
    DRESSI_TRY_HIP(hipMemsetAsync(mem, 0, sizeof(uint32_t) * n_bins, s));
    DRESSI_TRY_HIP(hipStreamSynchronize(s));
    DRESSI_TRY_HIP(hipFree(p->bin_mem));
    p->bin_mem = mem;
    fixed_bin_carve(mem, n_bins, cap, &p->d.bins);
    __atomic_store_n(p->over_host, 0u, __ATOMIC_RELEASE);
    drop_graph(p);  // the graphs hold the old bins
    return DRESSI_OK;
}

// After the targets change (HardSoftRas): the byte copy and d.tgt8, which
// is null unless every target is exactly 0 or 1. The captured graphs hold
// d by value, so a change of d.tgt8 drops them.
int refresh_target_bytes(dressi_hsr_plan* p) {
    if (!p->tgt_bytes) {
        return DRESSI_OK;
    }
    hipStream_t s = p->ctx->stream;
    const size_t n = (size_t)p->desc.n_views * p->desc.width * p->desc.height;
    DRESSI_TRY_HIP(hipMemsetAsync(p->nonbinary, 0, sizeof(uint32_t), s));
    hipLaunchKernelGGL(k_target_bytes, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                       p->d.targets, n, p->tgt_bytes, p->nonbinary);
    DRESSI_TRY_HIP(hipGetLastError());
    uint32_t nonbinary = 1;
    DRESSI_TRY_HIP(hipMemcpyAsync(&nonbinary, p->nonbinary, sizeof(uint32_t),
                                  hipMemcpyDeviceToHost, s));
    DRESSI_TRY_HIP(hipStreamSynchronize(s));
    const uint8_t* t8 = nonbinary ? nullptr : p->tgt_bytes;
    if (t8 != p->d.tgt8) {
        p->d.tgt8 = t8;
        drop_graph(p);
    }
    return DRESSI_OK;
}

}  // namespace

extern "C" {

int dressi_hsr_create(dressi_ctx* ctx, const dressi_hsr_desc* desc, dressi_hsr_plan** out) {
    DRESSI_REQUIRE(ctx && desc && out, "bad arguments");
    DRESSI_REQUIRE(desc->n_verts > 0 && desc->n_faces > 0, "empty mesh");
    DRESSI_REQUIRE(desc->n_views >= 1 && desc->n_views <= kMaxViews,
                   "n_views must be in [1, %u]", kMaxViews);
    DRESSI_REQUIRE(desc->width > 0 && desc->height > 0, "empty screen");
    DRESSI_REQUIRE(desc->radius_px > 0.f, "radius_px must be > 0");
    DRESSI_REQUIRE((uint64_t)desc->n_views * desc->n_faces < (1ull << 31), "too many faces");
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    dressi_hsr_plan* p = new dressi_hsr_plan();
    p->ctx = ctx;
    p->desc = *desc;
    HsrDev& d = p->d;
    d.g = make_geom(desc->width, desc->height, desc->n_views, desc->n_faces);
    d.n_verts = desc->n_verts;
    d.n_samples = desc->n_samples;
    d.flags = desc->flags;
    d.radius = desc->radius_px;
    d.sigma_scale = 7.f / desc->radius_px;
    d.inv_px = 1.f / (float)(desc->width * desc->height);
    d.lr = desc->lr;
    d.b1 = desc->beta1;
    d.b2 = desc->beta2;
    d.eps = desc->eps;
    const size_t V = desc->n_verts, F = desc->n_faces, N = desc->n_views;
    const size_t npx = (size_t)desc->width * desc->height;
    int rc = DRESSI_OK;
    float4* gtri = nullptr;
    rc = rc ? rc : plan_alloc(p, &d.pos, V * 3);
    rc = rc ? rc : plan_alloc(p, &d.m, V * 3);
    rc = rc ? rc : plan_alloc(p, &d.v, V * 3);
    rc = rc ? rc : plan_alloc(p, &d.t, 1);
    rc = rc ? rc : plan_alloc(p, &d.t_next, 1);
    rc = rc ? rc : plan_alloc(p, (float**)&d.mvps, N * 16);
    rc = rc ? rc : plan_alloc(p, (float**)&d.targets, N * npx);
    d.technique = (desc->flags & DRESSI_HSR_TECHNIQUE_AA) ? 1u : 0u;
    if (d.technique == 0) {
        rc = rc ? rc : plan_alloc(p, &d.recs, N * F);
        rc = rc ? rc : plan_alloc(p, &d.cull, N * F);
        rc = rc ? rc : plan_alloc(p, &d.fscr, N * F * 2);
        rc = rc ? rc : plan_alloc(p, &d.rimf, N * F);
        rc = rc ? rc : plan_alloc(p, &p->tgt_bytes, N * npx);
        rc = rc ? rc : plan_alloc(p, &p->nonbinary, 1);
        d.heavy.cap = heavy_seg_cap(d.g.n_tiles * d.g.n_views);
        d.heavy.min_count = heavy_min_count(d.g.n_tiles * d.g.n_views);
        rc = rc ? rc : plan_alloc(p, &d.heavy.count, kHeavySegs);
        rc = rc ? rc : plan_alloc(p, &d.heavy.list, kHeavyCap);
        rc = rc ? rc : plan_alloc(p, &d.heavy.slot, (size_t)N * d.g.n_tiles);
    } else {
        rc = rc ? rc : plan_alloc(p, &d.arecs, N * F);
        rc = rc ? rc : plan_alloc(p, &d.aa_list, N * F);
        rc = rc ? rc : plan_alloc(p, &d.gflag, (size_t)N * d.g.height * div_up(d.g.width, 256));
        rc = rc ? rc : plan_alloc(p, &d.aa_count, 1);
        rc = rc ? rc : plan_alloc(p, &d.clip, N * V);
    }
    rc = rc ? rc : plan_alloc(p, &d.ids, N * npx);
    rc = rc ? rc : plan_alloc(p, &d.loss, npx);
    rc = rc ? rc : plan_alloc(p, &gtri, N * 3 * F);
    if (!rc && ((desc->flags & DRESSI_HSR_KEEP_PRED) || d.technique == 1)) {
        rc = plan_alloc(p, &d.pred, N * npx);
    }
    if (!rc && (desc->flags & DRESSI_HSR_KEEP_GRAD)) rc = plan_alloc(p, &d.grad, V * 3);
    d.gtri = gtri;
    float2* bc = nullptr;
    if (!rc) rc = plan_alloc(p, &bc, kBiasTableLen);
    if (!rc) {
        std::vector<float2> tab(kBiasTableLen);
        for (uint32_t i = 0; i < kBiasTableLen; i++) {
            const float tn = (float)(i + 1);
            tab[i] = make_float2(1.f - powf(desc->beta1, tn), 1.f - powf(desc->beta2, tn));
        }
        hipError_t e = hipMemcpy(bc, tab.data(), sizeof(float2) * kBiasTableLen,
                                 hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            set_error("bias table upload failed: %s", hipGetErrorString(e));
            rc = DRESSI_ERR_HIP;
        }
        d.bc_tab = bc;
        d.bc_len = kBiasTableLen;
    }
    if (!rc) {
        const size_t bytes = fixed_bin_bytes(d.g.n_tiles * d.g.n_views, kSoftBinCap);
        if (hipMalloc(&p->bin_mem, bytes) != hipSuccess) {
            p->bin_mem = nullptr;
            set_error("out of device memory for the bins (%zu bytes)", bytes);
            rc = DRESSI_ERR_HIP;
        } else {
            fixed_bin_carve(p->bin_mem, d.g.n_tiles * d.g.n_views, kSoftBinCap, &d.bins);
        }
    }
    if (!rc) {
        // host-mapped overflow report (see grow_bins)
        void* h = nullptr;
        void* dp = nullptr;
        if (hipHostMalloc(&h, sizeof(uint32_t), hipHostMallocMapped) != hipSuccess ||
            hipHostGetDevicePointer(&dp, h, 0) != hipSuccess) {
            if (h) hipHostFree(h);
            set_error("hipHostMalloc failed for the bin overflow report");
            rc = DRESSI_ERR_HIP;
        } else {
            p->over_host = (uint32_t*)h;
            *p->over_host = 0;
            d.bin_over = (uint32_t*)dp;
        }
    }
    if (!rc) {
        uint32_t* mx = nullptr;
        rc = plan_alloc(p, &mx, 1);
        if (!rc && hipMemset(mx, 0, sizeof(uint32_t)) != hipSuccess) {
            set_error("bin overflow word init failed");
            rc = DRESSI_ERR_HIP;
        }
        d.bin_over_max = mx;
    }
    if (!rc) {
        hipError_t e = hipMemsetAsync(d.bins.counts, 0, sizeof(uint32_t) * d.bins.n_bins, ctx->stream);
        if (e == hipSuccess && d.heavy.count) {
            e = hipMemsetAsync(d.heavy.count, 0, sizeof(uint32_t) * kHeavySegs, ctx->stream);
        }
        if (e == hipSuccess && d.rimf) {
            e = hipMemsetAsync(d.rimf, 0, N * F, ctx->stream);
        }
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) {
            set_error("plan init failed: %s", hipGetErrorString(e));
            rc = DRESSI_ERR_HIP;
        }
    }
    if (rc) {
        dressi_hsr_destroy(p);
        return rc;
    }
    *out = p;
    return DRESSI_OK;
}

int dressi_hsr_destroy(dressi_hsr_plan* p) {
    if (!p) {
        return DRESSI_OK;
    }
    hipSetDevice(p->ctx->device);
    hipStreamSynchronize(p->ctx->stream);
    drop_graph(p);
    for (void* a : p->allocs) {
        hipFree(a);
    }
    if (p->bin_mem) {
        hipFree(p->bin_mem);
    }
    if (p->over_host) {
        hipHostFree(p->over_host);
    }
    delete p;
    return DRESSI_OK;
}

int dressi_hsr_set_mesh(dressi_hsr_plan* p, const float* faces, const float* mvps) {
    DRESSI_REQUIRE(p && faces && mvps, "bad arguments");
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    const uint32_t V = p->desc.n_verts, F = p->desc.n_faces;
    std::vector<int32_t> fi((size_t)F * 3);
    for (size_t i = 0; i < fi.size(); i++) {
        const float x = faces[i];
        DRESSI_REQUIRE(x >= 0.f && x < (float)V, "face index out of range at %zu", i);
        fi[i] = (int32_t)(uint32_t)(int64_t)(x + 0.5f);
    }
    // vertex -> incident faces (src/core/mesh_utils.cpp:53-71) plus a per-slot
    // corner mask: bit k set when faces[f][k] == v (LookupFacesBwd's test)
    std::vector<std::vector<uint32_t>> vf(V);
    for (uint32_t f = 0; f < F; f++) {
        for (int k = 0; k < 3; k++) {
            vf[fi[f * 3 + k]].push_back(f);
        }
    }
    uint32_t deg = 1;
    for (const auto& l : vf) {
        deg = l.size() > deg ? (uint32_t)l.size() : deg;
    }
    std::vector<int32_t> vft((size_t)deg * V, -1);
    std::vector<uint8_t> vfm((size_t)deg * V, 0);
    for (uint32_t v = 0; v < V; v++) {
        for (size_t dd = 0; dd < vf[v].size(); dd++) {
            const uint32_t f = vf[v][dd];
            vft[dd * V + v] = (int32_t)f;
            uint8_t m = 0;
            for (int k = 0; k < 3; k++) {
                m |= (uint32_t)fi[f * 3 + k] == v ? (uint8_t)(1u << k) : 0;
            }
            vfm[dd * V + v] = m;
        }
    }
    hipStream_t s = p->ctx->stream;
    int32_t* dfaces = nullptr;
    int32_t* dvf = nullptr;
    uint8_t* dvfm = nullptr;
    if (!p->mesh_set) {
        if (int rc = plan_alloc(p, &dfaces, fi.size())) return rc;
        if (int rc = plan_alloc(p, &dvf, vft.size())) return rc;
        if (int rc = plan_alloc(p, &dvfm, vfm.size())) return rc;
        p->d.faces = dfaces;
        p->d.vf = dvf;
        p->d.vf_mask = dvfm;
        p->d.max_deg = deg;
    } else {
        DRESSI_REQUIRE(deg == p->d.max_deg, "topology change needs a new plan");
    }
    DRESSI_TRY_HIP(hipMemcpyAsync((void*)p->d.faces, fi.data(), fi.size() * 4, hipMemcpyHostToDevice, s));
    DRESSI_TRY_HIP(hipMemcpyAsync((void*)p->d.vf, vft.data(), vft.size() * 4, hipMemcpyHostToDevice, s));
    DRESSI_TRY_HIP(hipMemcpyAsync((void*)p->d.vf_mask, vfm.data(), vfm.size(), hipMemcpyHostToDevice, s));
    DRESSI_TRY_HIP(hipMemcpyAsync((void*)p->d.mvps, mvps, sizeof(float) * 16 * p->desc.n_views,
                                  hipMemcpyHostToDevice, s));
    DRESSI_TRY_HIP(hipStreamSynchronize(s));
    p->mesh_set = true;
    drop_graph(p);
    return DRESSI_OK;
}

int dressi_hsr_set_targets(dressi_hsr_plan* p, const float* targets) {
    DRESSI_REQUIRE(p && targets, "bad arguments");
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    const size_t n = (size_t)p->desc.n_views * p->desc.width * p->desc.height;
    DRESSI_TRY_HIP(hipMemcpyAsync((void*)p->d.targets, targets, n * 4, hipMemcpyHostToDevice,
                                  p->ctx->stream));
    DRESSI_TRY_HIP(hipStreamSynchronize(p->ctx->stream));
    if (int rc = refresh_target_bytes(p)) return rc;
    p->targets_set = true;
    return DRESSI_OK;
}

int dressi_hsr_render_targets(dressi_hsr_plan* p, const float* tgt_pos, uint32_t n_tverts,
                              const float* tgt_faces, uint32_t n_tfaces) {
    DRESSI_REQUIRE(p && tgt_pos && tgt_faces && n_tverts > 0 && n_tfaces > 0, "bad arguments");
    DRESSI_REQUIRE(p->mesh_set, "dressi_hsr_set_mesh() first (the MVPs)");
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    const uint32_t N = p->desc.n_views;
    std::vector<int32_t> fi((size_t)n_tfaces * 3);
    for (size_t i = 0; i < fi.size(); i++) {
        DRESSI_REQUIRE(tgt_faces[i] >= 0.f && tgt_faces[i] < (float)n_tverts,
                       "target face index out of range at %zu", i);
        fi[i] = (int32_t)(uint32_t)(int64_t)tgt_faces[i];
    }
    // target clips on the host: TransformToClip (asset_utils.cpp:768-782)
    std::vector<float> mv((size_t)N * 16);
    DRESSI_TRY_HIP(hipMemcpy(mv.data(), p->d.mvps, mv.size() * 4, hipMemcpyDeviceToHost));
    std::vector<float> clip((size_t)N * n_tverts * 4);
    for (uint32_t v = 0; v < N; v++) {
        for (uint32_t i = 0; i < n_tverts; i++) {
            const float4 c = mvp_transform(&mv[v * 16], tgt_pos[i * 3], tgt_pos[i * 3 + 1],
                                           tgt_pos[i * 3 + 2]);
            float* o = &clip[((size_t)v * n_tverts + i) * 4];
            o[0] = c.x;
            o[1] = c.y;
            o[2] = c.z;
            o[3] = c.w;
        }
    }
    if (p->d.technique == 1) {
        // StopGradient(AntiAlias(Rasterize(tgt, 1), RasterizeFaceId(tgt), tgt_clip,
        // tgt_faces, ..., zero seed, 0)) per view (run.cpp:346-357)
        dressi_ctx* ctx = p->ctx;
        void *dclip = nullptr, *dfaces = nullptr;
        if (int rc = ctx_workspace(ctx, 7, clip.size() * 4, &dclip)) return rc;
        if (int rc = ctx_workspace(ctx, 8, (size_t)n_tfaces * 3 * 4, &dfaces)) return rc;
        DRESSI_TRY_HIP(hipMemcpy(dclip, clip.data(), clip.size() * 4, hipMemcpyHostToDevice));
        DRESSI_TRY_HIP(hipMemcpy(dfaces, tgt_faces, (size_t)n_tfaces * 3 * 4,
                                 hipMemcpyHostToDevice));
        const size_t npx = (size_t)p->desc.width * p->desc.height;
        for (uint32_t v = 0; v < N; v++) {
            if (int rc = aa_render_target(ctx, (const float*)dclip + (size_t)v * n_tverts * 4,
                                          n_tverts, (const float*)dfaces, n_tfaces,
                                          p->desc.width, p->desc.height,
                                          (float*)p->d.targets + v * npx)) return rc;
        }
        DRESSI_TRY_HIP(hipStreamSynchronize(ctx->stream));
        p->targets_set = true;
        return DRESSI_OK;
    }
    const RasterGeom g = make_geom(p->desc.width, p->desc.height, N, n_tfaces);
    const uint32_t cap = default_bin_cap(g, 8);
    dressi_ctx* ctx = p->ctx;
    void *dclip = nullptr, *dfi = nullptr, *recs = nullptr, *bins = nullptr, *ones = nullptr;
    if (int rc = ctx_workspace(ctx, 0, sizeof(HardRec) * (size_t)N * n_tfaces, &recs)) return rc;
    if (int rc = ctx_workspace(ctx, 1, bin_bytes(g.n_tiles * N, cap), &bins)) return rc;
    if (int rc = ctx_workspace(ctx, 2, fi.size() * 4, &dfi)) return rc;
    if (int rc = ctx_workspace(ctx, 3, clip.size() * 4, &dclip)) return rc;
    if (int rc = ctx_workspace(ctx, 4, (size_t)n_tverts * 4, &ones)) return rc;
    std::vector<float> one(n_tverts, 1.f);
    hipStream_t s = ctx->stream;
    DRESSI_TRY_HIP(hipMemcpyAsync(dfi, fi.data(), fi.size() * 4, hipMemcpyHostToDevice, s));
    DRESSI_TRY_HIP(hipMemcpyAsync(dclip, clip.data(), clip.size() * 4, hipMemcpyHostToDevice, s));
    DRESSI_TRY_HIP(hipMemcpyAsync(ones, one.data(), one.size() * 4, hipMemcpyHostToDevice, s));
    BinBuffers b;
    bin_carve(bins, g.n_tiles * N, cap, &b);
    DRESSI_TRY_HIP(hipMemsetAsync(b.counts, 0, sizeof(uint32_t) * b.n_bins, s));
    if (int rc = launch_hard_setup(s, g, (const float*)dclip, n_tverts, (const int32_t*)dfi,
                                   (HardRec*)recs)) return rc;
    if (int rc = launch_count_hard(s, g, (const HardRec*)recs, b)) return rc;
    if (int rc = launch_scan_bins(s, b)) return rc;
    if (int rc = launch_bin_hard(s, g, (const HardRec*)recs, b)) return rc;
    if (int rc = launch_raster_hard(s, g, (const HardRec*)recs, b, (const float*)ones, 1, 0,
                                    (float*)p->d.targets)) return rc;
    DRESSI_TRY_HIP(hipStreamSynchronize(s));
    if (int rc = refresh_target_bytes(p)) return rc;
    p->targets_set = true;
    return DRESSI_OK;
}

int dressi_hsr_set_state(dressi_hsr_plan* p, const float* pos, const float* m, const float* v,
                         float t) {
    DRESSI_REQUIRE(p && pos, "bad arguments");
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    hipStream_t s = p->ctx->stream;
    const size_t n = (size_t)p->desc.n_verts * 3 * 4;
    DRESSI_TRY_HIP(hipMemcpyAsync(p->d.pos, pos, n, hipMemcpyHostToDevice, s));
    if (m) {
        DRESSI_TRY_HIP(hipMemcpyAsync(p->d.m, m, n, hipMemcpyHostToDevice, s));
    } else {
        DRESSI_TRY_HIP(hipMemsetAsync(p->d.m, 0, n, s));
    }
    if (v) {
        DRESSI_TRY_HIP(hipMemcpyAsync(p->d.v, v, n, hipMemcpyHostToDevice, s));
    } else {
        DRESSI_TRY_HIP(hipMemsetAsync(p->d.v, 0, n, s));
    }
    DRESSI_TRY_HIP(hipMemcpyAsync(p->d.t, &t, 4, hipMemcpyHostToDevice, s));
    DRESSI_TRY_HIP(hipStreamSynchronize(s));
    p->state_set = true;
    return DRESSI_OK;
}

int dressi_hsr_get_state(dressi_hsr_plan* p, float* pos, float* m, float* v, float* t) {
    DRESSI_REQUIRE(p, "bad arguments");
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    hipStream_t s = p->ctx->stream;
    const size_t n = (size_t)p->desc.n_verts * 3 * 4;
    if (pos) DRESSI_TRY_HIP(hipMemcpyAsync(pos, p->d.pos, n, hipMemcpyDeviceToHost, s));
    if (m) DRESSI_TRY_HIP(hipMemcpyAsync(m, p->d.m, n, hipMemcpyDeviceToHost, s));
    if (v) DRESSI_TRY_HIP(hipMemcpyAsync(v, p->d.v, n, hipMemcpyDeviceToHost, s));
    if (t) DRESSI_TRY_HIP(hipMemcpyAsync(t, p->d.t, 4, hipMemcpyDeviceToHost, s));
    DRESSI_TRY_HIP(hipStreamSynchronize(s));
    return DRESSI_OK;
}

int dressi_hsr_step_eager(dressi_hsr_plan* p, uint32_t n_iters) {
    if (int rc = ready(p)) return rc;
    if (int rc = grow_bins(p)) return rc;
    for (uint32_t i = 0; i < n_iters; i++) {
        if (int rc = enqueue_iteration(p, p->ctx->stream)) return rc;
    }
    return DRESSI_OK;
}

int dressi_hsr_step(dressi_hsr_plan* p, uint32_t n_iters) {
    if (int rc = ready(p)) return rc;
    if (int rc = grow_bins(p)) return rc;
    hipStream_t s = p->ctx->stream;
    if (!p->exec || p->graph_stream != s) {
        drop_graph(p);
        // capture one iteration, and kGraphBatch of them, on a private
        // stream, then replay on `s`
        for (int which = 0; which < 2; which++) {
            hipStream_t cap_stream = nullptr, side = nullptr;
            hipEvent_t ev[2 * kGraphBatch] = {};
            int rc = DRESSI_OK;
            if (hipStreamCreateWithFlags(&cap_stream, hipStreamNonBlocking) != hipSuccess ||
                hipStreamCreateWithFlags(&side, hipStreamNonBlocking) != hipSuccess) {
                set_error("hipStreamCreate failed");
                rc = DRESSI_ERR_HIP;
            }
            for (hipEvent_t& x : ev) {
                if (!rc && hipEventCreateWithFlags(&x, hipEventDisableTiming) != hipSuccess) {
                    set_error("hipEventCreate failed");
                    rc = DRESSI_ERR_HIP;
                }
            }
            hipGraph_t g = nullptr;
            const hipError_t e =
                rc ? hipSuccess : hipStreamBeginCapture(cap_stream, hipStreamCaptureModeThreadLocal);
            if (!rc && e == hipSuccess) {
                const uint32_t reps = which == 0 ? 1u : kGraphBatch;
                // the loss on its own branch pays at large screens (2048 x 2048 x 4
                // views: 468 -> 454 us per iteration); at 512 x 512 the extra graph
                // edges cost more than the overlap gains (106 -> 113 us)
                if (p->d.technique == 0 &&
                    (uint64_t)p->desc.width * p->desc.height >= kForkLossMinPixels) {
                    rc = enqueue_iterations_forked(p, cap_stream, side, reps, ev);
                } else {
                    for (uint32_t r = 0; r < reps && !rc; r++) {
                        rc = enqueue_iteration(p, cap_stream);
                    }
                }
                hipError_t e2 = hipStreamEndCapture(cap_stream, &g);
                if (!rc && e2 != hipSuccess) {
                    set_error("graph capture failed: %s", hipGetErrorString(e2));
                    rc = DRESSI_ERR_HIP;
                }
            } else if (!rc) {
                set_error("hipStreamBeginCapture failed: %s", hipGetErrorString(e));
                rc = DRESSI_ERR_HIP;
            }
            for (hipEvent_t x : ev) {
                if (x) hipEventDestroy(x);
            }
            if (side) hipStreamDestroy(side);
            if (cap_stream) hipStreamDestroy(cap_stream);
            if (which == 0) {
                p->graph = g;
            } else {
                p->graph_batch = g;
            }
            if (rc) {
                drop_graph(p);
                return rc;
            }
        }
        DRESSI_TRY_HIP(hipGraphInstantiate(&p->exec, p->graph, nullptr, nullptr, 0));
        DRESSI_TRY_HIP(hipGraphInstantiate(&p->exec_batch, p->graph_batch, nullptr, nullptr, 0));
        p->graph_stream = s;
    }
    uint32_t i = 0;
    for (; i + kGraphBatch <= n_iters; i += kGraphBatch) {
        DRESSI_TRY_HIP(hipGraphLaunch(p->exec_batch, s));
    }
    for (; i < n_iters; i++) {
        DRESSI_TRY_HIP(hipGraphLaunch(p->exec, s));
    }
    return DRESSI_OK;
}

int dressi_hsr_bin_capacity(dressi_hsr_plan* p, uint32_t* entries) {
    DRESSI_REQUIRE(p && entries, "bad arguments");
    *entries = p->d.bins.cap;
    return DRESSI_OK;
}

int dressi_hsr_buffer(dressi_hsr_plan* p, int which, void** ptr, size_t* bytes) {
    DRESSI_REQUIRE(p && ptr, "bad arguments");
    const size_t npx = (size_t)p->desc.width * p->desc.height;
    const size_t N = p->desc.n_views, V = p->desc.n_verts;
    void* q = nullptr;
    size_t b = 0;
    switch (which) {
        case DRESSI_HSR_LOSS: q = p->d.loss; b = npx * 4; break;
        case DRESSI_HSR_PRED: q = p->d.pred; b = N * npx * 4; break;
        case DRESSI_HSR_TARGET: q = (void*)p->d.targets; b = N * npx * 4; break;
        case DRESSI_HSR_FACE_ID: q = p->d.ids; b = N * npx * 4; break;
        case DRESSI_HSR_GRAD: q = p->d.grad; b = V * 12; break;
        case DRESSI_HSR_POS: q = p->d.pos; b = V * 12; break;
        default: DRESSI_REQUIRE(false, "unknown plan buffer %d", which);
    }
    DRESSI_REQUIRE(q != nullptr, "buffer %d not kept by this plan (see DRESSI_HSR_* flags)", which);
    *ptr = q;
    if (bytes) {
        *bytes = b;
    }
    return DRESSI_OK;
}

int dressi_hsr_read(dressi_hsr_plan* p, int which, void* host, size_t bytes) {
    void* q = nullptr;
    size_t b = 0;
    if (int rc = dressi_hsr_buffer(p, which, &q, &b)) return rc;
    DRESSI_REQUIRE(host && bytes >= b, "host buffer too small (%zu < %zu)", bytes, b);
    DRESSI_TRY_HIP(hipSetDevice(p->ctx->device));
    DRESSI_TRY_HIP(hipMemcpyAsync(host, q, b, hipMemcpyDeviceToHost, p->ctx->stream));
    DRESSI_TRY_HIP(hipStreamSynchronize(p->ctx->stream));
    return DRESSI_OK;
}

int dressi_hsr_profile(dressi_hsr_plan* p, uint32_t iters, char* names, size_t name_stride,
                       float* usec, uint32_t cap, uint32_t* n) {
    if (int rc = ready(p)) return rc;
    DRESSI_REQUIRE(n, "bad arguments");
    // Average device time per launch of each kernel of the iteration, in
    // place: `iters` eager iterations on the plan stream with a HIP event
    // before each kernel and after the last (every kernel sees the state a
    // normal iteration leaves). The optimisation moves `iters` steps.
    const uint32_t reps = iters ? (iters < 256u ? iters : 256u) : 1u;
    *n = kIterKernels;
    hipStream_t s = p->ctx->stream;
    constexpr int kEv = kIterKernels + 1;
    std::vector<hipEvent_t> ev((size_t)reps * kEv, nullptr);
    int rc = DRESSI_OK;
    for (hipEvent_t& e : ev) {
        if (hipEventCreate(&e) != hipSuccess) {
            set_error("hipEventCreate failed");
            rc = DRESSI_ERR_HIP;
            break;
        }
    }
    for (uint32_t r = 0; r < reps && !rc; r++) {
        for (int k = 0; k < kIterKernels && !rc; k++) {
            if (hipEventRecord(ev[(size_t)r * kEv + k], s) != hipSuccess) {
                set_error("hipEventRecord failed");
                rc = DRESSI_ERR_HIP;
                break;
            }
            rc = launch_iter_kernel(p->d, s, k);
        }
        if (!rc && hipEventRecord(ev[(size_t)r * kEv + kIterKernels], s) != hipSuccess) {
            set_error("hipEventRecord failed");
            rc = DRESSI_ERR_HIP;
        }
    }
    if (!rc && hipEventSynchronize(ev.back()) != hipSuccess) {
        set_error("event synchronisation failed");
        rc = DRESSI_ERR_HIP;
    }
    float ms[kIterKernels] = {};
    for (uint32_t r = 0; r < reps && !rc; r++) {
        for (int k = 0; k < kIterKernels; k++) {
            float t = 0.f;
            if (hipEventElapsedTime(&t, ev[(size_t)r * kEv + k], ev[(size_t)r * kEv + k + 1]) !=
                hipSuccess) {
                set_error("hipEventElapsedTime failed");
                rc = DRESSI_ERR_HIP;
                break;
            }
            ms[k] += t / reps;
        }
    }
    for (uint32_t k = 0; k < (uint32_t)kIterKernels && k < cap && !rc; k++) {
        if (usec) {
            usec[k] = ms[k] * 1000.f;
        }
        if (names && name_stride > 0) {
            snprintf(names + k * name_stride, name_stride, "%s",
                     p->d.technique == 1 ? kAaKernelNames[k] : kIterKernelNames[k]);
        }
    }
    for (hipEvent_t e : ev) {
        if (e) {
            hipEventDestroy(e);
        }
    }
    if (!rc) {
        DRESSI_TRY_HIP(hipStreamSynchronize(s));
    }
    return rc;
}

// Per-op entry points --------------------------------------------------------

int dressi_lookup_faces_batch(dressi_ctx* ctx, const float* attr, uint32_t n_comp,
                              uint32_t n_attr, int attr_per_item, const float* faces,
                              uint32_t n_faces, uint32_t corner, uint32_t n_items, float* out) {
    DRESSI_REQUIRE(ctx && attr && faces && out, "bad arguments");
    DRESSI_REQUIRE(corner < 3, "LookupFaces: corner must be 0, 1 or 2");
    DRESSI_REQUIRE(n_comp >= 1 && n_comp <= 4, "n_comp must be 1..4");
    DRESSI_REQUIRE(n_items <= kMaxBatchItems, "batch of %u items exceeds %u", n_items,
                   kMaxBatchItems);
    if (!n_faces || !n_items) return DRESSI_OK;
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    hipLaunchKernelGGL(k_lookup_faces, dim3(div_up(n_faces, 256), n_items), dim3(256), 0,
                       ctx->stream, attr, n_comp, faces, n_faces, n_attr, corner, ctx->d_err, out,
                       attr_per_item ? (size_t)n_attr * n_comp : (size_t)0);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int dressi_lookup_faces(dressi_ctx* ctx, const float* attr, uint32_t n_comp, uint32_t n_attr,
                        const float* faces, uint32_t n_faces, uint32_t corner, float* out) {
    return dressi_lookup_faces_batch(ctx, attr, n_comp, n_attr, 0, faces, n_faces, corner, 1,
                                     out);
}

int dressi_lookup_faces_bwd_batch(dressi_ctx* ctx, const float* gy, uint32_t n_comp,
                                  const float* faces, uint32_t n_faces, const float* vtx_faces,
                                  uint32_t n_verts, uint32_t max_deg, uint32_t corner,
                                  uint32_t n_items, float* out) {
    DRESSI_REQUIRE(ctx && gy && faces && vtx_faces && out, "bad arguments");
    DRESSI_REQUIRE(corner < 3, "LookupFacesBwd: corner must be 0, 1 or 2");
    DRESSI_REQUIRE(n_comp >= 1 && n_comp <= 4, "n_comp must be 1..4");
    DRESSI_REQUIRE(n_items <= kMaxBatchItems, "batch of %u items exceeds %u", n_items,
                   kMaxBatchItems);
    if (!n_verts || !n_items) return DRESSI_OK;
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    hipLaunchKernelGGL(k_lookup_faces_bwd, dim3(div_up(n_verts, 256), n_items), dim3(256), 0,
                       ctx->stream, gy, n_comp, faces, n_faces, vtx_faces, n_verts, max_deg,
                       corner, ctx->d_err, out);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int dressi_lookup_faces_bwd(dressi_ctx* ctx, const float* gy, uint32_t n_comp,
                            const float* faces, uint32_t n_faces, const float* vtx_faces,
                            uint32_t n_verts, uint32_t max_deg, uint32_t corner, float* out) {
    return dressi_lookup_faces_bwd_batch(ctx, gy, n_comp, faces, n_faces, vtx_faces, n_verts,
                                         max_deg, corner, 1, out);
}

int dressi_face_fetch_batch(dressi_ctx* ctx, const float* attr, uint32_t n_comp,
                            uint32_t n_faces, int attr_per_item, const float* idx,
                            uint32_t width, uint32_t height, uint32_t n_items, float* out) {
    DRESSI_REQUIRE(ctx && attr && idx && out, "bad arguments");
    DRESSI_REQUIRE(n_comp >= 1 && n_comp <= 4, "n_comp must be 1..4");
    DRESSI_REQUIRE(n_items <= kMaxBatchItems, "batch of %u items exceeds %u", n_items,
                   kMaxBatchItems);
    const size_t npx = (size_t)width * height;
    if (!npx || !n_items) return DRESSI_OK;
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    hipLaunchKernelGGL(k_face_fetch, dim3((unsigned)((npx + 255) / 256), n_items), dim3(256), 0,
                       ctx->stream, attr, n_comp, n_faces, idx, npx, out,
                       attr_per_item ? (size_t)n_faces * n_comp : (size_t)0);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int dressi_face_fetch(dressi_ctx* ctx, const float* attr, uint32_t n_comp, uint32_t n_faces,
                      const float* idx, uint32_t width, uint32_t height, float* out) {
    return dressi_face_fetch_batch(ctx, attr, n_comp, n_faces, 0, idx, width, height, 1, out);
}

int dressi_face_fetch_bwd_batch(dressi_ctx* ctx, const float* gy, uint32_t n_comp,
                                const float* idx, uint32_t width, uint32_t height,
                                const float* prj0, const float* prj1, const float* prj2,
                                int prj_per_item, uint32_t n_faces, const float* seeds,
                                float radius_px, uint32_t n_samples, uint32_t n_items,
                                float* out) {
    DRESSI_REQUIRE(ctx && gy && idx && prj0 && prj1 && prj2 && seeds && out, "bad arguments");
    DRESSI_REQUIRE(n_comp >= 1 && n_comp <= 4, "n_comp must be 1..4");
    DRESSI_REQUIRE(radius_px > 0.f || n_samples == 0,
                   "FaceFetch: radius must be positive (or n_samples == 0)");
    DRESSI_REQUIRE(n_items <= kMaxBatchItems, "batch of %u items exceeds %u", n_items,
                   kMaxBatchItems);
    if (!n_faces || !n_items) return DRESSI_OK;
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    hipLaunchKernelGGL(k_face_fetch_bwd, dim3(div_up(n_faces, 256), n_items), dim3(256), 0,
                       ctx->stream, gy, n_comp, idx, width, height, (const float4*)prj0,
                       (const float4*)prj1, (const float4*)prj2, n_faces, seeds, radius_px,
                       n_samples, out, prj_per_item ? (size_t)n_faces : (size_t)0);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

int dressi_face_fetch_bwd(dressi_ctx* ctx, const float* gy, uint32_t n_comp, const float* idx,
                          uint32_t width, uint32_t height, const float* prj0, const float* prj1,
                          const float* prj2, uint32_t n_faces, const float* seed,
                          float radius_px, uint32_t n_samples, float* out) {
    return dressi_face_fetch_bwd_batch(ctx, gy, n_comp, idx, width, height, prj0, prj1, prj2, 0,
                                       n_faces, seed, radius_px, n_samples, 1, out);
}

}  // extern "C"
