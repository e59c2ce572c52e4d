// graph_c1.cpp -- the silhouette-fit example written against the graph API
// (#include "dressi/dressi.h") and run by DressiAD: the graph of
// examples/silhouette_optimization/run.cpp:229-437 (all views each
// iteration; technique hardsoftras with one peel, or aa; the in-graph Adam,
// optionally with the example's Laplacian / normal-consistency regulariser
// terms), built with the same C++ expressions, static images from the
// library's mesh builders, sent as CpuImage.
//
//   graph_c1 <in.bin> <out.bin>
// in.bin:  u32 V, F, Vt, Ft, N, S, samples, iters, technique (0 hardsoftras,
//          1 aa), packing (0 RSP, 1 Naive), regs (0 none, 1 regulariser terms),
//          peels (HardSoftRas depth peels, >= 1: run.cpp:302-343),
//          rebuild (0 the default reactive rebuild counts, 1
//          setRebuildCounts(0, 0)), regrow (1: after the third step, a
//          per-op call through DressiAD::context() that needs larger
//          workspaces than the graph's);
//          f32 radius, lr, laplacian weight, normal weight;
//          pos0 {V,3}, faces {F,3}, tgt_pos {Vt,3}, tgt_faces {Ft,3}, mvps N x 16
// out.bin: pos, m, v {V,3}, t, loss[iters] (sum of the loss image),
//          grad0 {V,3} (first iteration), preds and targets {N,S,S} (last),
//          kernels[iters] (getSubStageCount() after each step), ms[iters]
//          (each step's wall time, upload + step + loss download)
// stdout:  "graph_c1: plan=<name> stages=<n> substages=<n> funcs=<n>"
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <vector>

#include "dressi/dressi.h"
#include "dressi_hip.h"
#include "dressi/mesh_utils.h"
#include "dressi_examples/geometry_utils.h"

using namespace dressi;

namespace {

// the example's in-graph vertex transform and host clip images, from the
// library's example helpers (dressi_examples/geometry_utils.h)
dressi_examples::Mat4 MatOf(const float* m) {
    dressi_examples::Mat4 r{};
    std::copy(m, m + 16, r.begin());
    return r;
}

Variable ClipOf(const Variable& pos, const float* mvp) {
    return dressi_examples::TransformToClipVar(pos, MatOf(mvp));
}

CpuImage ClipImage(const std::vector<float>& pos, const float* m) {
    CpuImage p(uint32_t(pos.size() / 3), 1, 3);
    p.data = pos;
    return dressi_examples::TransformToClip(p, MatOf(m));
}

CpuImage Image(const std::vector<float>& d, uint32_t w, uint32_t h, uint32_t c) {
    CpuImage img(w, h, c);
    img.data = d;
    return img;
}

template <typename T>
void get(FILE* f, T* p, size_t n) {
    if (fread(p, sizeof(T), n, f) != n) {
        throw DressiError("short input file");
    }
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 3) {
        fprintf(stderr, "usage: graph_c1 in.bin out.bin\n");
        return 2;
    }
    try {
        FILE* fi = fopen(argv[1], "rb");
        if (!fi) {
            throw DressiError("cannot open input");
        }
        uint32_t hdr[14];
        float fp[4];
        get(fi, hdr, 14);
        get(fi, fp, 4);
        const uint32_t n_verts = hdr[0], n_faces = hdr[1], n_tverts = hdr[2], n_tfaces = hdr[3];
        const uint32_t n_views = hdr[4], S = hdr[5], samples = hdr[6], iters = hdr[7];
        const bool hardsoft = hdr[8] == 0;
        const bool naive = hdr[9] == 1;
        const bool regs = hdr[10] == 1;
        const uint32_t peels = hdr[11] < 1 ? 1 : hdr[11];
        const bool no_rebuild = hdr[12] == 1;
        const bool regrow = hdr[13] == 1;
        const float radius_px = fp[0], lr = fp[1], w_lap = fp[2], w_nrm = fp[3];
        std::vector<float> pos0(n_verts * 3), faces(n_faces * 3), tgt_pos(n_tverts * 3),
                tgt_faces(n_tfaces * 3), mvps(n_views * 16);
        get(fi, pos0.data(), pos0.size());
        get(fi, faces.data(), faces.size());
        get(fi, tgt_pos.data(), tgt_pos.size());
        get(fi, tgt_faces.data(), tgt_faces.size());
        get(fi, mvps.data(), mvps.size());
        fclose(fi);

        const ImgSize screen = {S, S};
        const CpuImage s_faces_img = Image(faces, n_faces, 1, 3);
        const CpuImage b_faces_img = Image(tgt_faces, n_tfaces, 1, 3);
        const CpuImage b_vf_img = VertexFacesTex(b_faces_img, n_tverts);
        const CpuImage s_vf_img = VertexFacesTex(s_faces_img, n_verts);
        const CpuImage s_vn_img = VertexNeighborsTex(s_faces_img, n_verts);
        const CpuImage s_fa_img = FaceNeighborsTex(s_faces_img);

        Variable b_ones(FLOAT, {n_tverts, 1});
        Variable b_faces_i(IVEC3, {n_tfaces, 1});
        Variable b_faces_f(VEC3, {n_tfaces, 1});
        Variable b_vtx_faces(FLOAT, b_vf_img.getImgSize());
        Variable s_ones(FLOAT, {n_verts, 1});
        Variable s_faces_i(IVEC3, {n_faces, 1});
        Variable s_faces_f(VEC3, {n_faces, 1});
        Variable s_vtx_faces(FLOAT, s_vf_img.getImgSize());
        Variable s_vtx_nbrs(FLOAT, s_vn_img.getImgSize());
        Variable s_face_adj(VEC3, {n_faces, 1});
        Variable s_face_id(FLOAT, {n_faces * 3, 1});
        Variable s_faces_soft(IVEC3, {n_faces, 1});
        Variable pos(VEC3, {n_verts, 1});
        Variable adam_m(VEC3, {n_verts, 1});
        Variable adam_v(VEC3, {n_verts, 1});
        Variable adam_t(FLOAT, {1, 1});
        Variable zero_seed(FLOAT, {1, 1});

        const float sigma_scale = 7.f / radius_px;
        const auto build_pred = [&](const Variable& clip_v) -> Variable {
            if (!hardsoft) {
                Variable mask = F::Rasterize(clip_v, s_ones, s_faces_i, screen);
                Variable tri = F::RasterizeFaceId(clip_v, s_ones, s_faces_i, screen);
                return F::AntiAlias(mask, tri, clip_v, s_faces_f, s_vtx_faces, adam_t, samples);
            }
            Variable soft_clip = F::SoftClip(clip_v, s_faces_f, screen, radius_px);
            Variable tri0 = F::LookupFaces(clip_v, s_faces_f, s_vtx_faces, 0);
            Variable tri1 = F::LookupFaces(clip_v, s_faces_f, s_vtx_faces, 1);
            Variable tri2 = F::LookupFaces(clip_v, s_faces_f, s_vtx_faces, 2);
            Variable pc = F::ScreenCoord(screen);
            Variable zero = F::Float(0.f);
            Variable one = F::Float(1.f);
            const auto soft_prob = [&](const Variable& idx) {
                Variable mask = F::Greater(idx, F::Float(0.5f));
                const auto fetch = [&](const Variable& tri) {
                    return F::FaceFetch(tri, idx, tri0, tri1, tri2, adam_t, radius_px, samples);
                };
                const auto screen_of = [&](const Variable& c) {
                    Variable w = F::GetW(c) + (1.f - mask);
                    Variable sx = (F::GetX(c) / w * 0.5f + 0.5f) * float(screen.w);
                    Variable sy = (F::GetY(c) / w * 0.5f + 0.5f) * float(screen.h);
                    return F::Vec2(sx, sy);
                };
                Variable s0 = screen_of(fetch(tri0));
                Variable s1 = screen_of(fetch(tri1));
                Variable s2 = screen_of(fetch(tri2));
                const auto edge_dist = [&](const Variable& a, const Variable& b) {
                    Variable e = b - a;
                    Variable t = F::Clamp(F::Dot(pc - a, e) / (F::Dot(e, e) + 1e-12f), zero, one);
                    Variable dd = pc - (a + t * e);
                    return F::Sqrt(F::Dot(dd, dd) + 1e-12f);
                };
                const auto edge_cross = [&](const Variable& a, const Variable& b) {
                    Variable e = b - a;
                    return F::GetX(e) * (F::GetY(pc) - F::GetY(a)) -
                           F::GetY(e) * (F::GetX(pc) - F::GetX(a));
                };
                Variable dmin = F::Min(F::Min(edge_dist(s0, s1), edge_dist(s1, s2)),
                                       edge_dist(s2, s0));
                Variable cr0 = edge_cross(s0, s1);
                Variable cr1 = edge_cross(s1, s2);
                Variable cr2 = edge_cross(s2, s0);
                Variable inside = F::Min(F::Step(zero, cr0) * F::Step(zero, cr1) *
                                                         F::Step(zero, cr2) +
                                                 F::Step(zero, -cr0) * F::Step(zero, -cr1) *
                                                         F::Step(zero, -cr2),
                                         one);
                Variable dist = (inside * 2.f - 1.f) * dmin;
                return mask * F::Sigmoid(dist * sigma_scale);
            };
            // Alg. 2 depth peeling: peel k rejects fragments at or in front of
            // peel k - 1's shifted depth; Eq. 6: 1 - prod_k (1 - D_k)
            Variable one_minus = one;
            Variable prev_shift(nullptr);
            Variable hard(nullptr);
            for (uint32_t peel = 0; peel < peels; peel++) {
                Variable rs = F::StopGradient(
                        peel == 0 ? F::RasterizeSoft(soft_clip, s_face_id, s_faces_soft, clip_v,
                                                     s_faces_f, s_vtx_faces, screen, radius_px)
                                  : F::RasterizeSoft(soft_clip, s_face_id, s_faces_soft, clip_v,
                                                     s_faces_f, s_vtx_faces, prev_shift, screen,
                                                     radius_px));
                Variable dist_c = F::GetX(rs);
                Variable cov = F::GetW(rs);
                Variable ge = F::Step(zero, dist_c);
                prev_shift = cov * (ge * (F::Clamp(F::GetZ(rs), zero, one) * 0.5f) +
                                    (1.f - ge) * (F::Clamp(-dist_c * (1.f / radius_px), zero,
                                                           one) * 0.5f + 0.5f));
                Variable idx = (F::GetY(rs) + 1.f) * cov;
                one_minus = one_minus * (1.f - soft_prob(idx));
                if (peel == 0) {
                    hard = cov * ge;
                }
            }
            Variable soft_sil = 1.f - one_minus;
            return F::Max(hard, soft_sil);
        };
        const auto build_target = [&](const Variable& tgt_clip) -> Variable {
            Variable t_mask = F::Rasterize(tgt_clip, b_ones, b_faces_i, screen);
            if (hardsoft) {
                return F::StopGradient(t_mask);
            }
            Variable t_tri = F::RasterizeFaceId(tgt_clip, b_ones, b_faces_i, screen);
            return F::StopGradient(
                    F::AntiAlias(t_mask, t_tri, tgt_clip, b_faces_f, b_vtx_faces, zero_seed, 0));
        };

        Variables targets, preds, view_losses;
        std::vector<Variable> tgt_clips;
        for (uint32_t v = 0; v < n_views; v++) {
            tgt_clips.emplace_back(VEC4, ImgSize{n_tverts, 1});
            targets.push_back(build_target(tgt_clips.back()));
            preds.push_back(build_pred(ClipOf(pos, mvps.data() + 16 * v)));
            Variable diff = targets[v] - preds[v];
            view_losses.push_back(diff * diff * (1.f / float(screen.w * screen.h)));
        }
        Variable loss = F::SumPixelWise(view_losses);
        Variable pos_mut = pos;
        pos_mut.setRequiresGradRecursively();

        DressiAD ad;
        ad.setPackingMode(naive ? DressiAD::PackingMode::Naive : DressiAD::PackingMode::RSP);
        if (no_rebuild) {
            ad.setRebuildCounts(0, 0);
        }
        ad.setLossVar(loss);
        bool state_registered = false;
        ad.setOptimizer([&](Variables xs, Variables gxs) {
            DRESSI_CHECK(xs.size() == 1 && xs[0] == pos,
                         "expected pos as the only optimizer target");
            Variable g = gxs[0];
            if (regs) {
                const float inv_cnt = 1.f / float(n_verts * 3);
                const auto rms = [&](const Variable& x) {
                    return F::Sqrt(F::SumAll(x * x) * inv_cnt + 1e-24f);
                };
                Variable data_rms = rms(g);
                Variable g_lap = pos - F::VertexNeighborMean(pos, s_vtx_nbrs);
                Variable g_nrm = F::NormalConsistencyVertexGrad(
                        F::NormalConsistencyFaceTerm(pos, s_faces_f, s_face_adj), pos, s_faces_f,
                        s_vtx_faces);
                g = g + g_lap * (data_rms / rms(g_lap) * w_lap) +
                    g_nrm * (data_rms / rms(g_nrm) * w_nrm);
            }
            const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
            Variable t_new = adam_t + 1.f;
            Variable m_new = adam_m * b1 + g * (1.f - b1);
            Variable v_new = adam_v * b2 + g * g * (1.f - b2);
            Variable bc1 = 1.f - F::Pow(F::Float(b1), t_new);
            Variable bc2 = 1.f - F::Pow(F::Float(b2), t_new);
            Variable step = (m_new / bc1) / (F::Sqrt(v_new / bc2) + eps) * lr;
            if (!state_registered) {
                ad.addUpdate(adam_m, m_new);
                ad.addUpdate(adam_v, v_new);
                ad.addUpdate(adam_t, t_new);
                state_registered = true;
            }
            return Variables{pos - step};
        });
        for (size_t i = 0; i < preds.size(); i++) {
            ad.markOutput(targets[i]);
            ad.markOutput(preds[i]);
        }
        ad.setGradOutputsEnabled(true);

        // one-time uploads (run.cpp:440-471)
        ad.sendImg(b_ones, CpuImage(n_tverts, 1, 1, 1.f));
        ad.sendImg(b_faces_i, b_faces_img);
        ad.sendImg(b_faces_f, b_faces_img);
        ad.sendImg(b_vtx_faces, b_vf_img);
        ad.sendImg(s_ones, CpuImage(n_verts, 1, 1, 1.f));
        ad.sendImg(s_faces_i, s_faces_img);
        ad.sendImg(s_faces_f, s_faces_img);
        ad.sendImg(s_vtx_faces, s_vf_img);
        ad.sendImg(s_vtx_nbrs, s_vn_img);
        ad.sendImg(s_face_adj, s_fa_img);
        if (hardsoft) {
            CpuImage face_id_img(n_faces * 3, 1, 1);
            CpuImage faces_soft_img(n_faces, 1, 3);
            for (uint32_t f = 0; f < n_faces; f++) {
                for (uint32_t k = 0; k < 3; k++) {
                    face_id_img.at(f * 3 + k, 0, 0) = float(f);
                    faces_soft_img.at(f, 0, k) = float(f * 3 + k);
                }
            }
            ad.sendImg(s_face_id, face_id_img);
            ad.sendImg(s_faces_soft, faces_soft_img);
        }
        ad.sendImg(adam_m, CpuImage(n_verts, 1, 3, 0.f));
        ad.sendImg(adam_v, CpuImage(n_verts, 1, 3, 0.f));
        ad.sendImg(adam_t, CpuImage(1, 1, 1, 0.f));
        if (!hardsoft) {
            ad.sendImg(zero_seed, CpuImage(1, 1, 1, 0.f));
        }
        for (uint32_t v = 0; v < n_views; v++) {
            ad.sendImg(tgt_clips[v], ClipImage(tgt_pos, mvps.data() + 16 * v));
        }

        // iterations: the starting positions go with the first step; every
        // step returns its loss image with the same synchronisation
        const CpuImage pos_img = Image(pos0, n_verts, 1, 3);
        std::vector<float> losses(iters), kernels(iters), step_ms(iters);
        CpuImage grad0;
        for (uint32_t it = 0; it < iters; it++) {
            std::vector<std::pair<Variable, CpuImageView>> sends;
            if (it == 0) {
                sends.emplace_back(pos, CpuImageView(pos_img));
            }
            if (regrow && it == 3) {
                // a per-op call on the instance's own C-ABI context whose
                // screen needs larger tile bins than any step so far
                dressi_ctx* c = ad.context();
                const uint32_t big = 4 * S + 64;
                std::vector<float> clip(n_verts * 4, 0.f);
                for (uint32_t i = 0; i < n_verts; i++) {
                    clip[i * 4 + 0] = pos0[i * 3 + 0] * 0.5f;
                    clip[i * 4 + 1] = pos0[i * 3 + 1] * 0.5f;
                    clip[i * 4 + 2] = 0.5f;
                    clip[i * 4 + 3] = 1.f;
                }
                void *d_clip = nullptr, *d_faces = nullptr, *d_ones = nullptr, *d_out = nullptr;
                const std::vector<float> ones(n_verts, 1.f);
                if (dressi_malloc(c, &d_clip, clip.size() * 4) ||
                    dressi_malloc(c, &d_faces, faces.size() * 4) ||
                    dressi_malloc(c, &d_ones, ones.size() * 4) ||
                    dressi_malloc(c, &d_out, size_t(big) * big * 4) ||
                    dressi_memcpy_h2d(c, d_clip, clip.data(), clip.size() * 4) ||
                    dressi_memcpy_h2d(c, d_faces, faces.data(), faces.size() * 4) ||
                    dressi_memcpy_h2d(c, d_ones, ones.data(), ones.size() * 4) ||
                    dressi_rasterize(c, (const float*)d_clip, n_verts, (const float*)d_ones, 1,
                                     (const float*)d_faces, n_faces, big, big, (float*)d_out) ||
                    dressi_ctx_synchronize(c)) {
                    throw DressiError(std::string("regrow call: ") + dressi_last_error());
                }
                dressi_free(c, d_clip);
                dressi_free(c, d_faces);
                dressi_free(c, d_ones);
                dressi_free(c, d_out);
            }
            const auto t0 = std::chrono::steady_clock::now();
            const CpuImage li = ad.execStepWithSendsAndRecvImgsStacked(sends, {loss});
            step_ms[it] = std::chrono::duration<float, std::milli>(
                                  std::chrono::steady_clock::now() - t0)
                                  .count();
            kernels[it] = float(ad.getSubStageCount());
            double s = 0.0;
            for (float x : li.data) {
                s += x;
            }
            losses[it] = float(s);
            if (it == 0) {
                grad0 = ad.recvImg(ad.inputGrads().at(0).second);
            }
        }
        const CpuImage pred_img = ad.recvImgsStacked(preds);
        const CpuImage tgt_img = ad.recvImgsStacked(targets);
        FILE* fo = fopen(argv[2], "wb");
        if (!fo) {
            throw DressiError("cannot open output");
        }
        for (const Variable& v : {pos, adam_m, adam_v, adam_t}) {
            const CpuImage d = ad.recvImg(v);
            fwrite(d.data.data(), sizeof(float), d.data.size(), fo);
        }
        fwrite(losses.data(), sizeof(float), losses.size(), fo);
        fwrite(grad0.data.data(), sizeof(float), grad0.data.size(), fo);
        fwrite(pred_img.data.data(), sizeof(float), pred_img.data.size(), fo);
        fwrite(tgt_img.data.data(), sizeof(float), tgt_img.data.size(), fo);
        fwrite(kernels.data(), sizeof(float), kernels.size(), fo);
        fwrite(step_ms.data(), sizeof(float), step_ms.size(), fo);
        fclose(fo);
        printf("graph_c1: plan=%s stages=%zu substages=%zu funcs=%zu device=%s\n",
               ad.getPlanName().c_str(), ad.getStageCount(), ad.getSubStageCount(),
               ad.getFuncCount(), ad.getDeviceName().c_str());
    } catch (const std::exception& e) {
        fprintf(stderr, "graph_c1: %s\n", e.what());
        return 1;
    }
    return 0;
}
