// graph_c1.cpp -- the silhouette fit written with the graph API
// (include/dressi_graph.h) and run by its generic executor: the graph of
// examples/silhouette_optimization/run.cpp:229-437 (technique hardsoftras
// with one peel, or aa; no regularisers), built with the same C++
// expressions so that node creation order -- hence the backward's
// summation order -- is the reference build's.
//
//   graph_c1 <in.bin> <out.bin>
// in.bin: u32 V, F, Vt, Ft, N, S, samples, iters, technique (0 hsr, 1 aa);
//         f32 radius, lr;
//         pos0 {V,3}, faces {F,3}, tgt_pos {Vt,3}, tgt_faces {Ft,3}, mvps N x 16
// out.bin: pos, m, v {V,3}, t, loss[iters] (sum of the loss image), grad0 {V,3}
#include <cstdio>
#include <cstring>
#include <vector>

#include "dressi_graph.h"

using namespace dressi;

namespace {

Variable ClipOf(const Variable& pos, const float* mvp) {
    Variable x = F::GetX(pos);
    Variable y = F::GetY(pos);
    Variable z = F::GetZ(pos);
    const auto row = [&](int r) {
        return x * mvp[size_t(0 * 4 + r)] + y * mvp[size_t(1 * 4 + r)] +
               z * mvp[size_t(2 * 4 + r)] + mvp[size_t(3 * 4 + r)];
    };
    return F::Vec4(row(0), row(1), row(2), row(3));
}

// {max_deg, V} incident faces, ascending, -1 padded
std::vector<float> VertexFaces(const std::vector<float>& faces, uint32_t nv, uint32_t* deg) {
    std::vector<std::vector<uint32_t>> inc(nv);
    for (uint32_t f = 0; f < faces.size() / 3; f++) {
        for (int k = 0; k < 3; k++) {
            inc[(uint32_t)faces[f * 3 + k]].push_back(f);
        }
    }
    uint32_t d = 1;
    for (const auto& l : inc) {
        d = std::max<uint32_t>(d, (uint32_t)l.size());
    }
    std::vector<float> out(size_t(d) * nv, -1.f);
    for (uint32_t v = 0; v < nv; v++) {
        for (size_t i = 0; i < inc[v].size(); i++) {
            out[i * nv + v] = float(inc[v][i]);
        }
    }
    *deg = d;
    return out;
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
        uint32_t hdr[9];
        float fp[2];
        get(fi, hdr, 9);
        get(fi, fp, 2);
        const uint32_t n_verts = hdr[0], n_faces = hdr[1], n_tverts = hdr[2], n_tfaces = hdr[3];
        const uint32_t n_views = hdr[4], S = hdr[5], samples = hdr[6], iters = hdr[7];
        const bool aa = hdr[8] == 1;
        const float radius_px = fp[0], lr = fp[1];
        std::vector<float> pos0(n_verts * 3), faces(n_faces * 3), tgt_pos(n_tverts * 3),
                tgt_faces(n_tfaces * 3), mvps(n_views * 16);
        get(fi, pos0.data(), pos0.size());
        get(fi, faces.data(), faces.size());
        get(fi, tgt_pos.data(), tgt_pos.size());
        get(fi, tgt_faces.data(), tgt_faces.size());
        get(fi, mvps.data(), mvps.size());
        fclose(fi);

        const ImgSize screen = {S, S};
        uint32_t deg = 0;
        const std::vector<float> vf = VertexFaces(faces, n_verts, &deg);

        Variable b_ones(FLOAT, {n_tverts, 1});
        Variable b_faces_i(IVEC3, {n_tfaces, 1});
        Variable s_faces_f(VEC3, {n_faces, 1});
        Variable s_vtx_faces(FLOAT, {n_verts, deg});
        Variable s_face_id(FLOAT, {n_faces * 3, 1});
        Variable s_faces_soft(IVEC3, {n_faces, 1});
        Variable pos(VEC3, {n_verts, 1});
        Variable adam_m(VEC3, {n_verts, 1});
        Variable adam_v(VEC3, {n_verts, 1});
        Variable adam_t(FLOAT, {1, 1});

        const float sigma_scale = 7.f / radius_px;
        const auto build_pred = [&](const Variable& clip_v) -> Variable {
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
            Variable one_minus = one;
            Variable rs = F::StopGradient(F::RasterizeSoft(soft_clip, s_face_id, s_faces_soft,
                                                           clip_v, s_faces_f, s_vtx_faces, screen,
                                                           radius_px));
            Variable dist_c = F::GetX(rs);
            Variable cov = F::GetW(rs);
            Variable ge = F::Step(zero, dist_c);
            Variable idx = (F::GetY(rs) + 1.f) * cov;
            one_minus = one_minus * (1.f - soft_prob(idx));
            Variable hard = cov * ge;
            Variable soft_sil = 1.f - one_minus;
            return F::Max(hard, soft_sil);
        };

        // technique aa (run.cpp:320-357): the prediction and the target are
        // AntiAlias'd hard masks
        uint32_t tdeg = 0;
        const std::vector<float> tvf = VertexFaces(tgt_faces, n_tverts, &tdeg);
        Variable b_faces_f(VEC3, {n_tfaces, 1});
        Variable b_vtx_faces(FLOAT, {n_tverts, tdeg});
        Variable s_ones(FLOAT, {n_verts, 1});
        Variable s_faces_i(IVEC3, {n_faces, 1});
        Variable zero_seed(FLOAT, {1, 1});
        const auto build_pred_aa = [&](const Variable& clip_v) -> Variable {
            Variable mask = F::Rasterize(clip_v, s_ones, s_faces_i, screen);
            Variable tri = F::RasterizeFaceId(clip_v, s_ones, s_faces_i, screen);
            return F::AntiAlias(mask, tri, clip_v, s_faces_f, s_vtx_faces, adam_t, samples);
        };
        const auto build_target_aa = [&](const Variable& tgt_clip) -> Variable {
            Variable t_mask = F::Rasterize(tgt_clip, b_ones, b_faces_i, screen);
            Variable t_tri = F::RasterizeFaceId(tgt_clip, b_ones, b_faces_i, screen);
            return F::StopGradient(
                    F::AntiAlias(t_mask, t_tri, tgt_clip, b_faces_f, b_vtx_faces, zero_seed, 0));
        };

        Variables targets, preds, view_losses;
        std::vector<Variable> tgt_clips;
        for (uint32_t v = 0; v < n_views; v++) {
            tgt_clips.emplace_back(VEC4, ImgSize{n_tverts, 1});
            if (aa) {
                targets.push_back(build_target_aa(tgt_clips.back()));
                preds.push_back(build_pred_aa(ClipOf(pos, mvps.data() + 16 * v)));
            } else {
                targets.push_back(F::StopGradient(
                        F::Rasterize(tgt_clips.back(), b_ones, b_faces_i, screen)));
                preds.push_back(build_pred(ClipOf(pos, mvps.data() + 16 * v)));
            }
            Variable diff = targets[v] - preds[v];
            view_losses.push_back(diff * diff * (1.f / float(screen.w * screen.h)));
        }
        Variable loss = F::SumPixelWise(view_losses);
        Variable pos_mut = pos;
        pos_mut.setRequiresGradRecursively();

        DressiAD ad;
        ad.setLossVar(loss);
        Variable g0;
        ad.setOptimizer([&](Variables xs, Variables gxs) {
            if (xs.size() != 1 || xs[0] != pos) {
                throw DressiError("expected pos as the only optimizer target");
            }
            Variable g = gxs[0];
            g0 = g;
            const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
            Variable t_new = adam_t + 1.f;
            Variable m_new = adam_m * b1 + g * (1.f - b1);
            Variable v_new = adam_v * b2 + g * g * (1.f - b2);
            Variable bc1 = 1.f - F::Pow(F::Float(b1), t_new);
            Variable bc2 = 1.f - F::Pow(F::Float(b2), t_new);
            Variable step = (m_new / bc1) / (F::Sqrt(v_new / bc2) + eps) * lr;
            ad.addUpdate(adam_m, m_new);
            ad.addUpdate(adam_v, v_new);
            ad.addUpdate(adam_t, t_new);
            return Variables{pos - step};
        });
        (void)ad.inputGrads();  // builds the backward and the optimizer graph
        ad.markOutput(g0);

        // static leaves
        std::vector<float> ones(n_tverts, 1.f), fid(n_faces * 3), fsoft(n_faces * 3);
        for (uint32_t f = 0; f < n_faces; f++) {
            for (uint32_t k = 0; k < 3; k++) {
                fid[f * 3 + k] = float(f);
                fsoft[f * 3 + k] = float(f * 3 + k);
            }
        }
        ad.sendImg(b_ones, ones.data());
        ad.sendImg(b_faces_i, tgt_faces.data());
        ad.sendImg(s_faces_f, faces.data());
        ad.sendImg(s_vtx_faces, vf.data());
        ad.sendImg(s_face_id, fid.data());
        ad.sendImg(s_faces_soft, fsoft.data());
        if (aa) {
            std::vector<float> s_ones_v(n_verts, 1.f), zero_v(1, 0.f);
            ad.sendImg(b_faces_f, tgt_faces.data());
            ad.sendImg(b_vtx_faces, tvf.data());
            ad.sendImg(s_ones, s_ones_v.data());
            ad.sendImg(s_faces_i, faces.data());
            ad.sendImg(zero_seed, zero_v.data());
        }
        for (uint32_t v = 0; v < n_views; v++) {
            const float* m = mvps.data() + 16 * v;
            std::vector<float> c(size_t(n_tverts) * 4);
            for (uint32_t i = 0; i < n_tverts; i++) {
                const float p[4] = {tgt_pos[i * 3 + 0], tgt_pos[i * 3 + 1], tgt_pos[i * 3 + 2], 1.f};
                for (int r = 0; r < 4; r++) {
                    float acc = 0.f;
                    for (int k = 0; k < 4; k++) {
                        acc += m[k * 4 + r] * p[k];
                    }
                    c[size_t(i) * 4 + r] = acc;
                }
            }
            ad.sendImg(tgt_clips[v], c.data());
        }
        std::vector<float> zeros(n_verts * 3, 0.f), zero1(1, 0.f);
        ad.sendImg(pos, pos0.data());
        ad.sendImg(adam_m, zeros.data());
        ad.sendImg(adam_v, zeros.data());
        ad.sendImg(adam_t, zero1.data());

        std::vector<float> losses(iters), grad0;
        for (uint32_t it = 0; it < iters; it++) {
            ad.execStep();
            const std::vector<float> li = ad.recvImg(loss);
            double s = 0.0;
            for (float x : li) {
                s += x;
            }
            losses[it] = float(s);
            if (it == 0) {
                grad0 = ad.recvImg(g0);
            }
        }
        FILE* fo = fopen(argv[2], "wb");
        if (!fo) {
            throw DressiError("cannot open output");
        }
        for (const Variable& v : {pos, adam_m, adam_v, adam_t}) {
            const std::vector<float> d = ad.recvImg(v);
            fwrite(d.data(), sizeof(float), d.size(), fo);
        }
        fwrite(losses.data(), sizeof(float), losses.size(), fo);
        fwrite(grad0.data(), sizeof(float), grad0.size(), fo);
        fclose(fo);
        printf("graph_c1: %zu functions per step, %u iterations\n", ad.getFuncCount(), iters);
    } catch (const std::exception& e) {
        fprintf(stderr, "graph_c1: %s\n", e.what());
        return 1;
    }
    return 0;
}
