// Reference-CPU harness: TEST INFRASTRUCTURE ONLY.
//
// This file is compiled together with the reference's own CPU sources
// (src/core/*.cpp and examples/common/geometry_utils.cpp, read in place from
// the reference checkout by oracle/Makefile) into oracle/_ref/libdressi_ref.so.
// It drives the reference's graph API + CpuEvaluator, so its outputs are the
// reference's own numbers. They are used to pin the C restatement in
// oracle/dressi_oracle.c (golden fixtures under tests/golden/) and as the
// "reference" CPU baseline. Nothing in the product path loads it.
//
// Every entry point is extern "C" with plain pointers so ctypes can call it.
// Return value: 0 on success, -1 on error (message via refh_last_error()).

#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "core/build_backward.h"
#include "core/cpu_eval.h"
#include "core/node.h"
#include "dressi/dressi.h"
#include "dressi/mesh_utils.h"

#include "dressi/ibl.h"
#include "geometry_utils.h"
#include "pbr_graph.h"

using namespace dressi;

namespace {

thread_local std::string g_err;

CpuTensor Tensor(VType vt, ImgSize sz, const float* data) {
    CpuTensor t;
    t.vtype = vt;
    t.size = sz;
    t.data.assign(data, data + size_t(sz.w) * sz.h * NumComponents(vt));
    return t;
}

CpuTensor Fill(VType vt, ImgSize sz, float v) {
    CpuTensor t;
    t.vtype = vt;
    t.size = sz;
    t.data.assign(size_t(sz.w) * sz.h * NumComponents(vt), v);
    return t;
}

void CopyOut(const CpuTensor& t, float* out) {
    if (out) {
        std::memcpy(out, t.data.data(), t.data.size() * sizeof(float));
    }
}

VType VecOf(uint32_t n) { return VecVTypeOf(n); }

template <typename Fn>
int Guard(Fn&& fn) {
    try {
        fn();
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -1;
    }
}

// Clip transform as an image-op chain (the silhouette example's
// TransformToClipVar expression: one row per clip component, column-major
// MVP), written with the same C++ expression shape so that node creation
// order matches the example build.
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

}  // namespace

extern "C" {

const char* refh_last_error() { return g_err.c_str(); }

// F::SoftClip: clip {V,1} VEC4 + faces {F,1} VEC3 -> {3F,1} VEC4
int refh_soft_clip(const float* clip, uint32_t n_verts, const float* faces,
                   uint32_t n_faces, uint32_t w, uint32_t h, float radius,
                   float* out) {
    return Guard([&] {
        Variable vc(VEC4, {n_verts, 1});
        Variable vf(VEC3, {n_faces, 1});
        Variable y = F::SoftClip(vc, vf, {w, h}, radius);
        CpuEvaluator ev;
        ev.bind(vc, Tensor(VEC4, {n_verts, 1}, clip));
        ev.bind(vf, Tensor(VEC3, {n_faces, 1}, faces));
        CopyOut(ev.eval(y), out);
    });
}

// F::RasterizeSoft (and its peel overload when prev != nullptr)
int refh_rasterize_soft(const float* soft_clip, const float* face_id,
                        const float* faces_soft, const float* hard_clip,
                        uint32_t n_verts, const float* faces_tex,
                        const float* vtx_faces, uint32_t max_deg,
                        uint32_t n_faces, uint32_t w, uint32_t h, float radius,
                        const float* prev, float* out) {
    return Guard([&] {
        Variable sc(VEC4, {3 * n_faces, 1});
        Variable fid(FLOAT, {3 * n_faces, 1});
        Variable fs(IVEC3, {n_faces, 1});
        Variable hc(VEC4, {n_verts, 1});
        Variable ft(VEC3, {n_faces, 1});
        Variable vf(FLOAT, {n_verts, max_deg});
        Variable pv(FLOAT, {w, h});
        Variable y = prev ? F::RasterizeSoft(sc, fid, fs, hc, ft, vf, pv,
                                             {w, h}, radius)
                          : F::RasterizeSoft(sc, fid, fs, hc, ft, vf, {w, h},
                                             radius);
        CpuEvaluator ev;
        ev.bind(sc, Tensor(VEC4, {3 * n_faces, 1}, soft_clip));
        ev.bind(fid, Tensor(FLOAT, {3 * n_faces, 1}, face_id));
        ev.bind(fs, Tensor(IVEC3, {n_faces, 1}, faces_soft));
        ev.bind(hc, Tensor(VEC4, {n_verts, 1}, hard_clip));
        ev.bind(ft, Tensor(VEC3, {n_faces, 1}, faces_tex));
        ev.bind(vf, Tensor(FLOAT, {n_verts, max_deg}, vtx_faces));
        if (prev) {
            ev.bind(pv, Tensor(FLOAT, {w, h}, prev));
        }
        CopyOut(ev.eval(y), out);
    });
}

// RasterizeSoft's backward w.r.t. the hard clip positions (f_ops.cpp:
// 1448-1455): ColSum(GatherDistGrad(gy, y, ..., wide)) for gy {w,h} VEC4
// (only the dist channel is read); out_wide {max_deg, V, 4} the gather's
// partials, out_vtx {V, 4} their ColSum.
int refh_rasterize_soft_bwd(const float* soft_clip, const float* face_id,
                            const float* faces_soft, const float* hard_clip,
                            uint32_t n_verts, const float* faces_tex,
                            const float* vtx_faces, uint32_t max_deg,
                            uint32_t n_faces, uint32_t w, uint32_t h, float radius,
                            const float* gy, float* out_wide, float* out_vtx) {
    return Guard([&] {
        Variable sc(VEC4, {3 * n_faces, 1});
        Variable fid(FLOAT, {3 * n_faces, 1});
        Variable fs(IVEC3, {n_faces, 1});
        Variable hc(VEC4, {n_verts, 1});
        Variable ft(VEC3, {n_faces, 1});
        Variable vf(FLOAT, {n_verts, max_deg});
        Variable vgy(VEC4, {w, h});
        Variable y = F::RasterizeSoft(sc, fid, fs, hc, ft, vf, {w, h}, radius);
        Variable g = y.getCreator().buildBwd(vgy, 3);
        CpuEvaluator ev;
        ev.bind(sc, Tensor(VEC4, {3 * n_faces, 1}, soft_clip));
        ev.bind(fid, Tensor(FLOAT, {3 * n_faces, 1}, face_id));
        ev.bind(fs, Tensor(IVEC3, {n_faces, 1}, faces_soft));
        ev.bind(hc, Tensor(VEC4, {n_verts, 1}, hard_clip));
        ev.bind(ft, Tensor(VEC3, {n_faces, 1}, faces_tex));
        ev.bind(vf, Tensor(FLOAT, {n_verts, max_deg}, vtx_faces));
        ev.bind(vgy, Tensor(VEC4, {w, h}, gy));
        if (out_vtx) {
            CopyOut(ev.eval(g), out_vtx);
        }
        if (out_wide) {
            CopyOut(ev.eval(g.getCreator().getInputVars()[0]), out_wide);
        }
    });
}

// F::Rasterize (hard, perspective-correct attribute interpolation)
int refh_rasterize(const float* clip, uint32_t n_verts, const float* attr,
                   uint32_t n_comp, const float* faces, uint32_t n_faces,
                   uint32_t w, uint32_t h, float* out) {
    return Guard([&] {
        Variable vc(VEC4, {n_verts, 1});
        Variable va(VecOf(n_comp), {n_verts, 1});
        Variable vf(IVEC3, {n_faces, 1});
        Variable y = F::Rasterize(vc, va, vf, {w, h});
        CpuEvaluator ev;
        ev.bind(vc, Tensor(VEC4, {n_verts, 1}, clip));
        ev.bind(va, Tensor(VecOf(n_comp), {n_verts, 1}, attr));
        ev.bind(vf, Tensor(IVEC3, {n_faces, 1}, faces));
        CopyOut(ev.eval(y), out);
    });
}

// F::RasterizeFaceId: float(f) + 1, 0 = background
int refh_rasterize_face_id(const float* clip, uint32_t n_verts,
                           const float* faces, uint32_t n_faces, uint32_t w,
                           uint32_t h, float* out) {
    return Guard([&] {
        Variable vc(VEC4, {n_verts, 1});
        Variable va(FLOAT, {n_verts, 1});
        Variable vf(IVEC3, {n_faces, 1});
        Variable y = F::RasterizeFaceId(vc, va, vf, {w, h});
        CpuEvaluator ev;
        ev.bind(vc, Tensor(VEC4, {n_verts, 1}, clip));
        ev.bind(va, Fill(FLOAT, {n_verts, 1}, 1.f));
        ev.bind(vf, Tensor(IVEC3, {n_faces, 1}, faces));
        CopyOut(ev.eval(y), out);
    });
}

// Backward of F::FaceFetch w.r.t. tri_attr (the stochastic / exact gather),
// obtained from the op's own backward generator.
int refh_face_fetch_bwd(const float* gy, uint32_t n_comp, const float* idx,
                        uint32_t w, uint32_t h, const float* prj0,
                        const float* prj1, const float* prj2,
                        uint32_t n_faces, float seed, float radius,
                        uint32_t n_samples, float* out) {
    return Guard([&] {
        Variable attr(VecOf(n_comp), {n_faces, 1});
        Variable vidx(FLOAT, {w, h});
        Variable p0(VEC4, {n_faces, 1});
        Variable p1(VEC4, {n_faces, 1});
        Variable p2(VEC4, {n_faces, 1});
        Variable vs(FLOAT, {1, 1});
        Variable vgy(VecOf(n_comp), {w, h});
        Variable y = F::FaceFetch(attr, vidx, p0, p1, p2, vs, radius,
                                  n_samples);
        Variable g = y.getCreator().buildBwd(vgy, 0);
        CpuEvaluator ev;
        ev.bind(vidx, Tensor(FLOAT, {w, h}, idx));
        ev.bind(p0, Tensor(VEC4, {n_faces, 1}, prj0));
        ev.bind(p1, Tensor(VEC4, {n_faces, 1}, prj1));
        ev.bind(p2, Tensor(VEC4, {n_faces, 1}, prj2));
        ev.bind(vs, Fill(FLOAT, {1, 1}, seed));
        ev.bind(vgy, Tensor(VecOf(n_comp), {w, h}, gy));
        CopyOut(ev.eval(g), out);
    });
}

// F::FaceFetch forward
int refh_face_fetch(const float* attr, uint32_t n_comp, uint32_t n_faces,
                    const float* idx, uint32_t w, uint32_t h, float* out) {
    return Guard([&] {
        Variable va(VecOf(n_comp), {n_faces, 1});
        Variable vidx(FLOAT, {w, h});
        Variable p(VEC4, {n_faces, 1});
        Variable vs(FLOAT, {1, 1});
        Variable y = F::FaceFetch(va, vidx, p, p, p, vs, 1.f, 4);
        CpuEvaluator ev;
        ev.bind(va, Tensor(VecOf(n_comp), {n_faces, 1}, attr));
        ev.bind(vidx, Tensor(FLOAT, {w, h}, idx));
        ev.bind(p, Fill(VEC4, {n_faces, 1}, 1.f));
        ev.bind(vs, Fill(FLOAT, {1, 1}, 0.f));
        CopyOut(ev.eval(y), out);
    });
}

// Backward of F::LookupFaces w.r.t. vtx_attr (exact adjacency gather)
int refh_lookup_faces_bwd(const float* gy, uint32_t n_comp,
                          const float* faces, uint32_t n_faces,
                          const float* vtx_faces, uint32_t n_verts,
                          uint32_t max_deg, uint32_t corner, float* out) {
    return Guard([&] {
        Variable attr(VecOf(n_comp), {n_verts, 1});
        Variable vf(VEC3, {n_faces, 1});
        Variable vvf(FLOAT, {n_verts, max_deg});
        Variable vgy(VecOf(n_comp), {n_faces, 1});
        Variable y = F::LookupFaces(attr, vf, vvf, corner);
        Variable g = y.getCreator().buildBwd(vgy, 0);
        CpuEvaluator ev;
        ev.bind(vf, Tensor(VEC3, {n_faces, 1}, faces));
        ev.bind(vvf, Tensor(FLOAT, {n_verts, max_deg}, vtx_faces));
        ev.bind(vgy, Tensor(VecOf(n_comp), {n_faces, 1}, gy));
        CopyOut(ev.eval(g), out);
    });
}

// VertexFacesTex: returns max degree in *deg_out; writes V*deg floats when
// `out` is non-null and `cap` >= V*deg
int refh_vertex_faces_tex(const float* faces, uint32_t n_faces,
                          uint32_t n_verts, uint32_t* deg_out, float* out,
                          uint32_t cap) {
    return Guard([&] {
        CpuImage fi(n_faces, 1, 3);
        std::memcpy(fi.data.data(), faces, sizeof(float) * 3 * n_faces);
        const CpuImage t = VertexFacesTex(fi, n_verts);
        *deg_out = t.height;
        if (out && cap >= t.data.size()) {
            std::memcpy(out, t.data.data(), t.data.size() * sizeof(float));
        }
    });
}

// GenerateIcosphere (examples/common/geometry_utils.cpp): counts only when
// pos/faces are null
int refh_icosphere(uint32_t level, uint32_t* n_verts, uint32_t* n_faces,
                   float* pos, float* faces) {
    return Guard([&] {
        const dressi_examples::Mesh m =
                dressi_examples::GenerateIcosphere(level);
        *n_verts = m.pos.width;
        *n_faces = m.faces.width;
        if (pos) {
            std::memcpy(pos, m.pos.data.data(),
                        m.pos.data.size() * sizeof(float));
        }
        if (faces) {
            std::memcpy(faces, m.faces.data.data(),
                        m.faces.data.size() * sizeof(float));
        }
    });
}

// GenerateUvSphere (examples/common/geometry_utils.cpp)
int refh_uv_sphere(uint32_t stacks, uint32_t slices, uint32_t* n_verts,
                   uint32_t* n_faces, float* pos, float* uv, float* faces) {
    return Guard([&] {
        const dressi_examples::Mesh m =
                dressi_examples::GenerateUvSphere(stacks, slices);
        *n_verts = m.pos.width;
        *n_faces = m.faces.width;
        if (pos) {
            std::memcpy(pos, m.pos.data.data(),
                        m.pos.data.size() * sizeof(float));
        }
        if (uv) {
            std::memcpy(uv, m.uv.data.data(),
                        m.uv.data.size() * sizeof(float));
        }
        if (faces) {
            std::memcpy(faces, m.faces.data.data(),
                        m.faces.data.size() * sizeof(float));
        }
    });
}

// The HardSoftRas silhouette fit of the reference example (technique
// hardsoftras, peels = 1, no regularizers), run on the reference's
// CpuEvaluator with DressiAD's end-of-frame copy-back semantics:
// per iteration every root is evaluated from the pre-update leaves, then
// pos/m/v/t are overwritten by their updated values.
//
//   pos0 {V,3}, faces {F,3} (float ids), tgt_pos {Vt,3}, tgt_faces {Ft,3},
//   mvps N x 16 column-major. Outputs (all nullable):
//   out_pos/m/v {V,3}, out_t {1}, out_loss {iters}: sum of the loss image,
//   out_grad0 {V,3}: d loss / d pos at iteration 0, out_pred0 {N,S,S},
//   out_target {N,S,S}, out_rs0 {N,S,S,4}: RasterizeSoft at iteration 0,
//   out_lossimg0 {S,S}.
// Depth peels of the HardSoftRas graph built by refh_hsr_fit (the example's
// --peels option, run.cpp:307); 1 unless set.
static uint32_t g_peels = 1;

int refh_set_peels(uint32_t peels) {
    g_peels = peels < 1 ? 1 : peels;
    return 0;
}

int refh_hsr_fit(const float* pos0, uint32_t n_verts, const float* faces,
                 uint32_t n_faces, const float* tgt_pos, uint32_t n_tverts,
                 const float* tgt_faces, uint32_t n_tfaces, const float* mvps,
                 uint32_t n_views, uint32_t screen_px, float radius_px,
                 uint32_t samples, float lr, uint32_t iters, float* out_pos,
                 float* out_m, float* out_v, float* out_t, float* out_loss,
                 float* out_grad0, float* out_pred0, float* out_target,
                 float* out_rs0, float* out_lossimg0) {
    return Guard([&] {
        const ImgSize screen = {screen_px, screen_px};
        CpuImage s_faces_img(n_faces, 1, 3);
        std::memcpy(s_faces_img.data.data(), faces,
                    sizeof(float) * 3 * n_faces);
        const CpuImage s_vf_img = VertexFacesTex(s_faces_img, n_verts);

        Variable b_ones(FLOAT, {n_tverts, 1});
        Variable b_faces_i(IVEC3, {n_tfaces, 1});
        Variable s_faces_f(VEC3, {n_faces, 1});
        Variable s_vtx_faces(FLOAT, s_vf_img.getImgSize());
        Variable s_face_id(FLOAT, {n_faces * 3, 1});
        Variable s_faces_soft(IVEC3, {n_faces, 1});
        Variable pos(VEC3, {n_verts, 1});
        Variable adam_m(VEC3, {n_verts, 1});
        Variable adam_v(VEC3, {n_verts, 1});
        Variable adam_t(FLOAT, {1, 1});

        const float sigma_scale = 7.f / radius_px;
        std::vector<Variable> rs_vars;
        const auto build_pred = [&](const Variable& clip_v) -> Variable {
            Variable soft_clip =
                    F::SoftClip(clip_v, s_faces_f, screen, radius_px);
            Variable tri0 = F::LookupFaces(clip_v, s_faces_f, s_vtx_faces, 0);
            Variable tri1 = F::LookupFaces(clip_v, s_faces_f, s_vtx_faces, 1);
            Variable tri2 = F::LookupFaces(clip_v, s_faces_f, s_vtx_faces, 2);
            Variable pc = F::ScreenCoord(screen);
            Variable zero = F::Float(0.f);
            Variable one = F::Float(1.f);
            const auto soft_prob = [&](const Variable& idx) {
                Variable mask = F::Greater(idx, F::Float(0.5f));
                const auto fetch = [&](const Variable& tri) {
                    return F::FaceFetch(tri, idx, tri0, tri1, tri2, adam_t,
                                        radius_px, samples);
                };
                const auto screen_of = [&](const Variable& c) {
                    Variable w = F::GetW(c) + (1.f - mask);
                    Variable sx = (F::GetX(c) / w * 0.5f + 0.5f) *
                                  float(screen.w);
                    Variable sy = (F::GetY(c) / w * 0.5f + 0.5f) *
                                  float(screen.h);
                    return F::Vec2(sx, sy);
                };
                Variable s0 = screen_of(fetch(tri0));
                Variable s1 = screen_of(fetch(tri1));
                Variable s2 = screen_of(fetch(tri2));
                const auto edge_dist = [&](const Variable& a,
                                           const Variable& b) {
                    Variable e = b - a;
                    Variable t = F::Clamp(F::Dot(pc - a, e) /
                                                  (F::Dot(e, e) + 1e-12f),
                                          zero, one);
                    Variable dd = pc - (a + t * e);
                    return F::Sqrt(F::Dot(dd, dd) + 1e-12f);
                };
                const auto edge_cross = [&](const Variable& a,
                                            const Variable& b) {
                    Variable e = b - a;
                    return F::GetX(e) * (F::GetY(pc) - F::GetY(a)) -
                           F::GetY(e) * (F::GetX(pc) - F::GetX(a));
                };
                Variable dmin = F::Min(F::Min(edge_dist(s0, s1),
                                              edge_dist(s1, s2)),
                                       edge_dist(s2, s0));
                Variable cr0 = edge_cross(s0, s1);
                Variable cr1 = edge_cross(s1, s2);
                Variable cr2 = edge_cross(s2, s0);
                Variable inside =
                        F::Min(F::Step(zero, cr0) * F::Step(zero, cr1) *
                                               F::Step(zero, cr2) +
                                       F::Step(zero, -cr0) *
                                               F::Step(zero, -cr1) *
                                               F::Step(zero, -cr2),
                               one);
                Variable dist = (inside * 2.f - 1.f) * dmin;
                return mask * F::Sigmoid(dist * sigma_scale);
            };
            // Alg. 2 depth peeling (run.cpp:302-343): peel k rejects
            // fragments at or in front of peel k - 1's shifted depth
            Variable one_minus = one;
            Variable prev_shift(nullptr);
            Variable hard(nullptr);
            for (uint32_t peel = 0; peel < g_peels; peel++) {
                Variable rs = F::StopGradient(
                        peel == 0 ? F::RasterizeSoft(soft_clip, s_face_id,
                                                     s_faces_soft, clip_v,
                                                     s_faces_f, s_vtx_faces,
                                                     screen, radius_px)
                                  : F::RasterizeSoft(soft_clip, s_face_id,
                                                     s_faces_soft, clip_v,
                                                     s_faces_f, s_vtx_faces,
                                                     prev_shift, screen,
                                                     radius_px));
                if (peel == 0) {
                    rs_vars.push_back(rs);
                }
                Variable dist_c = F::GetX(rs);
                Variable cov = F::GetW(rs);
                Variable ge = F::Step(zero, dist_c);
                prev_shift =
                        cov * (ge * (F::Clamp(F::GetZ(rs), zero, one) * 0.5f) +
                               (1.f - ge) *
                                       (F::Clamp(-dist_c * (1.f / radius_px),
                                                 zero, one) *
                                                0.5f +
                                        0.5f));
                Variable idx = (F::GetY(rs) + 1.f) * cov;
                one_minus = one_minus * (1.f - soft_prob(idx));
                if (peel == 0) {
                    hard = cov * ge;
                }
            }
            Variable soft_sil = 1.f - one_minus;
            return F::Max(hard, soft_sil);
        };

        Variables targets, preds, view_losses;
        std::vector<Variable> tgt_clips;
        for (uint32_t v = 0; v < n_views; v++) {
            tgt_clips.emplace_back(VEC4, ImgSize{n_tverts, 1});
            targets.push_back(F::StopGradient(F::Rasterize(
                    tgt_clips.back(), b_ones, b_faces_i, screen)));
            preds.push_back(build_pred(ClipOf(pos, mvps + 16 * v)));
            Variable diff = targets[v] - preds[v];
            view_losses.push_back(diff * diff *
                                  (1.f / float(screen.w * screen.h)));
        }
        Variable loss = F::SumPixelWise(view_losses);
        Variable pos_mut = pos;
        pos_mut.setRequiresGradRecursively();

        auto [xs, gxs] = BuildBackward(loss);
        DRESSI_CHECK(xs.size() == 1 && xs[0] == pos,
                     "expected pos as the only requires-grad leaf");
        const Variable g = gxs[0];
        const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
        Variable t_new = adam_t + 1.f;
        Variable m_new = adam_m * b1 + g * (1.f - b1);
        Variable v_new = adam_v * b2 + g * g * (1.f - b2);
        Variable bc1 = 1.f - F::Pow(F::Float(b1), t_new);
        Variable bc2 = 1.f - F::Pow(F::Float(b2), t_new);
        Variable step = (m_new / bc1) / (F::Sqrt(v_new / bc2) + eps) * lr;
        Variable pos_new = pos - step;

        // Static leaves
        std::vector<float> ones(n_tverts, 1.f);
        CpuTensor t_b_ones = Tensor(FLOAT, {n_tverts, 1}, ones.data());
        CpuTensor t_b_faces = Tensor(IVEC3, {n_tfaces, 1}, tgt_faces);
        CpuTensor t_s_faces = Tensor(VEC3, {n_faces, 1}, faces);
        CpuTensor t_vf = Tensor(FLOAT, s_vf_img.getImgSize(),
                                s_vf_img.data.data());
        std::vector<float> fid_img(size_t(n_faces) * 3), fsoft(n_faces * 3);
        for (uint32_t f = 0; f < n_faces; f++) {
            for (uint32_t k = 0; k < 3; k++) {
                fid_img[f * 3 + k] = float(f);
                fsoft[f * 3 + k] = float(f * 3 + k);
            }
        }
        CpuTensor t_fid = Tensor(FLOAT, {n_faces * 3, 1}, fid_img.data());
        CpuTensor t_fsoft = Tensor(IVEC3, {n_faces, 1}, fsoft.data());
        std::vector<CpuTensor> t_tgt_clips;
        for (uint32_t v = 0; v < n_views; v++) {
            const float* m = mvps + 16 * v;
            CpuTensor c = Fill(VEC4, {n_tverts, 1}, 0.f);
            for (uint32_t i = 0; i < n_tverts; i++) {
                const float p[4] = {tgt_pos[i * 3 + 0], tgt_pos[i * 3 + 1],
                                    tgt_pos[i * 3 + 2], 1.f};
                for (int row = 0; row < 4; row++) {
                    float acc = 0.f;
                    for (int k = 0; k < 4; k++) {
                        acc += m[k * 4 + row] * p[k];
                    }
                    c.data[size_t(i) * 4 + row] = acc;
                }
            }
            t_tgt_clips.push_back(std::move(c));
        }

        CpuTensor t_pos = Tensor(VEC3, {n_verts, 1}, pos0);
        CpuTensor t_m = Fill(VEC3, {n_verts, 1}, 0.f);
        CpuTensor t_v = Fill(VEC3, {n_verts, 1}, 0.f);
        CpuTensor t_t = Fill(FLOAT, {1, 1}, 0.f);
        for (uint32_t it = 0; it < iters; it++) {
            CpuEvaluator ev;
            ev.bind(b_ones, t_b_ones);
            ev.bind(b_faces_i, t_b_faces);
            ev.bind(s_faces_f, t_s_faces);
            ev.bind(s_vtx_faces, t_vf);
            ev.bind(s_face_id, t_fid);
            ev.bind(s_faces_soft, t_fsoft);
            for (uint32_t v = 0; v < n_views; v++) {
                ev.bind(tgt_clips[v], t_tgt_clips[v]);
            }
            ev.bind(pos, t_pos);
            ev.bind(adam_m, t_m);
            ev.bind(adam_v, t_v);
            ev.bind(adam_t, t_t);

            const CpuTensor li = ev.eval(loss);
            if (out_loss) {
                double s = 0.0;
                for (float x : li.data) {
                    s += x;
                }
                out_loss[it] = float(s);
            }
            if (it == 0) {
                CopyOut(li, out_lossimg0);
                if (out_grad0) {
                    CopyOut(ev.eval(g), out_grad0);
                }
                const size_t px = size_t(screen.w) * screen.h;
                for (uint32_t v = 0; v < n_views; v++) {
                    if (out_pred0) {
                        CopyOut(ev.eval(preds[v]), out_pred0 + v * px);
                    }
                    if (out_target) {
                        CopyOut(ev.eval(targets[v]), out_target + v * px);
                    }
                    if (out_rs0) {
                        CopyOut(ev.eval(rs_vars[v]), out_rs0 + v * px * 4);
                    }
                }
            }
            CpuTensor n_pos = ev.eval(pos_new);
            CpuTensor n_m = ev.eval(m_new);
            CpuTensor n_v = ev.eval(v_new);
            CpuTensor n_t = ev.eval(t_new);
            t_pos = std::move(n_pos);
            t_m = std::move(n_m);
            t_v = std::move(n_v);
            t_t = std::move(n_t);
        }
        CopyOut(t_pos, out_pos);
        CopyOut(t_m, out_m);
        CopyOut(t_v, out_v);
        CopyOut(t_t, out_t);
    });
}

// F::AntiAlias forward: img {w,h} n_comp, tri {w,h} FLOAT (face + 1),
// clip {V,1} VEC4, faces {F,1} VEC3, vtx_faces {V,deg}
int refh_antialias(const float* img, uint32_t n_comp, const float* tri,
                   const float* clip, uint32_t n_verts, const float* faces,
                   uint32_t n_faces, const float* vtx_faces, uint32_t max_deg,
                   uint32_t w, uint32_t h, float* out) {
    return Guard([&] {
        Variable vimg(VecOf(n_comp), {w, h});
        Variable vtri(FLOAT, {w, h});
        Variable vc(VEC4, {n_verts, 1});
        Variable vf(VEC3, {n_faces, 1});
        Variable vvf(FLOAT, {n_verts, max_deg});
        Variable vs(FLOAT, {1, 1});
        Variable y = F::AntiAlias(vimg, vtri, vc, vf, vvf, vs, 0);
        CpuEvaluator ev;
        ev.bind(vimg, Tensor(VecOf(n_comp), {w, h}, img));
        ev.bind(vtri, Tensor(FLOAT, {w, h}, tri));
        ev.bind(vc, Tensor(VEC4, {n_verts, 1}, clip));
        ev.bind(vf, Tensor(VEC3, {n_faces, 1}, faces));
        ev.bind(vvf, Tensor(FLOAT, {n_verts, max_deg}, vtx_faces));
        ev.bind(vs, Fill(FLOAT, {1, 1}, 0.f));
        CopyOut(ev.eval(y), out);
    });
}

// Backward of F::AntiAlias w.r.t. img (AntiAliasBwdImg) and w.r.t. vtx_clip
// (AntiAliasBwdVtx: n > 0 -> ColSum of the {V,deg} wide partials, written to
// out_wide / out_vtx; n = 0 -> the exact {V,1} scatter in out_vtx), from the
// op's own backward generator. Any output may be null.
int refh_antialias_bwd(const float* gy, const float* img, uint32_t n_comp,
                       const float* tri, const float* clip, uint32_t n_verts,
                       const float* faces, uint32_t n_faces, const float* vtx_faces,
                       uint32_t max_deg, float seed, uint32_t n_samples, uint32_t w,
                       uint32_t h, float* out_img, float* out_wide, float* out_vtx) {
    return Guard([&] {
        Variable vimg(VecOf(n_comp), {w, h});
        Variable vtri(FLOAT, {w, h});
        Variable vc(VEC4, {n_verts, 1});
        Variable vf(VEC3, {n_faces, 1});
        Variable vvf(FLOAT, {n_verts, max_deg});
        Variable vs(FLOAT, {1, 1});
        Variable vgy(VecOf(n_comp), {w, h});
        Variable y = F::AntiAlias(vimg, vtri, vc, vf, vvf, vs, n_samples);
        Variable g_img = y.getCreator().buildBwd(vgy, 0);
        Variable g_vtx = y.getCreator().buildBwd(vgy, 2);
        CpuEvaluator ev;
        ev.bind(vimg, Tensor(VecOf(n_comp), {w, h}, img));
        ev.bind(vtri, Tensor(FLOAT, {w, h}, tri));
        ev.bind(vc, Tensor(VEC4, {n_verts, 1}, clip));
        ev.bind(vf, Tensor(VEC3, {n_faces, 1}, faces));
        ev.bind(vvf, Tensor(FLOAT, {n_verts, max_deg}, vtx_faces));
        ev.bind(vs, Fill(FLOAT, {1, 1}, seed));
        ev.bind(vgy, Tensor(VecOf(n_comp), {w, h}, gy));
        if (out_img) {
            CopyOut(ev.eval(g_img), out_img);
        }
        if (out_vtx) {
            CopyOut(ev.eval(g_vtx), out_vtx);
        }
        if (out_wide && n_samples > 0) {
            CopyOut(ev.eval(g_vtx.getCreator().getInputVars()[0]), out_wide);
        }
    });
}

// The AA silhouette fit of the reference example (technique aa, no
// regularizers): same driver and outputs as refh_hsr_fit, with out_tri0
// {N,S,S} the RasterizeFaceId images of iteration 0 in place of out_rs0.
int refh_aa_fit(const float* pos0, uint32_t n_verts, const float* faces,
                uint32_t n_faces, const float* tgt_pos, uint32_t n_tverts,
                const float* tgt_faces, uint32_t n_tfaces, const float* mvps,
                uint32_t n_views, uint32_t screen_px, uint32_t samples, float lr,
                uint32_t iters, float* out_pos, float* out_m, float* out_v,
                float* out_t, float* out_loss, float* out_grad0, float* out_pred0,
                float* out_target, float* out_tri0, float* out_lossimg0) {
    return Guard([&] {
        const ImgSize screen = {screen_px, screen_px};
        CpuImage s_faces_img(n_faces, 1, 3);
        std::memcpy(s_faces_img.data.data(), faces, sizeof(float) * 3 * n_faces);
        const CpuImage s_vf_img = VertexFacesTex(s_faces_img, n_verts);
        CpuImage b_faces_img(n_tfaces, 1, 3);
        std::memcpy(b_faces_img.data.data(), tgt_faces, sizeof(float) * 3 * n_tfaces);
        const CpuImage b_vf_img = VertexFacesTex(b_faces_img, n_tverts);

        Variable b_ones(FLOAT, {n_tverts, 1});
        Variable b_faces_i(IVEC3, {n_tfaces, 1});
        Variable b_faces_f(VEC3, {n_tfaces, 1});
        Variable b_vtx_faces(FLOAT, b_vf_img.getImgSize());
        Variable s_ones(FLOAT, {n_verts, 1});
        Variable s_faces_i(IVEC3, {n_faces, 1});
        Variable s_faces_f(VEC3, {n_faces, 1});
        Variable s_vtx_faces(FLOAT, s_vf_img.getImgSize());
        Variable pos(VEC3, {n_verts, 1});
        Variable adam_m(VEC3, {n_verts, 1});
        Variable adam_v(VEC3, {n_verts, 1});
        Variable adam_t(FLOAT, {1, 1});
        Variable zero_seed(FLOAT, {1, 1});

        std::vector<Variable> tri_vars;
        const auto build_pred = [&](const Variable& clip_v) -> Variable {
            Variable mask = F::Rasterize(clip_v, s_ones, s_faces_i, screen);
            Variable tri = F::RasterizeFaceId(clip_v, s_ones, s_faces_i, screen);
            tri_vars.push_back(tri);
            return F::AntiAlias(mask, tri, clip_v, s_faces_f, s_vtx_faces, adam_t, samples);
        };
        const auto build_target = [&](const Variable& tgt_clip) -> Variable {
            Variable t_mask = F::Rasterize(tgt_clip, b_ones, b_faces_i, screen);
            Variable t_tri = F::RasterizeFaceId(tgt_clip, b_ones, b_faces_i, screen);
            return F::StopGradient(F::AntiAlias(t_mask, t_tri, tgt_clip, b_faces_f,
                                                b_vtx_faces, zero_seed, 0));
        };
        Variables targets, preds, view_losses;
        std::vector<Variable> tgt_clips;
        for (uint32_t v = 0; v < n_views; v++) {
            tgt_clips.emplace_back(VEC4, ImgSize{n_tverts, 1});
            targets.push_back(build_target(tgt_clips.back()));
            preds.push_back(build_pred(ClipOf(pos, mvps + 16 * v)));
            Variable diff = targets[v] - preds[v];
            view_losses.push_back(diff * diff * (1.f / float(screen.w * screen.h)));
        }
        Variable loss = F::SumPixelWise(view_losses);
        Variable pos_mut = pos;
        pos_mut.setRequiresGradRecursively();

        auto [xs, gxs] = BuildBackward(loss);
        DRESSI_CHECK(xs.size() == 1 && xs[0] == pos,
                     "expected pos as the only requires-grad leaf");
        const Variable g = gxs[0];
        const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
        Variable t_new = adam_t + 1.f;
        Variable m_new = adam_m * b1 + g * (1.f - b1);
        Variable v_new = adam_v * b2 + g * g * (1.f - b2);
        Variable bc1 = 1.f - F::Pow(F::Float(b1), t_new);
        Variable bc2 = 1.f - F::Pow(F::Float(b2), t_new);
        Variable step = (m_new / bc1) / (F::Sqrt(v_new / bc2) + eps) * lr;
        Variable pos_new = pos - step;

        std::vector<float> b_ones_v(n_tverts, 1.f), s_ones_v(n_verts, 1.f);
        CpuTensor t_b_ones = Tensor(FLOAT, {n_tverts, 1}, b_ones_v.data());
        CpuTensor t_s_ones = Tensor(FLOAT, {n_verts, 1}, s_ones_v.data());
        CpuTensor t_b_faces = Tensor(IVEC3, {n_tfaces, 1}, tgt_faces);
        CpuTensor t_b_faces_f = Tensor(VEC3, {n_tfaces, 1}, tgt_faces);
        CpuTensor t_b_vf = Tensor(FLOAT, b_vf_img.getImgSize(), b_vf_img.data.data());
        CpuTensor t_s_faces_i = Tensor(IVEC3, {n_faces, 1}, faces);
        CpuTensor t_s_faces = Tensor(VEC3, {n_faces, 1}, faces);
        CpuTensor t_vf = Tensor(FLOAT, s_vf_img.getImgSize(), s_vf_img.data.data());
        std::vector<CpuTensor> t_tgt_clips;
        for (uint32_t v = 0; v < n_views; v++) {
            const float* m = mvps + 16 * v;
            CpuTensor c = Fill(VEC4, {n_tverts, 1}, 0.f);
            for (uint32_t i = 0; i < n_tverts; i++) {
                const float p[4] = {tgt_pos[i * 3 + 0], tgt_pos[i * 3 + 1],
                                    tgt_pos[i * 3 + 2], 1.f};
                for (int row = 0; row < 4; row++) {
                    float acc = 0.f;
                    for (int k = 0; k < 4; k++) {
                        acc += m[k * 4 + row] * p[k];
                    }
                    c.data[size_t(i) * 4 + row] = acc;
                }
            }
            t_tgt_clips.push_back(std::move(c));
        }

        CpuTensor t_pos = Tensor(VEC3, {n_verts, 1}, pos0);
        CpuTensor t_m = Fill(VEC3, {n_verts, 1}, 0.f);
        CpuTensor t_v = Fill(VEC3, {n_verts, 1}, 0.f);
        CpuTensor t_t = Fill(FLOAT, {1, 1}, 0.f);
        for (uint32_t it = 0; it < iters; it++) {
            CpuEvaluator ev;
            ev.bind(b_ones, t_b_ones);
            ev.bind(b_faces_i, t_b_faces);
            ev.bind(b_faces_f, t_b_faces_f);
            ev.bind(b_vtx_faces, t_b_vf);
            ev.bind(s_ones, t_s_ones);
            ev.bind(s_faces_i, t_s_faces_i);
            ev.bind(s_faces_f, t_s_faces);
            ev.bind(s_vtx_faces, t_vf);
            ev.bind(zero_seed, Fill(FLOAT, {1, 1}, 0.f));
            for (uint32_t v = 0; v < n_views; v++) {
                ev.bind(tgt_clips[v], t_tgt_clips[v]);
            }
            ev.bind(pos, t_pos);
            ev.bind(adam_m, t_m);
            ev.bind(adam_v, t_v);
            ev.bind(adam_t, t_t);

            const CpuTensor li = ev.eval(loss);
            if (out_loss) {
                double acc = 0.0;
                for (float x : li.data) {
                    acc += x;
                }
                out_loss[it] = float(acc);
            }
            if (it == 0) {
                CopyOut(li, out_lossimg0);
                if (out_grad0) {
                    CopyOut(ev.eval(g), out_grad0);
                }
                const size_t px = size_t(screen.w) * screen.h;
                for (uint32_t v = 0; v < n_views; v++) {
                    if (out_pred0) {
                        CopyOut(ev.eval(preds[v]), out_pred0 + v * px);
                    }
                    if (out_target) {
                        CopyOut(ev.eval(targets[v]), out_target + v * px);
                    }
                    if (out_tri0) {
                        CopyOut(ev.eval(tri_vars[v]), out_tri0 + v * px);
                    }
                }
            }
            CpuTensor n_pos = ev.eval(pos_new);
            CpuTensor n_m = ev.eval(m_new);
            CpuTensor n_v = ev.eval(v_new);
            CpuTensor n_t = ev.eval(t_new);
            t_pos = std::move(n_pos);
            t_m = std::move(n_m);
            t_v = std::move(n_v);
            t_t = std::move(n_t);
        }
        CopyOut(t_pos, out_pos);
        CopyOut(t_m, out_m);
        CopyOut(t_v, out_v);
        CopyOut(t_t, out_t);
    });
}

// TextureBilinear (src/core/f_ops.cpp:2736-2780) through the evaluator:
// tex {tw,th} x n_comp, uv {uw,uh} VEC2 -> out {uw,uh} x n_comp.
int refh_texture_bilinear(const float* tex, uint32_t tw, uint32_t th, uint32_t n_comp,
                          const float* uv, uint32_t uw, uint32_t uh, float* out) {
    return Guard([&] {
        Variable t(VecOf(n_comp), {tw, th});
        Variable u(VEC2, {uw, uh});
        Variable iv(VEC4, {tw, th});
        Variable y = F::TextureBilinear(t, u, iv);
        CpuEvaluator ev;
        ev.bind(t, Tensor(VecOf(n_comp), {tw, th}, tex));
        ev.bind(u, Tensor(VEC2, {uw, uh}, uv));
        ev.bind(iv, Fill(VEC4, {tw, th}, 0.f));
        CopyOut(ev.eval(y), out);
    });
}

// GatherByInverseUVBilinear (src/core/f_ops.cpp:2650-2732), reached as the
// backward of TextureBilinear for the image loss TextureBilinear(tex) * gy
// (its seed 1 gives the sampled image the gradient gy exactly):
// gy {sw,sh} x n_comp, inv_uv {tw,th} VEC4, uv {sw,sh} VEC2 -> {tw,th}.
int refh_gather_bilinear(const float* gy, uint32_t n_comp, uint32_t sw, uint32_t sh,
                         const float* inv_uv, uint32_t tw, uint32_t th, const float* uv,
                         float* out) {
    return Guard([&] {
        Variable t(VecOf(n_comp), {tw, th});
        Variable u(VEC2, {sw, sh});
        Variable iv(VEC4, {tw, th});
        Variable g(VecOf(n_comp), {sw, sh});
        Variable loss = F::TextureBilinear(t, u, iv) * g;
        Variable t_mut = t;
        t_mut.setRequiresGradRecursively();
        auto [xs, gxs] = BuildBackward(loss);
        DRESSI_CHECK(xs.size() == 1 && xs[0] == t, "expected the texture as the only leaf");
        CpuEvaluator ev;
        ev.bind(t, Fill(VecOf(n_comp), {tw, th}, 0.f));
        ev.bind(u, Tensor(VEC2, {sw, sh}, uv));
        ev.bind(iv, Tensor(VEC4, {tw, th}, inv_uv));
        ev.bind(g, Tensor(VecOf(n_comp), {sw, sh}, gy));
        CopyOut(ev.eval(gxs[0]), out);
    });
}

// The C3 texture fit: the graph of examples/texture_optimization/run.cpp:
// 112-145 with TextureBilinear, an RGBA texture, the RGB L2 image loss and
// the silhouette example's in-graph Adam (run.cpp:404-437), on the
// reference's CpuEvaluator with DressiAD's copy-back. Per iteration `it` the
// host sends, per view v, clip = TransformToClip(pos, mvp) and
// inv_uv_attr = ScreenAttr(clip) with mvp = mvps[(it % n_sets) * n_views + v]
// (the example's per-iteration sendImg of moving cameras).
//   pos {V,3}, uv {V,2}, faces {F,3}, gt_tex / tex0 {tw,th} VEC4.
//   Outputs (nullable): out_tex/m/v {T,4}, out_t, out_loss {iters} (sum of
//   the loss image), out_grad0 {T,4}, out_pred0 / out_target0 {N,S,S,4},
//   out_lossimg0 {S,S,4}, out_uv0 {N,S,S,2}, out_invuv0 {N,T,4}.
int refh_tex_fit(const float* pos, uint32_t n_verts, const float* uv, const float* faces,
                 uint32_t n_faces, const float* mvps, uint32_t n_sets, uint32_t n_views,
                 uint32_t screen_px, uint32_t tex_w, uint32_t tex_h, const float* gt_tex,
                 const float* tex0, float lr, uint32_t iters, float* out_tex, float* out_m,
                 float* out_v, float* out_t, float* out_loss, float* out_grad0,
                 float* out_pred0, float* out_target0, float* out_lossimg0, float* out_uv0,
                 float* out_invuv0) {
    return Guard([&] {
        const ImgSize screen = {screen_px, screen_px};
        const ImgSize tex_size = {tex_w, tex_h};
        Variable vtx_uv(VEC2, {n_verts, 1});
        Variable faces_v(IVEC3, {n_faces, 1});
        Variable uv_clip(VEC4, {n_verts, 1});
        Variable ones(FLOAT, {n_verts, 1});
        Variable gt_tex_v(VEC4, tex_size);
        Variable tex(VEC4, tex_size);
        Variable adam_m(VEC4, tex_size);
        Variable adam_v(VEC4, tex_size);
        Variable adam_t(FLOAT, {1, 1});
        std::vector<Variable> clips, attrs, preds, targets, uvs, invs;
        Variables view_losses;
        const float c = 1.f / float(screen.w * screen.h);
        for (uint32_t v = 0; v < n_views; v++) {
            clips.emplace_back(VEC4, ImgSize{n_verts, 1});
            attrs.emplace_back(VEC4, ImgSize{n_verts, 1});
            Variable g_uv = F::Rasterize(clips[v], vtx_uv, faces_v, screen);
            Variable g_mask = F::Rasterize(clips[v], ones, faces_v, screen);
            Variable inv_uv = F::Rasterize(uv_clip, attrs[v], faces_v, tex_size);
            uvs.push_back(g_uv);
            invs.push_back(inv_uv);
            targets.push_back(g_mask * F::TextureBilinear(gt_tex_v, g_uv, inv_uv));
            preds.push_back(g_mask * F::TextureBilinear(tex, g_uv, inv_uv));
            Variable diff = F::StopGradient(targets[v]) - preds[v];
            view_losses.push_back(diff * diff * F::Vec4(c, c, c, 0.f));
        }
        Variable loss = F::SumPixelWise(view_losses);
        Variable tex_mut = tex;
        tex_mut.setRequiresGradRecursively();
        auto [xs, gxs] = BuildBackward(loss);
        DRESSI_CHECK(xs.size() == 1 && xs[0] == tex, "expected the texture as the only leaf");
        const Variable g = gxs[0];
        const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
        Variable t_new = adam_t + 1.f;
        Variable m_new = adam_m * b1 + g * (1.f - b1);
        Variable v_new = adam_v * b2 + g * g * (1.f - b2);
        Variable bc1 = 1.f - F::Pow(F::Float(b1), t_new);
        Variable bc2 = 1.f - F::Pow(F::Float(b2), t_new);
        Variable step = (m_new / bc1) / (F::Sqrt(v_new / bc2) + eps) * lr;
        Variable tex_new = tex - step;

        CpuImage uv_img(n_verts, 1, 2);
        std::memcpy(uv_img.data.data(), uv, sizeof(float) * 2 * n_verts);
        const CpuImage uv_clip_img = UvAsClip(uv_img);
        std::vector<float> ones_v(n_verts, 1.f);
        const size_t ntx = size_t(tex_w) * tex_h;
        CpuTensor t_tex = Tensor(VEC4, tex_size, tex0);
        CpuTensor t_m = Fill(VEC4, tex_size, 0.f);
        CpuTensor t_v = Fill(VEC4, tex_size, 0.f);
        CpuTensor t_t = Fill(FLOAT, {1, 1}, 0.f);
        for (uint32_t it = 0; it < iters; it++) {
            CpuEvaluator ev;
            ev.bind(vtx_uv, Tensor(VEC2, {n_verts, 1}, uv));
            ev.bind(faces_v, Tensor(IVEC3, {n_faces, 1}, faces));
            ev.bind(uv_clip, Tensor(VEC4, {n_verts, 1}, uv_clip_img.data.data()));
            ev.bind(ones, Tensor(FLOAT, {n_verts, 1}, ones_v.data()));
            ev.bind(gt_tex_v, Tensor(VEC4, tex_size, gt_tex));
            const float* set = mvps + size_t(it % n_sets) * n_views * 16;
            for (uint32_t v = 0; v < n_views; v++) {
                const float* m = set + 16 * v;
                CpuImage clip_img(n_verts, 1, 4);
                for (uint32_t i = 0; i < n_verts; i++) {
                    const float p[4] = {pos[i * 3 + 0], pos[i * 3 + 1], pos[i * 3 + 2], 1.f};
                    for (int row = 0; row < 4; row++) {
                        float acc = 0.f;
                        for (int k = 0; k < 4; k++) {
                            acc += m[k * 4 + row] * p[k];
                        }
                        clip_img.at(i, 0, uint32_t(row)) = acc;
                    }
                }
                const CpuImage attr_img = ScreenAttr(clip_img, screen);
                ev.bind(clips[v], Tensor(VEC4, {n_verts, 1}, clip_img.data.data()));
                ev.bind(attrs[v], Tensor(VEC4, {n_verts, 1}, attr_img.data.data()));
            }
            ev.bind(tex, t_tex);
            ev.bind(adam_m, t_m);
            ev.bind(adam_v, t_v);
            ev.bind(adam_t, t_t);
            const CpuTensor li = ev.eval(loss);
            if (out_loss) {
                double acc = 0.0;
                for (float x : li.data) {
                    acc += x;
                }
                out_loss[it] = float(acc);
            }
            if (it == 0) {
                CopyOut(li, out_lossimg0);
                if (out_grad0) {
                    CopyOut(ev.eval(g), out_grad0);
                }
                const size_t px = size_t(screen.w) * screen.h;
                for (uint32_t v = 0; v < n_views; v++) {
                    if (out_pred0) CopyOut(ev.eval(preds[v]), out_pred0 + v * px * 4);
                    if (out_target0) CopyOut(ev.eval(targets[v]), out_target0 + v * px * 4);
                    if (out_uv0) CopyOut(ev.eval(uvs[v]), out_uv0 + v * px * 2);
                    if (out_invuv0) CopyOut(ev.eval(invs[v]), out_invuv0 + v * ntx * 4);
                }
            }
            CpuTensor n_tex = ev.eval(tex_new);
            CpuTensor n_m = ev.eval(m_new);
            CpuTensor n_v = ev.eval(v_new);
            CpuTensor n_t = ev.eval(t_new);
            t_tex = std::move(n_tex);
            t_m = std::move(n_m);
            t_v = std::move(n_v);
            t_t = std::move(n_t);
        }
        CopyOut(t_tex, out_tex);
        CopyOut(t_m, out_m);
        CopyOut(t_v, out_v);
        CopyOut(t_t, out_t);
    });
}

// ---------------------------------------------------------------------------
// PBR / IBL ops (src/core/f_ops.cpp:2785-3415, src/core/ibl.cpp) and the C5
// material + environment fit (examples/common/pbr_graph.cpp)
// ---------------------------------------------------------------------------

}  // extern "C"

namespace {

// VJP of `y = op(x)` w.r.t. x for the image loss y * gy (seed 1 per pixel
// gives y the gradient gy exactly).
template <typename Op>
CpuTensor VjpOf(Op op, VType xt, ImgSize xs, const float* x, VType yt, ImgSize ys,
                const float* gy) {
    Variable xv(xt, xs);
    Variable g(yt, ys);
    Variable loss = op(xv) * g;
    Variable x_mut = xv;
    x_mut.setRequiresGradRecursively();
    auto [leaves, gxs] = BuildBackward(loss);
    DRESSI_CHECK(leaves.size() == 1 && leaves[0] == xv, "expected one leaf");
    CpuEvaluator ev;
    ev.bind(xv, Tensor(xt, xs, x));
    ev.bind(g, Tensor(yt, ys, gy));
    return ev.eval(gxs[0]);
}

template <typename Op>
CpuTensor FwdOf(Op op, VType xt, ImgSize xs, const float* x) {
    Variable xv(xt, xs);
    Variable y = op(xv);
    CpuEvaluator ev;
    ev.bind(xv, Tensor(xt, xs, x));
    return ev.eval(y);
}

}  // namespace

extern "C" {

// EquirectSample (f_ops.cpp:2921-2964): map {mw,mh} x n, dir {dw,dh} VEC3.
// gy != nullptr: its VJP w.r.t. the map (EquirectSampleBwd + TileSum,
// f_ops.cpp:2823-2919) for gy {dw,dh} x n, written to out {mw,mh} x n.
int refh_equirect_sample(const float* map, uint32_t mw, uint32_t mh, uint32_t n_comp,
                         const float* dir, uint32_t dw, uint32_t dh, const float* gy,
                         float* out) {
    return Guard([&] {
        Variable d(VEC3, {dw, dh});
        const auto op = [&](const Variable& m) { return F::EquirectSample(m, d); };
        Variable m(VecOf(n_comp), {mw, mh});
        Variable y = op(m);
        if (!gy) {
            CpuEvaluator ev;
            ev.bind(m, Tensor(VecOf(n_comp), {mw, mh}, map));
            ev.bind(d, Tensor(VEC3, {dw, dh}, dir));
            CopyOut(ev.eval(y), out);
            return;
        }
        Variable g(VecOf(n_comp), {dw, dh});
        Variable loss = y * g;
        Variable m_mut = m;
        m_mut.setRequiresGradRecursively();
        auto [leaves, gxs] = BuildBackward(loss);
        DRESSI_CHECK(leaves.size() == 1 && leaves[0] == m, "expected the map as the leaf");
        CpuEvaluator ev;
        ev.bind(m, Tensor(VecOf(n_comp), {mw, mh}, map));
        ev.bind(d, Tensor(VEC3, {dw, dh}, dir));
        ev.bind(g, Tensor(VecOf(n_comp), {dw, dh}, gy));
        CopyOut(ev.eval(gxs[0]), out);
    });
}

// AvgPool2x2 (f_ops.cpp:3411-3415) and its VJP: x {w,h} x n -> {w/2,h/2}.
int refh_avg_pool2x2(const float* x, uint32_t w, uint32_t h, uint32_t n_comp, const float* gy,
                     float* out) {
    return Guard([&] {
        const auto op = [](const Variable& v) { return F::AvgPool2x2(v); };
        const ImgSize half = {(w + 1) / 2, (h + 1) / 2};
        CopyOut(gy ? VjpOf(op, VecOf(n_comp), {w, h}, x, VecOf(n_comp), half, gy)
                   : FwdOf(op, VecOf(n_comp), {w, h}, x),
                out);
    });
}

// IrradianceConv (f_ops.cpp:3006-3087) env {sw,sh} -> {ow,oh}; with gy its
// VJP (IrradianceConvBwd, f_ops.cpp:2970-3004).
int refh_irradiance_conv(const float* env, uint32_t sw, uint32_t sh, uint32_t n_comp,
                         uint32_t ow, uint32_t oh, const float* gy, float* out) {
    return Guard([&] {
        const auto op = [&](const Variable& v) { return F::IrradianceConv(v, {ow, oh}); };
        CopyOut(gy ? VjpOf(op, VecOf(n_comp), {sw, sh}, env, VecOf(n_comp), {ow, oh}, gy)
                   : FwdOf(op, VecOf(n_comp), {sw, sh}, env),
                out);
    });
}

// PrefilterConv (f_ops.cpp:3264-3348, its normaliser PrefilterConvNorm
// :3166-3205) at `roughness`; with gy its VJP (PrefilterConvBwd :3207-3262).
int refh_prefilter_conv(const float* env, uint32_t sw, uint32_t sh, uint32_t n_comp,
                        uint32_t ow, uint32_t oh, float roughness, const float* gy,
                        float* out) {
    return Guard([&] {
        const auto op = [&](const Variable& v) {
            return F::PrefilterConv(v, {ow, oh}, roughness);
        };
        CopyOut(gy ? VjpOf(op, VecOf(n_comp), {sw, sh}, env, VecOf(n_comp), {ow, oh}, gy)
                   : FwdOf(op, VecOf(n_comp), {sw, sh}, env),
                out);
    });
}

// PrefilterEnv (f_ops.cpp:3089-3157), forward only.
int refh_prefilter_env(const float* env, uint32_t sw, uint32_t sh, uint32_t n_comp,
                       uint32_t ow, uint32_t oh, float roughness, uint32_t n_samples,
                       float* out) {
    return Guard([&] {
        const auto op = [&](const Variable& v) {
            return F::PrefilterEnv(v, {ow, oh}, roughness, n_samples);
        };
        CopyOut(FwdOf(op, VecOf(n_comp), {sw, sh}, env), out);
    });
}

// BrdfIntegrationLut (f_ops.cpp:3350-3409): {w,h} VEC2.
int refh_brdf_lut(uint32_t w, uint32_t h, uint32_t n_samples, float* out) {
    return Guard([&] {
        Variable y = F::BrdfIntegrationLut({w, h}, n_samples);
        CpuEvaluator ev;
        CopyOut(ev.eval(y), out);
    });
}

// The C5 split-sum PBR/IBL material + environment fit: per view the
// G-buffer of BuildPbrGBuffer and the shading of BuildPbrShade (normal
// mapping off; AO texture 1, emissive 0; the camera frame and light of
// examples/pbr_material_optimization/run.cpp:189-236), IBL maps from
// BuildIrradianceSample + BuildPrefEnvironmentSampleConv(env, levels) +
// BuildBrdfIntegrationMap (the env is optimized, so the differentiable
// prefilter), the L1 loss Mean(|StopGradient(target.mapped) - pred.mapped|)
// summed over views, and in-graph Adam on albedo, mr and env with a shared
// step counter; albedo / mr are clamped to [0,1] (run.cpp:285-288), the env
// to >= 0 (pbr_envmap_optimization/run.cpp:312-317). The target is the same
// graph with the ground-truth maps.
//   pos / normal {V,3}, uv {V,2}, faces {F,3}, mvps {N,16}, frames {N,12}
//   (cam_pos, cam_fwd, cam_right, cam_up), light {6} (pos, colour),
//   gt_albedo / gt_mr / albedo0 / mr0 {T,3}, gt_env / env0 {E,3}.
//   Outputs (nullable): out_albedo / out_mr {T,3}, out_env {E,3}, out_loss
//   {iters}, out_g_albedo0 / out_g_mr0 {T,3}, out_g_env0 {E,3} (gradients of
//   iteration 0), out_pred0 / out_target0 {N,S,S,3} (mapped), out_mask0
//   {N,S,S}.
int refh_pbr_fit(const float* pos, const float* normal, uint32_t n_verts, const float* uv,
                 const float* faces, uint32_t n_faces, const float* mvps, const float* frames,
                 const float* light, uint32_t n_views, uint32_t screen_px, uint32_t tex_w,
                 uint32_t tex_h, uint32_t env_w, uint32_t env_h, uint32_t levels,
                 const float* gt_albedo, const float* gt_mr, const float* gt_env,
                 const float* albedo0, const float* mr0, const float* env0, float lr,
                 uint32_t iters, float* out_albedo, float* out_mr, float* out_env,
                 float* out_loss, float* out_g_albedo0, float* out_g_mr0, float* out_g_env0,
                 float* out_pred0, float* out_target0, float* out_mask0) {
    using namespace dressi_examples;
    return Guard([&] {
        const ImgSize screen = {screen_px, screen_px};
        const ImgSize tex_size = {tex_w, tex_h};
        const ImgSize env_size = {env_w, env_h};
        PbrGeometryLeaves geom;
        geom.uvh = Variable(VEC4, {n_verts, 1});
        geom.normal = Variable(VEC3, {n_verts, 1});
        geom.tangent = Variable(VEC3, {n_verts, 1});
        geom.wpos = Variable(VEC3, {n_verts, 1});
        geom.faces = Variable(IVEC3, {n_faces, 1});
        PbrMaterialLeaves gt_mat;
        gt_mat.albedo = Variable(VEC3, tex_size);
        gt_mat.mr = Variable(VEC3, tex_size);
        gt_mat.normal_map = Variable(VEC3, tex_size);
        gt_mat.ao = Variable(VEC3, tex_size);
        gt_mat.emissive = Variable(VEC3, tex_size);
        PbrMaterialLeaves opt_mat = gt_mat;
        Variable albedo(VEC3, tex_size), mr(VEC3, tex_size);
        opt_mat.albedo = albedo;
        opt_mat.mr = mr;
        Variable env_gt(VEC3, env_size), env(VEC3, env_size);
        const auto ibl_of = [&](const Variable& e) {
            PbrIblMaps maps;
            maps.env = e;
            maps.irr = BuildIrradianceSample(e);
            maps.pref = BuildPrefEnvironmentSampleConv(e, levels);
            maps.lut = BuildBrdfIntegrationMap();
            return maps;
        };
        const PbrIblMaps ibl_gt = ibl_of(env_gt);
        const PbrIblMaps ibl = ibl_of(env);
        Variable uv_clip(VEC4, {n_verts, 1});
        Variable light_pos(VEC3, {1, 1}), light_col(VEC3, {1, 1});
        std::vector<Variable> clips, attrs, preds, targets, masks;
        std::vector<PbrFrameLeaves> frs(n_views);
        Variables view_losses;
        for (uint32_t v = 0; v < n_views; v++) {
            clips.emplace_back(VEC4, ImgSize{n_verts, 1});
            attrs.emplace_back(VEC4, ImgSize{n_verts, 1});
            frs[v].cam_pos = Variable(VEC3, {1, 1});
            frs[v].cam_fwd = Variable(VEC3, {1, 1});
            frs[v].cam_right = Variable(VEC3, {1, 1});
            frs[v].cam_up = Variable(VEC3, {1, 1});
            frs[v].light_pos = light_pos;
            frs[v].light_col = light_col;
            PbrGeometryLeaves vg = geom;
            vg.clip = clips[v];
            const PbrGBuffer gbuf = BuildPbrGBuffer(vg, screen);
            Variable inv_uv = F::Rasterize(uv_clip, attrs[v], geom.faces, tex_size);
            const PbrOutputs tgt = BuildPbrShade(gbuf, gt_mat, frs[v], ibl_gt, inv_uv, screen,
                                                 false);
            const PbrOutputs prd = BuildPbrShade(gbuf, opt_mat, frs[v], ibl, inv_uv, screen,
                                                 false);
            targets.push_back(tgt.mapped);
            preds.push_back(prd.mapped);
            masks.push_back(prd.mask);
            Variable diff = F::StopGradient(tgt.mapped) - prd.mapped;
            view_losses.push_back(F::Mean(F::Abs(diff)));
        }
        Variable loss = F::SumPixelWise(view_losses);
        Variable a_mut = albedo, m_mut = mr, e_mut = env;
        a_mut.setRequiresGradRecursively();
        m_mut.setRequiresGradRecursively();
        e_mut.setRequiresGradRecursively();
        auto [xs, gxs] = BuildBackward(loss);
        DRESSI_CHECK(xs.size() == 3, "expected albedo, mr and env as the leaves");
        Variable g_albedo{nullptr}, g_mr{nullptr}, g_env{nullptr};
        for (size_t i = 0; i < xs.size(); i++) {
            if (xs[i] == albedo) g_albedo = gxs[i];
            if (xs[i] == mr) g_mr = gxs[i];
            if (xs[i] == env) g_env = gxs[i];
        }
        DRESSI_CHECK(g_albedo && g_mr && g_env, "missing a leaf gradient");
        const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
        Variable adam_t(FLOAT, {1, 1});
        Variable t_new = adam_t + 1.f;
        Variable bc1 = 1.f - F::Pow(F::Float(b1), t_new);
        Variable bc2 = 1.f - F::Pow(F::Float(b2), t_new);
        struct Adam {
            Variable m, v, m_new, v_new, x_new;
        };
        const auto adam = [&](const Variable& x, const Variable& g, ImgSize sz, bool unit) {
            Adam a{Variable(VEC3, sz), Variable(VEC3, sz), Variable(nullptr),
                   Variable(nullptr), Variable(nullptr)};
            a.m_new = a.m * b1 + g * (1.f - b1);
            a.v_new = a.v * b2 + g * g * (1.f - b2);
            Variable step = (a.m_new / bc1) / (F::Sqrt(a.v_new / bc2) + eps) * lr;
            a.x_new = unit ? F::Clamp(x - step, F::Float(0.f), F::Float(1.f))
                           : F::Max(x - step, F::Float(0.f));
            return a;
        };
        Adam ad_a = adam(albedo, g_albedo, tex_size, true);
        Adam ad_m = adam(mr, g_mr, tex_size, true);
        Adam ad_e = adam(env, g_env, env_size, false);

        const size_t ntx = size_t(tex_w) * tex_h, nev = size_t(env_w) * env_h;
        std::vector<float> uvh(size_t(n_verts) * 4), zeros3(size_t(n_verts) * 3, 0.f);
        for (uint32_t i = 0; i < n_verts; i++) {
            uvh[i * 4 + 0] = uv[i * 2 + 0];
            uvh[i * 4 + 1] = uv[i * 2 + 1];
            uvh[i * 4 + 2] = 1.f;
            uvh[i * 4 + 3] = 1.f;
        }
        CpuImage uv_img(n_verts, 1, 2);
        std::memcpy(uv_img.data.data(), uv, sizeof(float) * 2 * n_verts);
        const CpuImage uv_clip_img = UvAsClip(uv_img);
        std::vector<CpuImage> clip_imgs, attr_imgs;
        for (uint32_t v = 0; v < n_views; v++) {
            const float* m = mvps + 16 * v;
            CpuImage clip_img(n_verts, 1, 4);
            for (uint32_t i = 0; i < n_verts; i++) {
                const float p[4] = {pos[i * 3 + 0], pos[i * 3 + 1], pos[i * 3 + 2], 1.f};
                for (int row = 0; row < 4; row++) {
                    float acc = 0.f;
                    for (int k = 0; k < 4; k++) {
                        acc += m[k * 4 + row] * p[k];
                    }
                    clip_img.at(i, 0, uint32_t(row)) = acc;
                }
            }
            attr_imgs.push_back(ScreenAttr(clip_img, screen));
            clip_imgs.push_back(std::move(clip_img));
        }
        CpuTensor t_a = Tensor(VEC3, tex_size, albedo0), t_m = Tensor(VEC3, tex_size, mr0);
        CpuTensor t_e = Tensor(VEC3, env_size, env0);
        CpuTensor am = Fill(VEC3, tex_size, 0.f), av = am, mm = am, mv = am;
        CpuTensor em = Fill(VEC3, env_size, 0.f), ev_ = em;
        CpuTensor t_t = Fill(FLOAT, {1, 1}, 0.f);
        const size_t px = size_t(screen_px) * screen_px;
        for (uint32_t it = 0; it < iters; it++) {
            CpuEvaluator ev;
            ev.bind(geom.uvh, Tensor(VEC4, {n_verts, 1}, uvh.data()));
            ev.bind(geom.normal, Tensor(VEC3, {n_verts, 1}, normal));
            ev.bind(geom.tangent, Tensor(VEC3, {n_verts, 1}, zeros3.data()));
            ev.bind(geom.wpos, Tensor(VEC3, {n_verts, 1}, pos));
            ev.bind(geom.faces, Tensor(IVEC3, {n_faces, 1}, faces));
            ev.bind(gt_mat.albedo, Tensor(VEC3, tex_size, gt_albedo));
            ev.bind(gt_mat.mr, Tensor(VEC3, tex_size, gt_mr));
            ev.bind(gt_mat.normal_map, Fill(VEC3, tex_size, 0.5f));
            ev.bind(gt_mat.ao, Fill(VEC3, tex_size, 1.f));
            ev.bind(gt_mat.emissive, Fill(VEC3, tex_size, 0.f));
            ev.bind(env_gt, Tensor(VEC3, env_size, gt_env));
            ev.bind(uv_clip, Tensor(VEC4, {n_verts, 1}, uv_clip_img.data.data()));
            ev.bind(light_pos, Tensor(VEC3, {1, 1}, light));
            ev.bind(light_col, Tensor(VEC3, {1, 1}, light + 3));
            for (uint32_t v = 0; v < n_views; v++) {
                ev.bind(clips[v], Tensor(VEC4, {n_verts, 1}, clip_imgs[v].data.data()));
                ev.bind(attrs[v], Tensor(VEC4, {n_verts, 1}, attr_imgs[v].data.data()));
                const float* fr = frames + 12 * v;
                ev.bind(frs[v].cam_pos, Tensor(VEC3, {1, 1}, fr + 0));
                ev.bind(frs[v].cam_fwd, Tensor(VEC3, {1, 1}, fr + 3));
                ev.bind(frs[v].cam_right, Tensor(VEC3, {1, 1}, fr + 6));
                ev.bind(frs[v].cam_up, Tensor(VEC3, {1, 1}, fr + 9));
            }
            ev.bind(albedo, t_a);
            ev.bind(mr, t_m);
            ev.bind(env, t_e);
            ev.bind(ad_a.m, am);
            ev.bind(ad_a.v, av);
            ev.bind(ad_m.m, mm);
            ev.bind(ad_m.v, mv);
            ev.bind(ad_e.m, em);
            ev.bind(ad_e.v, ev_);
            ev.bind(adam_t, t_t);
            const CpuTensor li = ev.eval(loss);
            if (out_loss) out_loss[it] = li.data[0];
            if (it == 0) {
                if (out_g_albedo0) CopyOut(ev.eval(g_albedo), out_g_albedo0);
                if (out_g_mr0) CopyOut(ev.eval(g_mr), out_g_mr0);
                if (out_g_env0) CopyOut(ev.eval(g_env), out_g_env0);
                for (uint32_t v = 0; v < n_views; v++) {
                    if (out_pred0) CopyOut(ev.eval(preds[v]), out_pred0 + v * px * 3);
                    if (out_target0) CopyOut(ev.eval(targets[v]), out_target0 + v * px * 3);
                    if (out_mask0) CopyOut(ev.eval(masks[v]), out_mask0 + v * px);
                }
            }
            CpuTensor n_a = ev.eval(ad_a.x_new), n_am = ev.eval(ad_a.m_new);
            CpuTensor n_av = ev.eval(ad_a.v_new);
            CpuTensor n_m = ev.eval(ad_m.x_new), n_mm = ev.eval(ad_m.m_new);
            CpuTensor n_mv = ev.eval(ad_m.v_new);
            CpuTensor n_e = ev.eval(ad_e.x_new), n_em = ev.eval(ad_e.m_new);
            CpuTensor n_ev = ev.eval(ad_e.v_new);
            CpuTensor n_t = ev.eval(t_new);
            t_a = std::move(n_a);
            am = std::move(n_am);
            av = std::move(n_av);
            t_m = std::move(n_m);
            mm = std::move(n_mm);
            mv = std::move(n_mv);
            t_e = std::move(n_e);
            em = std::move(n_em);
            ev_ = std::move(n_ev);
            t_t = std::move(n_t);
        }
        (void)ntx;
        (void)nev;
        CopyOut(t_a, out_albedo);
        CopyOut(t_m, out_mr);
        CopyOut(t_e, out_env);
    });
}

}  // extern "C"
