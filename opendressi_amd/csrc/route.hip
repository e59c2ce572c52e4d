// route.hip -- recognition of the silhouette-fit and texture-fit example
// graphs and their execution on the fused plans (route.h). Host code: the
// plans' kernels live in hsr.hip / aa.hip / tex.hip.
#include <algorithm>
#include <functional>
#include <cstring>
#include <set>
#include <unordered_map>
#include <unordered_set>

#include "dressi/f.h"
#include "dressi/ibl.h"
#include "dressi/mesh_utils.h"
#include "dressi_examples/pbr_graph.h"
#include "dressi_hip.h"
#include "route.h"

namespace dressi {

namespace {

// Leaf roles of the example graph (run.cpp:205-226)
enum Role : int {
    kPos,
    kAdamM,
    kAdamV,
    kAdamT,
    kSFacesF,     // VEC3 {F,1}: the optimised mesh's faces
    kSFacesI,     // IVEC3 {F,1}: the same faces (aa)
    kSVtxFaces,   // FLOAT {V,deg}: VertexFacesTex of them
    kSFaceId,     // FLOAT {3F,1}: f per soft corner (hardsoftras)
    kSFacesSoft,  // IVEC3 {F,1}: (3f, 3f+1, 3f+2) (hardsoftras)
    kSOnes,       // FLOAT {V,1}: 1 (aa)
    kBOnes,       // target mesh: ones, faces, faces as VEC3, vertex-face table
    kBFacesI,
    kBFacesF,
    kBVtxFaces,
    kZeroSeed,  // seed of the frozen target antialias (aa)
    kSVtxNbrs,  // regulariser inputs (weight 0)
    kSFaceAdj,
    kTgtClip0,  // + view: the target mesh in clip space
};

// What a readable variable of the graph holds
enum Serve : int { kServeLoss, kServeGrad, kServePos, kServeM, kServeV, kServeT, kServePred0 = 16,
                   kServeTarget0 = 32 };

struct Params {
    bool aa = false, regs = false;
    uint32_t views = 0;
    ImgSize screen;
    float radius = 3.f;
    uint32_t samples = 0;
    uint32_t V = 0, F = 0, Vt = 0, Ft = 0, deg_s = 1, deg_b = 1, deg_n = 1;
};

// The example's graph built from Params. Free constants: slot 16 v + k is
// entry k (column-major) of view v's MVP, then lr, the Laplacian weight and
// the normal-consistency weight.
struct Template {
    std::map<int, Variable> leaves;
    Variable g{nullptr};  // stands for the optimizer's gradient input
    Variables targets, preds;
    Variable loss{nullptr}, updated{nullptr};
    std::vector<std::pair<Variable, Variable>> updates;
    std::unordered_map<const FunctionNode*, int> free_slot;
    int slot_lr = 0, slot_lap = 0, slot_nrm = 0, n_slots = 0;
};

Template build_template(const Params& p) {
    Template T;
    const ImgSize S = p.screen;
    auto leaf = [&](int role, VType t, ImgSize s) {
        Variable v(t, s);
        T.leaves[role] = v;
        return v;
    };
    auto free_const = [&](int slot) {
        Variable c = F::Float(0.f);
        T.free_slot[NodeAccess::Node(c)->creator.get()] = slot;
        return c;
    };
    T.slot_lr = 16 * (int)p.views;
    T.slot_lap = T.slot_lr + 1;
    T.slot_nrm = T.slot_lr + 2;
    T.n_slots = T.slot_lr + 3;

    const Variable b_ones = leaf(kBOnes, FLOAT, {p.Vt, 1});
    const Variable b_faces_i = leaf(kBFacesI, IVEC3, {p.Ft, 1});
    const Variable s_faces_f = leaf(kSFacesF, VEC3, {p.F, 1});
    const Variable s_vtx_faces = leaf(kSVtxFaces, FLOAT, {p.V, p.deg_s});
    const Variable pos = leaf(kPos, VEC3, {p.V, 1});
    const Variable adam_m = leaf(kAdamM, VEC3, {p.V, 1});
    const Variable adam_v = leaf(kAdamV, VEC3, {p.V, 1});
    const Variable adam_t = leaf(kAdamT, FLOAT, {1, 1});
    Variable b_faces_f{nullptr}, b_vtx_faces{nullptr}, s_ones{nullptr}, s_faces_i{nullptr};
    Variable zero_seed{nullptr}, s_face_id{nullptr}, s_faces_soft{nullptr};
    if (p.aa) {
        b_faces_f = leaf(kBFacesF, VEC3, {p.Ft, 1});
        b_vtx_faces = leaf(kBVtxFaces, FLOAT, {p.Vt, p.deg_b});
        s_ones = leaf(kSOnes, FLOAT, {p.V, 1});
        s_faces_i = leaf(kSFacesI, IVEC3, {p.F, 1});
        zero_seed = leaf(kZeroSeed, FLOAT, {1, 1});
    } else {
        s_face_id = leaf(kSFaceId, FLOAT, {p.F * 3, 1});
        s_faces_soft = leaf(kSFacesSoft, IVEC3, {p.F, 1});
    }

    // clip = MVP * (pos, 1), row by row (geometry_utils.cpp:391-402)
    auto clip_of = [&](uint32_t v) {
        const Variable x = F::GetX(pos), y = F::GetY(pos), z = F::GetZ(pos);
        auto row = [&](int r) {
            const int b = 16 * (int)v;
            return F::Add(F::Add(F::Add(F::Mul(x, free_const(b + r)),
                                        F::Mul(y, free_const(b + 4 + r))),
                                 F::Mul(z, free_const(b + 8 + r))),
                          free_const(b + 12 + r));
        };
        return F::Vec4(row(0), row(1), row(2), row(3));
    };

    // hardsoftras prediction with one peel (run.cpp:240-339)
    auto pred_hsr = [&](const Variable& clip) {
        const Variable soft_clip = F::SoftClip(clip, s_faces_f, S, p.radius);
        const Variable tri0 = F::LookupFaces(clip, s_faces_f, s_vtx_faces, 0);
        const Variable tri1 = F::LookupFaces(clip, s_faces_f, s_vtx_faces, 1);
        const Variable tri2 = F::LookupFaces(clip, s_faces_f, s_vtx_faces, 2);
        const Variable pc = F::ScreenCoord(S);
        const Variable zero = F::Float(0.f);
        const Variable one = F::Float(1.f);
        auto coverage_prob = [&](const Variable& idx) {
            const Variable mask = F::Greater(idx, F::Float(0.5f));
            auto corner_px = [&](const Variable& tri) {
                const Variable c =
                        F::FaceFetch(tri, idx, tri0, tri1, tri2, adam_t, p.radius, p.samples);
                const Variable w = F::Add(F::GetW(c), F::Sub(F::Float(1.f), mask));
                auto axis = [&](const Variable& u, uint32_t extent) {
                    return F::Mul(F::Add(F::Mul(F::Div(u, w), F::Float(0.5f)), F::Float(0.5f)),
                                  F::Float((float)extent));
                };
                return F::Vec2(axis(F::GetX(c), S.w), axis(F::GetY(c), S.h));
            };
            const Variable s0 = corner_px(tri0), s1 = corner_px(tri1), s2 = corner_px(tri2);
            auto seg_dist = [&](const Variable& a, const Variable& b) {
                const Variable e = F::Sub(b, a);
                const Variable t =
                        F::Clamp(F::Div(F::Dot(F::Sub(pc, a), e),
                                        F::Add(F::Dot(e, e), F::Float(1e-12f))),
                                 zero, one);
                const Variable d = F::Sub(pc, F::Add(a, F::Mul(t, e)));
                return F::Sqrt(F::Add(F::Dot(d, d), F::Float(1e-12f)));
            };
            auto side = [&](const Variable& a, const Variable& b) {
                const Variable e = F::Sub(b, a);
                return F::Sub(F::Mul(F::GetX(e), F::Sub(F::GetY(pc), F::GetY(a))),
                              F::Mul(F::GetY(e), F::Sub(F::GetX(pc), F::GetX(a))));
            };
            const Variable dmin =
                    F::Min(F::Min(seg_dist(s0, s1), seg_dist(s1, s2)), seg_dist(s2, s0));
            const Variable c0 = side(s0, s1), c1 = side(s1, s2), c2 = side(s2, s0);
            const Variable pos_side =
                    F::Mul(F::Mul(F::Step(zero, c0), F::Step(zero, c1)), F::Step(zero, c2));
            const Variable neg_side = F::Mul(F::Mul(F::Step(zero, F::Neg(c0)),
                                                    F::Step(zero, F::Neg(c1))),
                                             F::Step(zero, F::Neg(c2)));
            const Variable inside = F::Min(F::Add(pos_side, neg_side), one);
            const Variable dist =
                    F::Mul(F::Sub(F::Mul(inside, F::Float(2.f)), F::Float(1.f)), dmin);
            return F::Mul(mask, F::Sigmoid(F::Mul(dist, F::Float(7.f / p.radius))));
        };
        const Variable rs = F::StopGradient(F::RasterizeSoft(
                soft_clip, s_face_id, s_faces_soft, clip, s_faces_f, s_vtx_faces, S, p.radius));
        const Variable cov = F::GetW(rs);
        const Variable ge = F::Step(zero, F::GetX(rs));
        const Variable idx = F::Mul(F::Add(F::GetY(rs), F::Float(1.f)), cov);
        const Variable none = F::Mul(one, F::Sub(F::Float(1.f), coverage_prob(idx)));
        const Variable hard = F::Mul(cov, ge);
        return F::Max(hard, F::Sub(F::Float(1.f), none));
    };
    // aa prediction and targets (run.cpp:231-238, 342-357)
    auto pred_aa = [&](const Variable& clip) {
        const Variable mask = F::Rasterize(clip, s_ones, s_faces_i, S);
        const Variable tri = F::RasterizeFaceId(clip, s_ones, s_faces_i, S);
        return F::AntiAlias(mask, tri, clip, s_faces_f, s_vtx_faces, adam_t, p.samples);
    };
    auto target_of = [&](const Variable& tclip) {
        const Variable mask = F::Rasterize(tclip, b_ones, b_faces_i, S);
        if (!p.aa) {
            return F::StopGradient(mask);
        }
        const Variable tri = F::RasterizeFaceId(tclip, b_ones, b_faces_i, S);
        return F::StopGradient(
                F::AntiAlias(mask, tri, tclip, b_faces_f, b_vtx_faces, zero_seed, 0));
    };

    Variables view_losses;
    for (uint32_t v = 0; v < p.views; v++) {
        const Variable tclip = leaf(kTgtClip0 + (int)v, VEC4, {p.Vt, 1});
        T.targets.push_back(target_of(tclip));
        const Variable clip = clip_of(v);
        T.preds.push_back(p.aa ? pred_aa(clip) : pred_hsr(clip));
        const Variable diff = F::Sub(T.targets[v], T.preds[v]);
        view_losses.push_back(
                F::Mul(F::Mul(diff, diff), F::Float(1.f / (float)(S.w * S.h))));
    }
    T.loss = F::SumPixelWise(view_losses);

    // the optimizer (run.cpp:400-437)
    T.g = Variable(VEC3, ImgSize{p.V, 1});
    Variable g = T.g;
    if (p.regs) {
        const Variable s_vtx_nbrs = leaf(kSVtxNbrs, FLOAT, {p.V, p.deg_n});
        const Variable s_face_adj = leaf(kSFaceAdj, VEC3, {p.F, 1});
        const float inv_cnt = 1.f / (float)(p.V * 3);
        auto rms = [&](const Variable& x) {
            return F::Sqrt(
                    F::Add(F::Mul(F::SumAll(F::Mul(x, x)), F::Float(inv_cnt)), F::Float(1e-24f)));
        };
        const Variable data_rms = rms(g);
        const Variable g_lap = F::Sub(pos, F::VertexNeighborMean(pos, s_vtx_nbrs));
        const Variable g_nrm = F::NormalConsistencyVertexGrad(
                F::NormalConsistencyFaceTerm(pos, s_faces_f, s_face_adj), pos, s_faces_f,
                s_vtx_faces);
        g = F::Add(F::Add(g, F::Mul(g_lap, F::Mul(F::Div(data_rms, rms(g_lap)),
                                                  free_const(T.slot_lap)))),
                   F::Mul(g_nrm, F::Mul(F::Div(data_rms, rms(g_nrm)), free_const(T.slot_nrm))));
    }
    const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
    const Variable t_new = F::Add(adam_t, F::Float(1.f));
    const Variable m_new = F::Add(F::Mul(adam_m, F::Float(b1)), F::Mul(g, F::Float(1.f - b1)));
    const Variable v_new =
            F::Add(F::Mul(adam_v, F::Float(b2)), F::Mul(F::Mul(g, g), F::Float(1.f - b2)));
    const Variable bc1 = F::Sub(F::Float(1.f), F::Pow(F::Float(b1), t_new));
    const Variable bc2 = F::Sub(F::Float(1.f), F::Pow(F::Float(b2), t_new));
    const Variable step =
            F::Mul(F::Div(F::Div(m_new, bc1), F::Add(F::Sqrt(F::Div(v_new, bc2)), F::Float(eps))),
                   free_const(T.slot_lr));
    T.updates = {{adam_m, m_new}, {adam_v, v_new}, {adam_t, t_new}};
    T.updated = F::Sub(pos, step);
    return T;
}

// Sizes and attributes of the user's graph that the template needs
bool read_params(const GraphRoots& g, Params* p) {
    if (g.input_vars.size() != 1 || g.updated_vars.size() != 1 || g.input_grad_vars.size() != 1) {
        return false;
    }
    const Variable& pos = g.input_vars[0];
    if (pos.getVType() != VEC3 || pos.getImgSize().h != 1) {
        return false;
    }
    p->V = pos.getImgSize().w;
    std::vector<const FunctionNode*> soft, aa_pred, aa_tgt, rast_tgt, clip, look, fetch, vnm;
    for (const auto& f : *g.funcs) {
        const auto& n = NodeAccess::Node(f);
        switch (n->op) {
            case Op::kRasterizeSoft: soft.push_back(n.get()); break;
            case Op::kAntiAlias:
                (n->xs[2]->creator ? aa_pred : aa_tgt).push_back(n.get());
                break;
            case Op::kRasterize:
                if (!n->xs[0]->creator) {
                    rast_tgt.push_back(n.get());
                }
                break;
            case Op::kSoftClip: clip.push_back(n.get()); break;
            case Op::kLookupFaces: look.push_back(n.get()); break;
            case Op::kFaceFetch: fetch.push_back(n.get()); break;
            case Op::kVertexNeighborMean: vnm.push_back(n.get()); break;
            case Op::kCustom:
            case Op::kSetFragDepth:
            case Op::kPeelDepth: return false;
            default: break;
        }
    }
    if (!soft.empty() == !aa_pred.empty()) {
        return false;  // neither technique, or both
    }
    p->aa = !aa_pred.empty();
    if (p->aa) {
        if (aa_tgt.size() != aa_pred.size()) {
            return false;
        }
        const FunctionNode* pr = aa_pred[0];
        const FunctionNode* tg = aa_tgt[0];
        p->views = (uint32_t)aa_pred.size();
        p->screen = pr->y.lock()->size;
        p->samples = pr->a0;
        p->F = pr->xs[3]->size.w;
        p->deg_s = pr->xs[4]->size.h;
        p->Vt = tg->xs[2]->size.w;
        p->Ft = tg->xs[3]->size.w;
        p->deg_b = tg->xs[4]->size.h;
    } else {
        if (clip.empty() || look.empty() || fetch.empty() || rast_tgt.empty()) {
            return false;
        }
        p->views = (uint32_t)soft.size();
        p->screen = soft[0]->y.lock()->size;
        p->radius = soft[0]->f0;
        p->F = clip[0]->xs[1]->size.w;
        p->deg_s = look[0]->xs[2]->size.h;
        p->samples = fetch[0]->a0;
        p->Vt = rast_tgt[0]->xs[0]->size.w;
        p->Ft = rast_tgt[0]->xs[2]->size.w;
    }
    p->regs = !vnm.empty();
    if (p->regs) {
        p->deg_n = vnm[0]->xs[1]->size.h;
    }
    return p->views >= 1 && p->views <= 8 && p->radius > 0.f && p->F > 0 && p->Vt > 0 &&
           p->Ft > 0;
}

// Structural comparison of a user graph with a template (free_slot, n_slots),
// from the roots
template <typename TT>
struct MatcherT {
    const TT& T;
    std::set<std::pair<const VariableNode*, const VariableNode*>> done;  // (user, template)
    std::unordered_map<const VariableNode*, const VariableNode*> leaf_of;  // template -> user
    std::vector<float> slot_val;
    std::vector<bool> slot_set;

    explicit MatcherT(const TT& t)
        : T(t), slot_val(t.n_slots, 0.f), slot_set(t.n_slots, false) {}

    bool match(const std::shared_ptr<VariableNode>& u, const std::shared_ptr<VariableNode>& t) {
        if (!u || !t) {
            return false;
        }
        if (done.count({u.get(), t.get()})) {
            return true;
        }
        if (u->vtype != t->vtype || !(u->size == t->size)) {
            return false;
        }
        if (!t->creator) {
            auto it = leaf_of.find(t.get());
            if (it != leaf_of.end()) {
                if (it->second != u.get()) {
                    return false;
                }
            } else {
                if (u->creator) {
                    return false;  // the template reads an input the user computes
                }
                leaf_of[t.get()] = u.get();
            }
            done.insert({u.get(), t.get()});
            return true;
        }
        if (!u->creator) {
            return false;
        }
        const FunctionNode& fu = *u->creator;
        const FunctionNode& ft = *t->creator;
        if (fu.op != ft.op || fu.a0 != ft.a0 || fu.a1 != ft.a1 || fu.flag != ft.flag ||
            std::memcmp(&fu.f0, &ft.f0, sizeof(float)) != 0 || fu.xs.size() != ft.xs.size() ||
            fu.op == Op::kCustom) {
            return false;
        }
        if (ft.op == Op::kConst) {
            auto fs = T.free_slot.find(&ft);
            if (fs != T.free_slot.end()) {
                if (fu.cval.size() != 1) {
                    return false;
                }
                const int k = fs->second;
                if (slot_set[k] && std::memcmp(&slot_val[k], &fu.cval[0], sizeof(float)) != 0) {
                    return false;
                }
                slot_val[k] = fu.cval[0];
                slot_set[k] = true;
            } else if (fu.cval.size() != ft.cval.size() ||
                       std::memcmp(fu.cval.data(), ft.cval.data(),
                                   sizeof(float) * fu.cval.size()) != 0) {
                return false;
            }
        }
        for (size_t i = 0; i < fu.xs.size(); i++) {
            if (!match(fu.xs[i], ft.xs[i])) {
                return false;
            }
        }
        done.insert({u.get(), t.get()});
        return true;
    }
    bool match(const Variable& u, const Variable& t) {
        return match(NodeAccess::Node(u), NodeAccess::Node(t));
    }
};

using Matcher = MatcherT<Template>;

bool is_integer_below(float x, uint32_t n) {
    return x >= 0.f && x < (float)n && x == (float)(uint32_t)x;
}

void check_hip_rc(int rc, const char* what) {
    if (rc != DRESSI_OK) {
        throw DressiError(std::string(what) + ": " + dressi_last_error());
    }
}

}  // namespace

struct SilhouetteRoute::State {
    Params p;
    std::vector<float> mvps;  // N x 16, column-major
    float lr = 0.f;
    // leaf roles: user variable per role, roles per user leaf
    std::map<int, Variable> user_leaf;
    std::unordered_map<const VariableNode*, std::vector<int>> roles_of;
    std::unordered_map<const VariableNode*, int> serve;  // readable computed variables
    std::unordered_set<const VariableNode*> in_graph;
    bool keep_pred = false, keep_grad = false;
    // host images of the leaves
    std::map<int, CpuImage> data;
    bool mesh_dirty = true, targets_dirty = true;
    std::set<int> state_dirty;
    // the plan
    dressi_ctx* ctx = nullptr;
    dressi_hsr_plan* plan = nullptr;
    bool state_on_plan = false;  // the plan holds the optimiser state
    uint32_t steps = 0;

    ~State() { drop_plan(); }

    void drop_plan() {
        if (plan) {
            dressi_hsr_destroy(plan);
            plan = nullptr;
        }
        state_on_plan = false;
    }

    bool have(int role) const { return data.count(role) != 0; }

    // the static leaf images the plan derives from the faces
    bool mesh_fits() const {
        if (!have(kSFacesF) || !have(kSVtxFaces)) {
            return false;
        }
        const CpuImage& faces = data.at(kSFacesF);
        for (float x : faces.data) {
            if (!is_integer_below(x, p.V)) {
                return false;
            }
        }
        const CpuImage vf = VertexFacesTex(faces, p.V);
        const CpuImage& got = data.at(kSVtxFaces);
        if (vf.height != got.height || vf.data != got.data) {
            return false;
        }
        if (p.aa) {
            if (!have(kSFacesI) || data.at(kSFacesI).data != faces.data || !have(kSOnes)) {
                return false;
            }
            for (float x : data.at(kSOnes).data) {
                if (x != 1.f) {
                    return false;
                }
            }
        } else {
            if (!have(kSFaceId) || !have(kSFacesSoft)) {
                return false;
            }
            const CpuImage& fid = data.at(kSFaceId);
            const CpuImage& fs = data.at(kSFacesSoft);
            for (uint32_t i = 0; i < p.F * 3; i++) {
                if (fid.data[i] != (float)(i / 3) || fs.data[i] != (float)i) {
                    return false;
                }
            }
        }
        return true;
    }

    bool targets_fit() const {
        if (!have(kBOnes) || !have(kBFacesI)) {
            return false;
        }
        for (float x : data.at(kBFacesI).data) {
            if (!is_integer_below(x, p.Vt)) {
                return false;
            }
        }
        if (p.aa) {
            if (!have(kBFacesF) || data.at(kBFacesF).data != data.at(kBFacesI).data) {
                return false;
            }
        }
        for (uint32_t v = 0; v < p.views; v++) {
            if (!have(kTgtClip0 + (int)v)) {
                return false;
            }
        }
        return true;
    }

    // The frozen targets with the per-op kernels (the graph's own target
    // branch: Rasterize, and for aa RasterizeFaceId + AntiAlias)
    void render_targets() {
        const size_t npx = (size_t)p.screen.w * p.screen.h;
        std::vector<float> host(npx * p.views);
        std::vector<void*> tmp;
        auto dev = [&](const std::vector<float>& h) {
            void* d = nullptr;
            check_hip_rc(dressi_malloc(ctx, &d, std::max<size_t>(h.size(), 1) * sizeof(float)),
                         "target images");
            tmp.push_back(d);
            check_hip_rc(dressi_memcpy_h2d(ctx, d, h.data(), h.size() * sizeof(float)),
                         "target images");
            return (float*)d;
        };
        try {
            const float* ones = dev(data.at(kBOnes).data);
            const float* faces = dev(data.at(kBFacesI).data);
            float* out = nullptr;
            float* mask = nullptr;
            float* tri = nullptr;
            out = dev(std::vector<float>(npx));
            if (p.aa) {
                mask = dev(std::vector<float>(npx));
                tri = dev(std::vector<float>(npx));
            }
            for (uint32_t v = 0; v < p.views; v++) {
                const float* clip = dev(data.at(kTgtClip0 + (int)v).data);
                if (p.aa) {
                    check_hip_rc(dressi_rasterize(ctx, clip, p.Vt, ones, 1, faces, p.Ft,
                                                  p.screen.w, p.screen.h, mask),
                                 "target Rasterize");
                    check_hip_rc(dressi_rasterize_face_id(ctx, clip, p.Vt, faces, p.Ft,
                                                          p.screen.w, p.screen.h, tri),
                                 "target RasterizeFaceId");
                    check_hip_rc(dressi_antialias(ctx, mask, 1, tri, clip, p.Vt, faces, p.Ft,
                                                  p.screen.w, p.screen.h, out),
                                 "target AntiAlias");
                } else {
                    check_hip_rc(dressi_rasterize(ctx, clip, p.Vt, ones, 1, faces, p.Ft,
                                                  p.screen.w, p.screen.h, out),
                                 "target Rasterize");
                }
                check_hip_rc(dressi_memcpy_d2h(ctx, host.data() + npx * v, out,
                                               npx * sizeof(float)),
                             "target images");
                check_hip_rc(dressi_ctx_synchronize(ctx), "target images");
            }
        } catch (...) {
            dressi_ctx_synchronize(ctx);
            for (void* d : tmp) {
                dressi_free(ctx, d);
            }
            throw;
        }
        check_hip_rc(dressi_ctx_synchronize(ctx), "target images");
        for (void* d : tmp) {
            dressi_free(ctx, d);
        }
        check_hip_rc(dressi_hsr_set_targets(plan, host.data()), "dressi_hsr_set_targets");
    }

    void read_state(CpuImage* pos, CpuImage* m, CpuImage* v, float* t) {
        *pos = CpuImage(p.V, 1, 3);
        *m = CpuImage(p.V, 1, 3);
        *v = CpuImage(p.V, 1, 3);
        check_hip_rc(dressi_hsr_get_state(plan, pos->data.data(), m->data.data(), v->data.data(),
                                          t),
                     "dressi_hsr_get_state");
    }

    // the plan's current state into the host images
    void pull_state() {
        if (!plan || !state_on_plan) {
            return;
        }
        CpuImage pos, m, v;
        float t = 0.f;
        read_state(&pos, &m, &v, &t);
        // images sent since the last step stay as sent
        if (!state_dirty.count(kPos)) data[kPos] = pos;
        if (!state_dirty.count(kAdamM)) data[kAdamM] = m;
        if (!state_dirty.count(kAdamV)) data[kAdamV] = v;
        if (!state_dirty.count(kAdamT)) data[kAdamT] = CpuImage(1, 1, 1, t);
    }

    void push_state() {
        for (int r : {kPos, kAdamM, kAdamV, kAdamT}) {
            if (!have(r)) {
                data[r] = r == kAdamT ? CpuImage(1, 1, 1) : CpuImage(p.V, 1, 3);
            }
        }
        check_hip_rc(dressi_hsr_set_state(plan, data.at(kPos).data.data(),
                                          data.at(kAdamM).data.data(),
                                          data.at(kAdamV).data.data(), data.at(kAdamT).data[0]),
                     "dressi_hsr_set_state");
        state_dirty.clear();
        state_on_plan = true;
    }

    void create_plan() {
        dressi_hsr_desc d{};
        d.n_verts = p.V;
        d.n_faces = p.F;
        d.n_views = p.views;
        d.width = p.screen.w;
        d.height = p.screen.h;
        d.radius_px = p.radius;
        d.n_samples = p.samples;
        d.lr = lr;
        d.beta1 = 0.9f;
        d.beta2 = 0.999f;
        d.eps = 1e-8f;
        d.flags = (keep_pred ? DRESSI_HSR_KEEP_PRED : 0u) | (keep_grad ? DRESSI_HSR_KEEP_GRAD : 0u) |
                  (p.aa ? DRESSI_HSR_TECHNIQUE_AA : 0u);
        check_hip_rc(dressi_hsr_create(ctx, &d, &plan), "dressi_hsr_create");
        check_hip_rc(dressi_hsr_set_mesh(plan, data.at(kSFacesF).data.data(), mvps.data()),
                     "dressi_hsr_set_mesh");
    }
};

SilhouetteRoute::SilhouetteRoute(std::unique_ptr<State> st) : st_(std::move(st)) {}
SilhouetteRoute::~SilhouetteRoute() = default;

std::string SilhouetteRoute::name() const {
    return st_->p.aa ? "fused:aa" : "fused:hardsoftras";
}

size_t SilhouetteRoute::kernels() const { return 5; }

std::unique_ptr<SilhouetteRoute> SilhouetteRoute::Recognise(const GraphRoots& g) {
    Params p;
    if (!g.funcs || !g.loss || !read_params(g, &p)) {
        return nullptr;
    }
    std::unique_ptr<Template> T;
    try {
        T = std::make_unique<Template>(build_template(p));
    } catch (const DressiError&) {
        return nullptr;  // sizes the example's ops reject
    }
    Matcher M(*T);
    const Variable& g_user = g.input_grad_vars[0];
    M.leaf_of[NodeAccess::Node(T->g).get()] = NodeAccess::Node(g_user).get();
    if (g_user.getVType() != VEC3 || !(g_user.getImgSize() == T->g.getImgSize())) {
        return nullptr;
    }
    if (!M.match(g.loss, T->loss) || !M.match(g.updated_vars[0], T->updated)) {
        return nullptr;
    }
    if (g.extra_updates.size() != T->updates.size()) {
        return nullptr;
    }
    for (size_t i = 0; i < T->updates.size(); i++) {
        const auto& [leaf_u, upd_u] = g.extra_updates[i];
        const auto& [leaf_t, upd_t] = T->updates[i];
        if (!M.match(upd_u, upd_t) || !M.match(leaf_u, leaf_t)) {
            return nullptr;
        }
    }
    auto pos_leaf = M.leaf_of.find(NodeAccess::Node(T->leaves.at(kPos)).get());
    if (pos_leaf == M.leaf_of.end() || pos_leaf->second != NodeAccess::Node(g.input_vars[0]).get()) {
        return nullptr;
    }
    for (int k = 0; k < 16 * (int)p.views + 1; k++) {
        if (!M.slot_set[k]) {
            return nullptr;
        }
    }
    if (p.regs && !(M.slot_set[T->slot_lap] && M.slot_set[T->slot_nrm] &&
                    M.slot_val[T->slot_lap] == 0.f && M.slot_val[T->slot_nrm] == 0.f)) {
        return nullptr;  // the plan runs the fit without regularisers
    }

    auto st = std::make_unique<State>();
    st->p = p;
    st->mvps.assign(M.slot_val.begin(), M.slot_val.begin() + 16 * p.views);
    st->lr = M.slot_val[T->slot_lr];
    for (const auto& [role, tv] : T->leaves) {
        auto it = M.leaf_of.find(NodeAccess::Node(tv).get());
        if (it == M.leaf_of.end()) {
            continue;  // a leaf the matched graph does not read
        }
        // the user's handle: found among the user graph's leaves
        st->roles_of[it->second].push_back(role);
    }
    std::unordered_map<const VariableNode*, int> serve_t;  // template node -> what it holds
    serve_t[NodeAccess::Node(T->loss).get()] = kServeLoss;
    serve_t[NodeAccess::Node(T->updated).get()] = kServePos;
    serve_t[NodeAccess::Node(T->updates[0].second).get()] = kServeM;
    serve_t[NodeAccess::Node(T->updates[1].second).get()] = kServeV;
    serve_t[NodeAccess::Node(T->updates[2].second).get()] = kServeT;
    for (uint32_t v = 0; v < p.views; v++) {
        serve_t[NodeAccess::Node(T->preds[v]).get()] = kServePred0 + (int)v;
        serve_t[NodeAccess::Node(T->targets[v]).get()] = kServeTarget0 + (int)v;
    }
    for (const auto& [u, t] : M.done) {
        st->in_graph.insert(u);
        auto s = serve_t.find(t);
        if (s != serve_t.end()) {
            st->serve[u] = s->second;
        }
    }
    st->serve[NodeAccess::Node(g_user).get()] = kServeGrad;
    st->in_graph.insert(NodeAccess::Node(g_user).get());
    st->keep_grad = g.grad_outputs;
    for (const auto& v : g.extra_outputs) {
        const VariableNode* n = NodeAccess::Node(v).get();
        auto s = st->serve.find(n);
        if (s != st->serve.end()) {
            st->keep_pred |= s->second >= kServePred0 && s->second < kServeTarget0;
            st->keep_grad |= s->second == kServeGrad;
        } else if (!st->roles_of.count(n)) {
            return nullptr;  // an output the plan does not keep
        }
    }
    if (p.aa) {
        st->keep_pred = true;  // the aa plan always writes its predictions
    }
    // user handles of the role leaves
    for (const auto& f : *g.funcs) {
        for (const auto& x : f.getInputVars()) {
            auto it = st->roles_of.find(NodeAccess::Node(x).get());
            if (it != st->roles_of.end()) {
                for (int r : it->second) {
                    st->user_leaf.emplace(r, x);
                }
            }
        }
    }
    for (const auto& [leaf_u, upd_u] : g.extra_updates) {
        auto it = st->roles_of.find(NodeAccess::Node(leaf_u).get());
        if (it != st->roles_of.end()) {
            for (int r : it->second) {
                st->user_leaf.emplace(r, leaf_u);
            }
        }
    }
    return std::unique_ptr<SilhouetteRoute>(new SilhouetteRoute(std::move(st)));
}

bool SilhouetteRoute::Accept(const Variable& var, const CpuImageView& img) {
    State& s = *st_;
    const VariableNode* n = NodeAccess::Node(var).get();
    auto it = s.roles_of.find(n);
    if (it == s.roles_of.end()) {
        return !s.in_graph.count(n);
    }
    CpuImage copy(img.width, img.height, img.channels);
    std::copy(img.data, img.data + img.numElems(), copy.data.begin());
    for (int r : it->second) {
        s.data[r] = copy;
        if (r == kPos || r == kAdamM || r == kAdamV || r == kAdamT) {
            s.state_dirty.insert(r);
        } else if (r == kBOnes || r == kBFacesI || r == kBFacesF || r == kBVtxFaces ||
                   r >= kTgtClip0) {
            s.targets_dirty = true;
        } else if (r != kZeroSeed && r != kSVtxNbrs && r != kSFaceAdj) {
            s.mesh_dirty = true;  // read by neither the targets nor the plan at weight 0
        }
    }
    return true;
}

void SilhouetteRoute::Export(std::map<Variable, CpuImage>* back) {
    State& s = *st_;
    s.pull_state();
    for (const auto& [role, var] : s.user_leaf) {
        auto d = s.data.find(role);
        if (d != s.data.end()) {
            (*back)[var] = d->second;
        }
    }
}

bool SilhouetteRoute::Step(dressi_ctx* ctx, std::map<Variable, CpuImage>* back) {
    State& s = *st_;
    if (s.plan && s.ctx != ctx) {
        throw DressiError("the fused silhouette plan moved to another context");
    }
    s.ctx = ctx;
    if (s.mesh_dirty) {
        if (!s.mesh_fits()) {
            Export(back);
            return false;
        }
        if (s.plan) {
            // new faces: a new plan, with the current state
            s.pull_state();
            for (int r : {kPos, kAdamM, kAdamV, kAdamT}) {
                s.state_dirty.insert(r);
            }
            s.drop_plan();
        }
    }
    if (s.targets_dirty && !s.targets_fit()) {
        Export(back);
        return false;
    }
    if (!s.plan) {
        s.create_plan();
        s.targets_dirty = true;
        for (int r : {kPos, kAdamM, kAdamV, kAdamT}) {
            s.state_dirty.insert(r);
        }
    }
    s.mesh_dirty = false;
    if (s.targets_dirty) {
        s.render_targets();
        s.targets_dirty = false;
    }
    if (!s.state_dirty.empty()) {
        s.pull_state();
        s.push_state();
    }
    check_hip_rc(dressi_hsr_step(s.plan, 1), "dressi_hsr_step");
    s.steps++;
    return true;
}

bool SilhouetteRoute::Readable(const Variable& var) const {
    const VariableNode* n = NodeAccess::Node(var).get();
    auto it = st_->serve.find(n);
    if (it != st_->serve.end()) {
        const int k = it->second;
        if (k >= kServePred0 && k < kServeTarget0) {
            return st_->keep_pred;
        }
        return k != kServeGrad || st_->keep_grad;
    }
    return st_->roles_of.count(n) != 0;
}

CpuImage SilhouetteRoute::Recv(const Variable& var) {
    State& s = *st_;
    const VariableNode* n = NodeAccess::Node(var).get();
    DRESSI_CHECK(Readable(var),
                 "recvImg: the fused silhouette plan does not keep this Variable (markOutput it "
                 "before the first execStep)");
    DRESSI_CHECK(s.plan && s.steps > 0, "recvImg before the first execStep()");
    auto sv = s.serve.find(n);
    if (sv == s.serve.end()) {
        // a leaf: its current image
        s.pull_state();
        auto d = s.data.find(s.roles_of.at(n)[0]);
        DRESSI_CHECK(d != s.data.end(), "recvImg: no image was sent to this leaf");
        return d->second;
    }
    const int k = sv->second;
    const uint32_t W = s.p.screen.w, H = s.p.screen.h;
    const size_t npx = (size_t)W * H;
    // the plan buffer whole, then the part that is `img`
    auto read = [&](int which, size_t off, CpuImage img) {
        void* dev = nullptr;
        size_t bytes = 0;
        check_hip_rc(dressi_hsr_buffer(s.plan, which, &dev, &bytes), "dressi_hsr_buffer");
        std::vector<float> all(bytes / sizeof(float));
        DRESSI_CHECK(off + img.data.size() <= all.size(), "recvImg: plan buffer size");
        check_hip_rc(dressi_hsr_read(s.plan, which, all.data(), bytes), "dressi_hsr_read");
        std::copy(all.begin() + (ptrdiff_t)off, all.begin() + (ptrdiff_t)(off + img.data.size()),
                  img.data.begin());
        return img;
    };
    switch (k) {
        case kServeLoss: return read(DRESSI_HSR_LOSS, 0, CpuImage(W, H, 1));
        case kServeGrad: return read(DRESSI_HSR_GRAD, 0, CpuImage(s.p.V, 1, 3));
        case kServePos:
        case kServeM:
        case kServeV:
        case kServeT: {
            CpuImage pos, m, v;
            float t = 0.f;
            s.read_state(&pos, &m, &v, &t);
            return k == kServePos ? pos : k == kServeM ? m : k == kServeV ? v
                                                                          : CpuImage(1, 1, 1, t);
        }
        default: break;
    }
    if (k >= kServeTarget0) {
        return read(DRESSI_HSR_TARGET, npx * (size_t)(k - kServeTarget0), CpuImage(W, H, 1));
    }
    return read(DRESSI_HSR_PRED, npx * (size_t)(k - kServePred0), CpuImage(W, H, 1));
}

// ---- the texture fit ---------------------------------------------------------

namespace {

// Leaf roles of the texture graph (tests/graph_tex.cpp: the deferred unlit
// graph of examples/texture_optimization/run.cpp:112-145 with
// TextureBilinear, the RGB L2 image loss and the in-graph Adam of the
// silhouette example, run.cpp:404-437)
enum TexRole : int {
    kTUv,      // VEC2 {V,1}: vertex uv
    kTFaces,   // IVEC3 {F,1}
    kTUvClip,  // VEC4 {V,1}: UvAsClip(uv)
    kTOnes,    // FLOAT {V,1}: 1
    kTGt,      // VEC4 {T}: the target texture
    kTTex,     // VEC4 {T}: the optimised texture
    kTM,
    kTV,
    kTT,
    kTClip0 = 16,  // + view: the view's clip positions, sent each step
    kTAttr0 = 32,  // + view: ScreenAttr of them
};

enum TexServe : int { kTServeLoss, kTServeGrad, kTServeTex, kTServeM, kTServeV, kTServeT,
                      kTServePred0 = 16, kTServeTarget0 = 32 };

struct TexParams {
    uint32_t V = 0, F = 0, N = 0;
    ImgSize S, T;
};

struct TexTemplate {
    std::map<int, Variable> leaves;
    Variable g{nullptr};
    Variables targets, preds;
    Variables g_uvs, inv_uvs;  // per view
    Variable loss{nullptr}, updated{nullptr};
    std::vector<std::pair<Variable, Variable>> updates;
    std::unordered_map<const FunctionNode*, int> free_slot;
    int slot_lr = 0, n_slots = 1;
};

TexTemplate build_tex_template(const TexParams& p) {
    TexTemplate T;
    auto leaf = [&](int role, VType t, ImgSize s) {
        Variable v(t, s);
        T.leaves[role] = v;
        return v;
    };
    const Variable vtx_uv = leaf(kTUv, VEC2, {p.V, 1});
    const Variable faces = leaf(kTFaces, IVEC3, {p.F, 1});
    const Variable uv_clip = leaf(kTUvClip, VEC4, {p.V, 1});
    const Variable ones = leaf(kTOnes, FLOAT, {p.V, 1});
    const Variable gt_tex = leaf(kTGt, VEC4, p.T);
    const Variable tex = leaf(kTTex, VEC4, p.T);
    const Variable adam_m = leaf(kTM, VEC4, p.T);
    const Variable adam_v = leaf(kTV, VEC4, p.T);
    const Variable adam_t = leaf(kTT, FLOAT, {1, 1});
    const float c = 1.f / float(p.S.w * p.S.h);
    Variables view_losses;
    for (uint32_t v = 0; v < p.N; v++) {
        const Variable clip = leaf(kTClip0 + (int)v, VEC4, {p.V, 1});
        const Variable attr = leaf(kTAttr0 + (int)v, VEC4, {p.V, 1});
        const Variable g_uv = F::Rasterize(clip, vtx_uv, faces, p.S);
        const Variable g_mask = F::Rasterize(clip, ones, faces, p.S);
        const Variable inv_uv = F::Rasterize(uv_clip, attr, faces, p.T);
        const Variable target = g_mask * F::TextureBilinear(gt_tex, g_uv, inv_uv);
        const Variable pred = g_mask * F::TextureBilinear(tex, g_uv, inv_uv);
        const Variable diff = F::StopGradient(target) - pred;
        view_losses.push_back(diff * diff * F::Vec4(c, c, c, 0.f));
        T.targets.push_back(target);
        T.preds.push_back(pred);
        T.g_uvs.push_back(g_uv);
        T.inv_uvs.push_back(inv_uv);
    }
    T.loss = F::SumPixelWise(view_losses);
    T.g = Variable(VEC4, p.T);
    const Variable g = T.g;
    const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
    const Variable t_new = adam_t + 1.f;
    const Variable m_new = adam_m * b1 + g * (1.f - b1);
    const Variable v_new = adam_v * b2 + g * g * (1.f - b2);
    const Variable bc1 = 1.f - F::Pow(F::Float(b1), t_new);
    const Variable bc2 = 1.f - F::Pow(F::Float(b2), t_new);
    const Variable lr = F::Float(0.f);
    T.free_slot[NodeAccess::Node(lr)->creator.get()] = T.slot_lr;
    const Variable step = F::Mul((m_new / bc1) / (F::Sqrt(v_new / bc2) + eps), lr);
    T.updates = {{adam_m, m_new}, {adam_v, v_new}, {adam_t, t_new}};
    T.updated = tex - step;
    return T;
}

bool read_tex_params(const GraphRoots& g, TexParams* p) {
    if (g.input_vars.size() != 1 || g.updated_vars.size() != 1 || g.input_grad_vars.size() != 1) {
        return false;
    }
    const Variable& tex = g.input_vars[0];
    if (tex.getVType() != VEC4) {
        return false;
    }
    p->T = tex.getImgSize();
    std::vector<const FunctionNode*> tb;
    for (const auto& f : *g.funcs) {
        const auto& n = NodeAccess::Node(f);
        switch (n->op) {
            case Op::kTextureBilinear: tb.push_back(n.get()); break;
            case Op::kCustom:
            case Op::kSetFragDepth:
            case Op::kPeelDepth: return false;
            default: break;
        }
    }
    // TextureBilinear(tex, uv): inv_uv is held by its backward
    if (tb.empty() || tb.size() % 2 != 0 || tb[0]->xs.size() != 2) {
        return false;
    }
    p->N = (uint32_t)(tb.size() / 2);
    const auto& uv = tb[0]->xs[1];
    if (!uv->creator || uv->creator->op != Op::kRasterize || uv->creator->xs.size() != 3) {
        return false;
    }
    p->S = uv->size;
    p->V = uv->creator->xs[0]->size.w;
    p->F = uv->creator->xs[2]->size.w;
    return p->N >= 1 && p->N <= 8 && p->V > 0 && p->F > 0 && p->S.w == p->S.h && p->S.w > 0 &&
           p->T.w > 0 && p->T.h > 0;
}

}  // namespace

struct TextureRoute::State {
    TexParams p;
    float lr = 0.f;
    std::map<int, Variable> user_leaf;
    std::unordered_map<const VariableNode*, std::vector<int>> roles_of;
    std::unordered_map<const VariableNode*, int> serve;
    std::unordered_set<const VariableNode*> in_graph;
    bool keep_pred = false, keep_grad = false;
    std::map<int, CpuImage> data;
    bool mesh_dirty = true, target_dirty = true, clips_dirty = true;
    std::set<int> state_dirty;
    dressi_ctx* ctx = nullptr;
    dressi_tex_plan* plan = nullptr;
    bool state_on_plan = false;
    uint32_t steps = 0;

    ~State() { drop_plan(); }

    void drop_plan() {
        if (plan) {
            dressi_tex_destroy(plan);
            plan = nullptr;
        }
        state_on_plan = false;
    }

    bool have(int role) const { return data.count(role) != 0; }

    // the static leaves the plan derives from uv and faces
    bool mesh_fits() const {
        if (!have(kTUv) || !have(kTFaces) || !have(kTUvClip) || !have(kTOnes)) {
            return false;
        }
        for (float x : data.at(kTFaces).data) {
            if (!is_integer_below(x, p.V)) {
                return false;
            }
        }
        if (UvAsClip(data.at(kTUv)).data != data.at(kTUvClip).data) {
            return false;
        }
        for (float x : data.at(kTOnes).data) {
            if (x != 1.f) {
                return false;
            }
        }
        return true;
    }

    // every view's clip and ScreenAttr image (z = 1, w = 0)
    bool clips_fit() const {
        for (uint32_t v = 0; v < p.N; v++) {
            if (!have(kTClip0 + (int)v) || !have(kTAttr0 + (int)v)) {
                return false;
            }
            const std::vector<float>& a = data.at(kTAttr0 + (int)v).data;
            for (size_t i = 0; i + 3 < a.size(); i += 4) {
                if (a[i + 2] != 1.f || a[i + 3] != 0.f) {
                    return false;
                }
            }
        }
        return true;
    }

    void read_state(CpuImage* tex, CpuImage* m, CpuImage* v, float* t) {
        *tex = CpuImage(p.T.w, p.T.h, 4);
        *m = CpuImage(p.T.w, p.T.h, 4);
        *v = CpuImage(p.T.w, p.T.h, 4);
        check_hip_rc(dressi_tex_get_state(plan, tex->data.data(), m->data.data(), v->data.data(),
                                          t),
                     "dressi_tex_get_state");
    }

    void pull_state() {
        if (!plan || !state_on_plan) {
            return;
        }
        CpuImage tex, m, v;
        float t = 0.f;
        read_state(&tex, &m, &v, &t);
        if (!state_dirty.count(kTTex)) data[kTTex] = tex;
        if (!state_dirty.count(kTM)) data[kTM] = m;
        if (!state_dirty.count(kTV)) data[kTV] = v;
        if (!state_dirty.count(kTT)) data[kTT] = CpuImage(1, 1, 1, t);
    }

    void push_state() {
        for (int r : {kTTex, kTM, kTV, kTT}) {
            if (!have(r)) {
                data[r] = r == kTT ? CpuImage(1, 1, 1) : CpuImage(p.T.w, p.T.h, 4);
            }
        }
        check_hip_rc(dressi_tex_set_state(plan, data.at(kTTex).data.data(), data.at(kTM).data.data(),
                                          data.at(kTV).data.data(), data.at(kTT).data[0]),
                     "dressi_tex_set_state");
        state_dirty.clear();
        state_on_plan = true;
    }

    void create_plan() {
        dressi_tex_desc d{};
        d.n_verts = p.V;
        d.n_faces = p.F;
        d.n_views = p.N;
        d.width = p.S.w;
        d.height = p.S.h;
        d.tex_w = p.T.w;
        d.tex_h = p.T.h;
        d.n_sets = 1;
        d.lr = lr;
        d.beta1 = 0.9f;
        d.beta2 = 0.999f;
        d.eps = 1e-8f;
        d.flags = DRESSI_TEX_EXTERNAL_CLIP | (keep_pred ? DRESSI_TEX_KEEP_IMAGES : 0u) |
                  (keep_grad ? DRESSI_TEX_KEEP_GRAD : 0u);
        check_hip_rc(dressi_tex_create(ctx, &d, &plan), "dressi_tex_create");
        const std::vector<float> pos((size_t)p.V * 3, 0.f);  // unused with external clips
        check_hip_rc(dressi_tex_set_mesh(plan, pos.data(), data.at(kTUv).data.data(),
                                         data.at(kTFaces).data.data()),
                     "dressi_tex_set_mesh");
    }

    void upload_clips() {
        const size_t nv = (size_t)p.V * 4;
        std::vector<float> clips(nv * p.N), attrs(nv * p.N);
        for (uint32_t v = 0; v < p.N; v++) {
            std::copy(data.at(kTClip0 + (int)v).data.begin(), data.at(kTClip0 + (int)v).data.end(),
                      clips.begin() + (ptrdiff_t)(nv * v));
            std::copy(data.at(kTAttr0 + (int)v).data.begin(), data.at(kTAttr0 + (int)v).data.end(),
                      attrs.begin() + (ptrdiff_t)(nv * v));
        }
        check_hip_rc(dressi_tex_set_clips(plan, clips.data(), attrs.data()), "dressi_tex_set_clips");
    }
};

TextureRoute::TextureRoute(std::unique_ptr<State> st) : st_(std::move(st)) {}
TextureRoute::~TextureRoute() = default;

std::string TextureRoute::name() const { return "fused:texture"; }

size_t TextureRoute::kernels() const { return 5; }

std::unique_ptr<TextureRoute> TextureRoute::Recognise(const GraphRoots& g) {
    TexParams p;
    if (!g.funcs || !g.loss || !read_tex_params(g, &p)) {
        return nullptr;
    }
    std::unique_ptr<TexTemplate> T;
    try {
        T = std::make_unique<TexTemplate>(build_tex_template(p));
    } catch (const DressiError&) {
        return nullptr;
    }
    MatcherT<TexTemplate> M(*T);
    const Variable& g_user = g.input_grad_vars[0];
    if (g_user.getVType() != VEC4 || !(g_user.getImgSize() == T->g.getImgSize())) {
        return nullptr;
    }
    M.leaf_of[NodeAccess::Node(T->g).get()] = NodeAccess::Node(g_user).get();
    if (!M.match(g.loss, T->loss) || !M.match(g.updated_vars[0], T->updated)) {
        return nullptr;
    }
    if (g.extra_updates.size() != T->updates.size()) {
        return nullptr;
    }
    for (size_t i = 0; i < T->updates.size(); i++) {
        const auto& [leaf_u, upd_u] = g.extra_updates[i];
        const auto& [leaf_t, upd_t] = T->updates[i];
        if (!M.match(upd_u, upd_t) || !M.match(leaf_u, leaf_t)) {
            return nullptr;
        }
    }
    // The inverse-UV rasters: TextureBilinear keeps inv_uv for its backward,
    // so the graph holds them as the inputs of the GatherByInverseUVBilinear
    // nodes built for the prediction of each view: (gy, inv_uv, g_uv).
    {
        std::unordered_map<const VariableNode*, const VariableNode*> user_of;  // template -> user
        for (const auto& [u, t] : M.done) {
            user_of[t] = u;
        }
        std::vector<int> seen(p.N, 0);
        for (const auto& f : *g.funcs) {
            const auto& n = NodeAccess::Node(f);
            if (n->op != Op::kGatherInvUvBilinear) {
                continue;
            }
            if (n->xs.size() != 3) {
                return nullptr;
            }
            uint32_t v = 0;
            while (v < p.N) {
                auto it = user_of.find(NodeAccess::Node(T->g_uvs[v]).get());
                if (it != user_of.end() && it->second == n->xs[2].get()) {
                    break;
                }
                v++;
            }
            if (v == p.N || !M.match(n->xs[1], NodeAccess::Node(T->inv_uvs[v]))) {
                return nullptr;
            }
            seen[v]++;
        }
        for (uint32_t v = 0; v < p.N; v++) {
            if (!seen[v]) {
                return nullptr;  // no backward through a view's prediction
            }
        }
    }
    auto tex_leaf = M.leaf_of.find(NodeAccess::Node(T->leaves.at(kTTex)).get());
    if (tex_leaf == M.leaf_of.end() ||
        tex_leaf->second != NodeAccess::Node(g.input_vars[0]).get() || !M.slot_set[T->slot_lr]) {
        return nullptr;
    }
    auto st = std::make_unique<State>();
    st->p = p;
    st->lr = M.slot_val[T->slot_lr];
    for (const auto& [role, tv] : T->leaves) {
        auto it = M.leaf_of.find(NodeAccess::Node(tv).get());
        if (it != M.leaf_of.end()) {
            st->roles_of[it->second].push_back(role);
        }
    }
    std::unordered_map<const VariableNode*, int> serve_t;
    serve_t[NodeAccess::Node(T->loss).get()] = kTServeLoss;
    serve_t[NodeAccess::Node(T->updated).get()] = kTServeTex;
    serve_t[NodeAccess::Node(T->updates[0].second).get()] = kTServeM;
    serve_t[NodeAccess::Node(T->updates[1].second).get()] = kTServeV;
    serve_t[NodeAccess::Node(T->updates[2].second).get()] = kTServeT;
    for (uint32_t v = 0; v < p.N; v++) {
        serve_t[NodeAccess::Node(T->preds[v]).get()] = kTServePred0 + (int)v;
        serve_t[NodeAccess::Node(T->targets[v]).get()] = kTServeTarget0 + (int)v;
    }
    for (const auto& [u, t] : M.done) {
        st->in_graph.insert(u);
        auto s = serve_t.find(t);
        if (s != serve_t.end()) {
            st->serve[u] = s->second;
        }
    }
    st->serve[NodeAccess::Node(g_user).get()] = kTServeGrad;
    st->in_graph.insert(NodeAccess::Node(g_user).get());
    st->keep_grad = g.grad_outputs;
    for (const auto& v : g.extra_outputs) {
        const VariableNode* n = NodeAccess::Node(v).get();
        auto s = st->serve.find(n);
        if (s != st->serve.end()) {
            st->keep_pred |= s->second >= kTServePred0;
            st->keep_grad |= s->second == kTServeGrad;
        } else if (!st->roles_of.count(n)) {
            return nullptr;  // an output the plan does not keep
        }
    }
    for (const auto& f : *g.funcs) {
        for (const auto& x : f.getInputVars()) {
            auto it = st->roles_of.find(NodeAccess::Node(x).get());
            if (it != st->roles_of.end()) {
                for (int r : it->second) {
                    st->user_leaf.emplace(r, x);
                }
            }
        }
    }
    for (const auto& [leaf_u, upd_u] : g.extra_updates) {
        auto it = st->roles_of.find(NodeAccess::Node(leaf_u).get());
        if (it != st->roles_of.end()) {
            for (int r : it->second) {
                st->user_leaf.emplace(r, leaf_u);
            }
        }
    }
    return std::unique_ptr<TextureRoute>(new TextureRoute(std::move(st)));
}

bool TextureRoute::Accept(const Variable& var, const CpuImageView& img) {
    State& s = *st_;
    const VariableNode* n = NodeAccess::Node(var).get();
    auto it = s.roles_of.find(n);
    if (it == s.roles_of.end()) {
        return !s.in_graph.count(n);
    }
    CpuImage copy(img.width, img.height, img.channels);
    std::copy(img.data, img.data + img.numElems(), copy.data.begin());
    for (int r : it->second) {
        s.data[r] = copy;
        if (r == kTTex || r == kTM || r == kTV || r == kTT) {
            s.state_dirty.insert(r);
        } else if (r == kTGt) {
            s.target_dirty = true;
        } else if (r >= kTClip0) {
            s.clips_dirty = true;
        } else {
            s.mesh_dirty = true;
        }
    }
    return true;
}

void TextureRoute::Export(std::map<Variable, CpuImage>* back) {
    State& s = *st_;
    s.pull_state();
    for (const auto& [role, var] : s.user_leaf) {
        auto d = s.data.find(role);
        if (d != s.data.end()) {
            (*back)[var] = d->second;
        }
    }
}

bool TextureRoute::Step(dressi_ctx* ctx, std::map<Variable, CpuImage>* back) {
    State& s = *st_;
    if (s.plan && s.ctx != ctx) {
        throw DressiError("the fused texture plan moved to another context");
    }
    s.ctx = ctx;
    if (s.mesh_dirty) {
        if (!s.mesh_fits()) {
            Export(back);
            return false;
        }
        if (s.plan) {
            s.pull_state();
            for (int r : {kTTex, kTM, kTV, kTT}) {
                s.state_dirty.insert(r);
            }
            s.drop_plan();
        }
    }
    if (!s.clips_fit() || !s.have(kTGt)) {
        Export(back);
        return false;
    }
    if (!s.plan) {
        s.create_plan();
        s.target_dirty = true;
        s.clips_dirty = true;
        for (int r : {kTTex, kTM, kTV, kTT}) {
            s.state_dirty.insert(r);
        }
    }
    s.mesh_dirty = false;
    if (s.target_dirty) {
        check_hip_rc(dressi_tex_set_target(s.plan, s.data.at(kTGt).data.data()),
                     "dressi_tex_set_target");
        s.target_dirty = false;
    }
    if (s.clips_dirty) {
        s.upload_clips();
        s.clips_dirty = false;
    }
    if (!s.state_dirty.empty()) {
        s.pull_state();
        s.push_state();
    }
    check_hip_rc(dressi_tex_step(s.plan, 1), "dressi_tex_step");
    s.steps++;
    return true;
}

bool TextureRoute::Readable(const Variable& var) const {
    const VariableNode* n = NodeAccess::Node(var).get();
    auto it = st_->serve.find(n);
    if (it != st_->serve.end()) {
        const int k = it->second;
        if (k >= kTServePred0) {
            return st_->keep_pred;
        }
        return k != kTServeGrad || st_->keep_grad;
    }
    return st_->roles_of.count(n) != 0;
}

CpuImage TextureRoute::Recv(const Variable& var) {
    State& s = *st_;
    const VariableNode* n = NodeAccess::Node(var).get();
    DRESSI_CHECK(Readable(var),
                 "recvImg: the fused texture plan does not keep this Variable (markOutput it "
                 "before the first execStep)");
    DRESSI_CHECK(s.plan && s.steps > 0, "recvImg before the first execStep()");
    auto sv = s.serve.find(n);
    if (sv == s.serve.end()) {
        s.pull_state();
        auto d = s.data.find(s.roles_of.at(n)[0]);
        DRESSI_CHECK(d != s.data.end(), "recvImg: no image was sent to this leaf");
        return d->second;
    }
    const int k = sv->second;
    const size_t npx4 = (size_t)s.p.S.w * s.p.S.h * 4;
    auto read = [&](int which, size_t off, CpuImage img) {
        void* dev = nullptr;
        size_t bytes = 0;
        check_hip_rc(dressi_tex_buffer(s.plan, which, &dev, &bytes), "dressi_tex_buffer");
        std::vector<float> all(bytes / sizeof(float));
        DRESSI_CHECK(off + img.data.size() <= all.size(), "recvImg: plan buffer size");
        check_hip_rc(dressi_tex_read(s.plan, which, all.data(), bytes), "dressi_tex_read");
        std::copy(all.begin() + (ptrdiff_t)off, all.begin() + (ptrdiff_t)(off + img.data.size()),
                  img.data.begin());
        return img;
    };
    switch (k) {
        case kTServeLoss: return read(DRESSI_TEX_LOSS, 0, CpuImage(s.p.S.w, s.p.S.h, 4));
        case kTServeGrad: return read(DRESSI_TEX_GRAD, 0, CpuImage(s.p.T.w, s.p.T.h, 4));
        case kTServeTex:
        case kTServeM:
        case kTServeV:
        case kTServeT: {
            CpuImage tex, m, v;
            float t = 0.f;
            s.read_state(&tex, &m, &v, &t);
            return k == kTServeTex ? tex : k == kTServeM ? m : k == kTServeV ? v
                                                                           : CpuImage(1, 1, 1, t);
        }
        default: break;
    }
    if (k >= kTServeTarget0) {
        return read(DRESSI_TEX_TARGET, npx4 * (size_t)(k - kTServeTarget0),
                    CpuImage(s.p.S.w, s.p.S.h, 4));
    }
    return read(DRESSI_TEX_PRED, npx4 * (size_t)(k - kTServePred0), CpuImage(s.p.S.w, s.p.S.h, 4));
}

// ---- the PBR material + environment fit -------------------------------------------

namespace {

// Leaf roles of the PBR fit graph (tests/graph_pbr.cpp: per view the
// G-buffer and the shading of examples/common/pbr_graph.cpp with normal
// mapping off, the target from the ground-truth maps, the L1 loss
// Mean(|StopGradient(target) - pred|) summed over views, in-graph Adam on
// albedo, mr and env with one step counter, albedo / mr clamped to [0,1] and
// env to >= 0; examples/pbr_material_optimization/run.cpp:189-288)
enum PbrRole : int {
    kQUvh, kQNormal, kQTangent, kQWpos, kQFaces,
    kQGtAlbedo, kQGtMr, kQNmap, kQAo, kQEmis,
    kQAlbedo, kQMr, kQEnvGt, kQEnv, kQUvClip, kQLightPos, kQLightCol,
    kQT, kQM0, kQV0 = kQM0 + 3,  // + param (0 albedo, 1 mr, 2 env)
    kQClip0 = 32, kQAttr0 = 64, kQCamPos0 = 96, kQCamFwd0 = 128, kQCamRight0 = 160,
    kQCamUp0 = 192,  // + view
};

enum PbrServe : int { kQServeLoss, kQServeGrad0 = 1, kQServeP0 = 4, kQServeM0 = 7, kQServeV0 = 10,
                      kQServeT = 13 };  // + param where it applies

constexpr int kQParamRole[3] = {kQAlbedo, kQMr, kQEnv};
// the optimiser's state: parameters, moments, step counter
constexpr int kQStateRoles[10] = {kQAlbedo, kQMr, kQEnv, kQT, kQM0, kQM0 + 1, kQM0 + 2,
                                  kQV0, kQV0 + 1, kQV0 + 2};

struct PbrParams {
    uint32_t V = 0, F = 0, N = 0, levels = 0;
    ImgSize S, T, E;
};

struct PbrTemplate {
    std::map<int, Variable> leaves;
    Variable g[3] = {Variable(nullptr), Variable(nullptr), Variable(nullptr)};
    Variable loss{nullptr}, t_new{nullptr};
    Variable updated[3] = {Variable(nullptr), Variable(nullptr), Variable(nullptr)};
    Variable m_new[3] = {Variable(nullptr), Variable(nullptr), Variable(nullptr)};
    Variable v_new[3] = {Variable(nullptr), Variable(nullptr), Variable(nullptr)};
    Variables g_uvs, inv_uvs;  // per view
    std::unordered_map<const FunctionNode*, int> free_slot;
    int slot_lr = 0, n_slots = 1;
};

PbrTemplate build_pbr_template(const PbrParams& p) {
    using namespace dressi_examples;
    PbrTemplate T;
    auto leaf = [&](int role, VType t, ImgSize s) {
        Variable v(t, s);
        T.leaves[role] = v;
        return v;
    };
    PbrGeometryLeaves geom;
    geom.uvh = leaf(kQUvh, VEC4, {p.V, 1});
    geom.normal = leaf(kQNormal, VEC3, {p.V, 1});
    geom.tangent = leaf(kQTangent, VEC3, {p.V, 1});
    geom.wpos = leaf(kQWpos, VEC3, {p.V, 1});
    geom.faces = leaf(kQFaces, IVEC3, {p.F, 1});
    PbrMaterialLeaves gt_mat;
    gt_mat.albedo = leaf(kQGtAlbedo, VEC3, p.T);
    gt_mat.mr = leaf(kQGtMr, VEC3, p.T);
    gt_mat.normal_map = leaf(kQNmap, VEC3, p.T);
    gt_mat.ao = leaf(kQAo, VEC3, p.T);
    gt_mat.emissive = leaf(kQEmis, VEC3, p.T);
    PbrMaterialLeaves mat = gt_mat;
    mat.albedo = leaf(kQAlbedo, VEC3, p.T);
    mat.mr = leaf(kQMr, VEC3, p.T);
    const Variable env_gt = leaf(kQEnvGt, VEC3, p.E);
    const Variable env = leaf(kQEnv, VEC3, p.E);
    const auto maps_of = [&](const Variable& e) {
        PbrIblMaps m;
        m.env = e;
        m.irr = BuildIrradianceSample(e);
        m.pref = BuildPrefEnvironmentSampleConv(e, p.levels);
        m.lut = BuildBrdfIntegrationMap();
        return m;
    };
    const PbrIblMaps ibl_gt = maps_of(env_gt), ibl = maps_of(env);
    const Variable uv_clip = leaf(kQUvClip, VEC4, {p.V, 1});
    const Variable light_pos = leaf(kQLightPos, VEC3, {1, 1});
    const Variable light_col = leaf(kQLightCol, VEC3, {1, 1});
    Variables view_losses;
    for (uint32_t v = 0; v < p.N; v++) {
        const Variable clip = leaf(kQClip0 + (int)v, VEC4, {p.V, 1});
        const Variable attr = leaf(kQAttr0 + (int)v, VEC4, {p.V, 1});
        PbrFrameLeaves fr;
        fr.cam_pos = leaf(kQCamPos0 + (int)v, VEC3, {1, 1});
        fr.cam_fwd = leaf(kQCamFwd0 + (int)v, VEC3, {1, 1});
        fr.cam_right = leaf(kQCamRight0 + (int)v, VEC3, {1, 1});
        fr.cam_up = leaf(kQCamUp0 + (int)v, VEC3, {1, 1});
        fr.light_pos = light_pos;
        fr.light_col = light_col;
        PbrGeometryLeaves vg = geom;
        vg.clip = clip;
        const PbrGBuffer gb = BuildPbrGBuffer(vg, p.S);
        const Variable inv_uv = F::Rasterize(uv_clip, attr, geom.faces, p.T);
        const PbrOutputs target = BuildPbrShade(gb, gt_mat, fr, ibl_gt, inv_uv, p.S, false);
        const PbrOutputs pred = BuildPbrShade(gb, mat, fr, ibl, inv_uv, p.S, false);
        view_losses.push_back(F::Mean(F::Abs(F::StopGradient(target.mapped) - pred.mapped)));
        T.g_uvs.push_back(gb.uv);
        T.inv_uvs.push_back(inv_uv);
    }
    T.loss = F::SumPixelWise(view_losses);
    const Variable adam_t = leaf(kQT, FLOAT, {1, 1});
    const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
    T.t_new = adam_t + 1.f;
    const Variable bc1 = 1.f - F::Pow(F::Float(b1), T.t_new);
    const Variable bc2 = 1.f - F::Pow(F::Float(b2), T.t_new);
    const Variable params[3] = {mat.albedo, mat.mr, env};
    for (int k = 0; k < 3; k++) {
        const ImgSize sz = k < 2 ? p.T : p.E;
        const Variable adam_m = leaf(kQM0 + k, VEC3, sz);
        const Variable adam_v = leaf(kQV0 + k, VEC3, sz);
        T.g[k] = Variable(VEC3, sz);
        const Variable& g = T.g[k];
        T.m_new[k] = adam_m * b1 + g * (1.f - b1);
        T.v_new[k] = adam_v * b2 + g * g * (1.f - b2);
        const Variable lr = F::Float(0.f);
        T.free_slot[NodeAccess::Node(lr)->creator.get()] = T.slot_lr;
        const Variable step = F::Mul((T.m_new[k] / bc1) / (F::Sqrt(T.v_new[k] / bc2) + eps), lr);
        T.updated[k] = k < 2 ? F::Clamp(params[k] - step, F::Float(0.f), F::Float(1.f))
                             : F::Max(params[k] - step, F::Float(0.f));
    }
    return T;
}

bool read_pbr_params(const GraphRoots& g, PbrParams* p) {
    if (g.input_vars.size() != 3 || g.updated_vars.size() != 3 || g.input_grad_vars.size() != 3) {
        return false;
    }
    std::set<std::pair<uint32_t, uint32_t>> pref_sizes;  // one per prefilter level
    std::unordered_set<const VariableNode*> raster_pos;  // the rasters' position inputs
    const FunctionNode* inv = nullptr;
    for (const auto& f : *g.funcs) {
        const auto& n = NodeAccess::Node(f);
        switch (n->op) {
            case Op::kRasterize:
                if (!n->xs.empty()) {
                    raster_pos.insert(n->xs[0].get());
                }
                break;
            case Op::kPrefilterConv:
                if (const auto y = n->y.lock()) {
                    pref_sizes.insert({y->size.w, y->size.h});
                }
                break;
            case Op::kTextureBilinear:
                // TextureBilinear(tex, uv) at the G-buffer's pixels
                if (n->xs.size() == 2 && n->xs[1]->creator) {
                    inv = n.get();
                }
                break;
            case Op::kCustom:
            case Op::kSetFragDepth:
            case Op::kPeelDepth: return false;
            default: break;
        }
    }
    if (!inv || raster_pos.size() < 2 || pref_sizes.empty()) {
        return false;
    }
    // the rasters read each view's clip positions and UvAsClip(uv) (the
    // inverse-UV tables, reached through TextureBilinear's backward)
    p->N = (uint32_t)raster_pos.size() - 1;
    p->levels = (uint32_t)pref_sizes.size();
    p->S = inv->xs[1]->size;
    // the optimised images: albedo and mr of one size, the env (or all three alike)
    for (const auto& x : g.input_vars) {
        if (x.getVType() != VEC3) {
            return false;
        }
    }
    const ImgSize s0 = g.input_vars[0].getImgSize(), s1 = g.input_vars[1].getImgSize(),
                  s2 = g.input_vars[2].getImgSize();
    if (s0 == s1) {
        p->T = s0;
        p->E = s2;
    } else if (s0 == s2) {
        p->T = s0;
        p->E = s1;
    } else if (s1 == s2) {
        p->T = s1;
        p->E = s0;
    } else {
        return false;
    }
    // the G-buffer's uv raster: Rasterize(clip, uvh, faces)
    std::function<const FunctionNode*(const VariableNode*, int)> find_raster =
            [&](const VariableNode* v, int depth) -> const FunctionNode* {
        if (!v || !v->creator || depth > 4) return nullptr;
        if (v->creator->op == Op::kRasterize) return v->creator.get();
        for (const auto& x : v->creator->xs) {
            if (auto r = find_raster(x.get(), depth + 1)) return r;
        }
        return nullptr;
    };
    const FunctionNode* r = find_raster(inv->xs[1].get(), 0);
    if (!r || r->xs.size() != 3) {
        return false;
    }
    p->V = r->xs[0]->size.w;
    p->F = r->xs[2]->size.w;
    return p->N >= 1 && p->N <= 16 && p->levels >= 2 && p->levels <= 8 && p->V > 0 &&
           p->F > 0 && p->S.w > 0 && p->S.w == p->S.h && p->T.w > 0 && p->E.w > 0;
}

}  // namespace

struct PbrRoute::State {
    PbrParams p;
    float lr = 0.f;
    int order[3] = {0, 1, 2};  // param of the user's optimizer input i
    std::map<int, Variable> user_leaf;
    std::unordered_map<const VariableNode*, std::vector<int>> roles_of;
    std::unordered_map<const VariableNode*, int> serve;
    std::unordered_set<const VariableNode*> in_graph;
    bool keep_grad = false;
    std::map<int, CpuImage> data;
    bool scene_dirty = true, target_dirty = true;
    std::set<int> state_dirty;
    dressi_ctx* ctx = nullptr;
    dressi_pbr_plan* plan = nullptr;
    bool state_on_plan = false;
    uint32_t steps = 0;

    ~State() { drop_plan(); }

    void drop_plan() {
        if (plan) {
            dressi_pbr_destroy(plan);
            plan = nullptr;
        }
        state_on_plan = false;
    }

    bool have(int role) const { return data.count(role) != 0; }
    ImgSize size_of(int k) const { return k < 2 ? p.T : p.E; }

    static bool all_equal(const CpuImage& img, float x) {
        for (float y : img.data) {
            if (y != x) {
                return false;
            }
        }
        return true;
    }

    // the static leaves: the plan derives the G-buffer from them, with
    // normal mapping off, AO 1 and emissive 0
    bool scene_fits() const {
        // what the plan reads must have been sent; the maps it assumes
        // (normal map, AO, emissive, tangents) only where the graph reads them
        for (int r : {kQUvh, kQNormal, kQWpos, kQFaces, kQUvClip, kQLightPos, kQLightCol}) {
            if (!have(r)) {
                return false;
            }
        }
        for (int r : {kQNmap, kQAo, kQEmis, kQTangent}) {
            if (user_leaf.count(r) && !have(r)) {
                return false;
            }
        }
        if (have(kQTangent) && user_leaf.count(kQTangent) && !all_equal(data.at(kQTangent), 0.f)) {
            return false;
        }
        for (float x : data.at(kQFaces).data) {
            if (!is_integer_below(x, p.V)) {
                return false;
            }
        }
        const CpuImage& uvh = data.at(kQUvh);
        CpuImage uv(p.V, 1, 2);
        for (uint32_t i = 0; i < p.V; i++) {
            if (uvh.at(i, 0, 2) != 1.f || uvh.at(i, 0, 3) != 1.f) {
                return false;
            }
            uv.at(i, 0, 0) = uvh.at(i, 0, 0);
            uv.at(i, 0, 1) = uvh.at(i, 0, 1);
        }
        if (UvAsClip(uv).data != data.at(kQUvClip).data) {
            return false;
        }
        if ((have(kQAo) && user_leaf.count(kQAo) && !all_equal(data.at(kQAo), 1.f)) ||
            (have(kQEmis) && user_leaf.count(kQEmis) && !all_equal(data.at(kQEmis), 0.f))) {
            return false;
        }
        for (uint32_t v = 0; v < p.N; v++) {
            for (int base : {kQClip0, kQAttr0, kQCamPos0, kQCamFwd0, kQCamRight0, kQCamUp0}) {
                if (!have(base + (int)v)) {
                    return false;
                }
            }
            if (ScreenAttr(data.at(kQClip0 + (int)v), p.S).data != data.at(kQAttr0 + (int)v).data) {
                return false;
            }
        }
        return true;
    }

    void create_plan() {
        dressi_pbr_desc d{};
        d.n_verts = p.V;
        d.n_faces = p.F;
        d.n_views = p.N;
        d.width = p.S.w;
        d.height = p.S.h;
        d.tex_w = p.T.w;
        d.tex_h = p.T.h;
        d.env_w = p.E.w;
        d.env_h = p.E.h;
        d.levels = p.levels;
        d.lr = lr;
        d.beta1 = 0.9f;
        d.beta2 = 0.999f;
        d.eps = 1e-8f;
        d.flags = keep_grad ? DRESSI_PBR_KEEP_GRAD : 0u;
        check_hip_rc(dressi_pbr_create(ctx, &d, &plan), "dressi_pbr_create");
        const CpuImage& uvh = data.at(kQUvh);
        std::vector<float> uv((size_t)p.V * 2), clips((size_t)p.N * p.V * 4), frames(p.N * 12);
        for (uint32_t i = 0; i < p.V; i++) {
            uv[i * 2] = uvh.at(i, 0, 0);
            uv[i * 2 + 1] = uvh.at(i, 0, 1);
        }
        for (uint32_t v = 0; v < p.N; v++) {
            const std::vector<float>& c = data.at(kQClip0 + (int)v).data;
            std::copy(c.begin(), c.end(), clips.begin() + (ptrdiff_t)((size_t)v * p.V * 4));
            int j = 0;
            for (int base : {kQCamPos0, kQCamFwd0, kQCamRight0, kQCamUp0}) {
                for (int c3 = 0; c3 < 3; c3++) {
                    frames[v * 12 + j++] = data.at(base + (int)v).data[c3];
                }
            }
        }
        const float light[6] = {data.at(kQLightPos).data[0], data.at(kQLightPos).data[1],
                                data.at(kQLightPos).data[2], data.at(kQLightCol).data[0],
                                data.at(kQLightCol).data[1], data.at(kQLightCol).data[2]};
        check_hip_rc(dressi_pbr_set_scene_clips(plan, data.at(kQWpos).data.data(),
                                                data.at(kQNormal).data.data(), uv.data(),
                                                data.at(kQFaces).data.data(), clips.data(),
                                                frames.data(), light),
                     "dressi_pbr_set_scene_clips");
    }

    void pull_state() {
        if (!plan || !state_on_plan) {
            return;
        }
        CpuImage x[3], m[3], v[3];
        for (int k = 0; k < 3; k++) {
            const ImgSize sz = size_of(k);
            x[k] = CpuImage(sz.w, sz.h, 3);
            m[k] = CpuImage(sz.w, sz.h, 3);
            v[k] = CpuImage(sz.w, sz.h, 3);
        }
        float t = 0.f;
        check_hip_rc(dressi_pbr_get_state(plan, x[0].data.data(), x[1].data.data(),
                                          x[2].data.data(), &t),
                     "dressi_pbr_get_state");
        check_hip_rc(dressi_pbr_get_adam(plan, m[0].data.data(), v[0].data.data(),
                                         m[1].data.data(), v[1].data.data(), m[2].data.data(),
                                         v[2].data.data()),
                     "dressi_pbr_get_adam");
        for (int k = 0; k < 3; k++) {
            if (!state_dirty.count(kQParamRole[k])) data[kQParamRole[k]] = x[k];
            if (!state_dirty.count(kQM0 + k)) data[kQM0 + k] = m[k];
            if (!state_dirty.count(kQV0 + k)) data[kQV0 + k] = v[k];
        }
        if (!state_dirty.count(kQT)) data[kQT] = CpuImage(1, 1, 1, t);
    }

    void push_state() {
        for (int k = 0; k < 3; k++) {
            const ImgSize sz = size_of(k);
            for (int r : {kQParamRole[k], kQM0 + k, kQV0 + k}) {
                if (!have(r)) {
                    data[r] = CpuImage(sz.w, sz.h, 3);
                }
            }
        }
        if (!have(kQT)) {
            data[kQT] = CpuImage(1, 1, 1);
        }
        check_hip_rc(dressi_pbr_set_state(plan, data.at(kQAlbedo).data.data(),
                                          data.at(kQMr).data.data(), data.at(kQEnv).data.data(),
                                          data.at(kQT).data[0]),
                     "dressi_pbr_set_state");
        check_hip_rc(dressi_pbr_set_adam(plan, data.at(kQM0).data.data(), data.at(kQV0).data.data(),
                                         data.at(kQM0 + 1).data.data(),
                                         data.at(kQV0 + 1).data.data(),
                                         data.at(kQM0 + 2).data.data(),
                                         data.at(kQV0 + 2).data.data()),
                     "dressi_pbr_set_adam");
        state_dirty.clear();
        state_on_plan = true;
    }
};

PbrRoute::PbrRoute(std::unique_ptr<State> st) : st_(std::move(st)) {}
PbrRoute::~PbrRoute() = default;

std::string PbrRoute::name() const { return "fused:pbr"; }

size_t PbrRoute::kernels() const { return 11; }

std::unique_ptr<PbrRoute> PbrRoute::Recognise(const GraphRoots& g) {
    PbrParams p;
    if (!g.funcs || !g.loss || !read_pbr_params(g, &p)) {
        return nullptr;
    }
    std::unique_ptr<PbrTemplate> T;
    try {
        T = std::make_unique<PbrTemplate>(build_pbr_template(p));
    } catch (const DressiError&) {
        return nullptr;
    }
    MatcherT<PbrTemplate> M(*T);
    if (!M.match(g.loss, T->loss)) {
        return nullptr;
    }
    // the user's optimizer inputs: which parameter each is
    auto st = std::make_unique<State>();
    for (int i = 0; i < 3; i++) {
        const VariableNode* u = NodeAccess::Node(g.input_vars[i]).get();
        int k = -1;
        for (int q = 0; q < 3; q++) {
            auto it = M.leaf_of.find(NodeAccess::Node(T->leaves.at(kQParamRole[q])).get());
            if (it != M.leaf_of.end() && it->second == u) {
                k = q;
            }
        }
        if (k < 0) {
            return nullptr;
        }
        st->order[i] = k;
        const Variable& gu = g.input_grad_vars[i];
        if (gu.getVType() != VEC3 || !(gu.getImgSize() == T->g[k].getImgSize())) {
            return nullptr;
        }
        M.leaf_of[NodeAccess::Node(T->g[k]).get()] = NodeAccess::Node(gu).get();
    }
    for (int i = 0; i < 3; i++) {
        if (!M.match(g.updated_vars[i], T->updated[st->order[i]])) {
            return nullptr;
        }
    }
    // addUpdate pairs in the optimizer's input order, then the step counter
    if (g.extra_updates.size() != 7) {
        return nullptr;
    }
    for (int i = 0; i < 3; i++) {
        const int k = st->order[i];
        const auto& [lm, um] = g.extra_updates[2 * i];
        const auto& [lv, uv] = g.extra_updates[2 * i + 1];
        if (!M.match(um, T->m_new[k]) || !M.match(lm, T->leaves.at(kQM0 + k)) ||
            !M.match(uv, T->v_new[k]) || !M.match(lv, T->leaves.at(kQV0 + k))) {
            return nullptr;
        }
    }
    if (!M.match(g.extra_updates[6].second, T->t_new) ||
        !M.match(g.extra_updates[6].first, T->leaves.at(kQT)) || !M.slot_set[T->slot_lr]) {
        return nullptr;
    }
    // the inverse-UV rasters, held by TextureBilinear's backward: every
    // GatherByInverseUVBilinear (gy, inv_uv, uv) reads a view's G-buffer uv
    // and that view's inv_uv
    {
        std::unordered_map<const VariableNode*, const VariableNode*> user_of;
        for (const auto& [u, t] : M.done) {
            user_of[t] = u;
        }
        std::vector<int> seen(p.N, 0);
        for (const auto& f : *g.funcs) {
            const auto& n = NodeAccess::Node(f);
            if (n->op != Op::kGatherInvUvBilinear) {
                continue;
            }
            if (n->xs.size() != 3) {
                return nullptr;
            }
            uint32_t v = 0;
            while (v < p.N) {
                auto it = user_of.find(NodeAccess::Node(T->g_uvs[v]).get());
                if (it != user_of.end() && it->second == n->xs[2].get()) {
                    break;
                }
                v++;
            }
            if (v == p.N || !M.match(n->xs[1], NodeAccess::Node(T->inv_uvs[v]))) {
                return nullptr;
            }
            seen[v]++;
        }
        for (uint32_t v = 0; v < p.N; v++) {
            if (!seen[v]) {
                return nullptr;
            }
        }
    }
    st->p = p;
    st->lr = M.slot_val[T->slot_lr];
    for (const auto& [role, tv] : T->leaves) {
        auto it = M.leaf_of.find(NodeAccess::Node(tv).get());
        if (it != M.leaf_of.end()) {
            st->roles_of[it->second].push_back(role);
        }
    }
    std::unordered_map<const VariableNode*, int> serve_t;
    serve_t[NodeAccess::Node(T->loss).get()] = kQServeLoss;
    serve_t[NodeAccess::Node(T->t_new).get()] = kQServeT;
    for (int k = 0; k < 3; k++) {
        serve_t[NodeAccess::Node(T->updated[k]).get()] = kQServeP0 + k;
        serve_t[NodeAccess::Node(T->m_new[k]).get()] = kQServeM0 + k;
        serve_t[NodeAccess::Node(T->v_new[k]).get()] = kQServeV0 + k;
    }
    for (const auto& [u, t] : M.done) {
        st->in_graph.insert(u);
        auto s = serve_t.find(t);
        if (s != serve_t.end()) {
            st->serve[u] = s->second;
        }
    }
    for (int i = 0; i < 3; i++) {
        const VariableNode* gn = NodeAccess::Node(g.input_grad_vars[i]).get();
        st->serve[gn] = kQServeGrad0 + st->order[i];
        st->in_graph.insert(gn);
    }
    st->keep_grad = g.grad_outputs;
    for (const auto& v : g.extra_outputs) {
        const VariableNode* n = NodeAccess::Node(v).get();
        auto s = st->serve.find(n);
        if (s != st->serve.end()) {
            st->keep_grad |= s->second >= kQServeGrad0 && s->second < kQServeP0;
        } else if (!st->roles_of.count(n)) {
            return nullptr;  // an output the plan does not keep
        }
    }
    for (const auto& f : *g.funcs) {
        for (const auto& x : f.getInputVars()) {
            auto it = st->roles_of.find(NodeAccess::Node(x).get());
            if (it != st->roles_of.end()) {
                for (int r : it->second) {
                    st->user_leaf.emplace(r, x);
                }
            }
        }
    }
    for (const auto& [leaf_u, upd_u] : g.extra_updates) {
        auto it = st->roles_of.find(NodeAccess::Node(leaf_u).get());
        if (it != st->roles_of.end()) {
            for (int r : it->second) {
                st->user_leaf.emplace(r, leaf_u);
            }
        }
    }
    return std::unique_ptr<PbrRoute>(new PbrRoute(std::move(st)));
}

bool PbrRoute::Accept(const Variable& var, const CpuImageView& img) {
    State& s = *st_;
    const VariableNode* n = NodeAccess::Node(var).get();
    auto it = s.roles_of.find(n);
    if (it == s.roles_of.end()) {
        return !s.in_graph.count(n);
    }
    CpuImage copy(img.width, img.height, img.channels);
    std::copy(img.data, img.data + img.numElems(), copy.data.begin());
    for (int r : it->second) {
        s.data[r] = copy;
        if (r == kQAlbedo || r == kQMr || r == kQEnv || r == kQT ||
            (r >= kQM0 && r < kQV0 + 3)) {
            s.state_dirty.insert(r);
        } else if (r == kQGtAlbedo || r == kQGtMr || r == kQEnvGt) {
            s.target_dirty = true;
        } else {
            s.scene_dirty = true;
        }
    }
    return true;
}

void PbrRoute::Export(std::map<Variable, CpuImage>* back) {
    State& s = *st_;
    s.pull_state();
    for (const auto& [role, var] : s.user_leaf) {
        auto d = s.data.find(role);
        if (d != s.data.end()) {
            (*back)[var] = d->second;
        }
    }
}

bool PbrRoute::Step(dressi_ctx* ctx, std::map<Variable, CpuImage>* back) {
    State& s = *st_;
    if (s.plan && s.ctx != ctx) {
        throw DressiError("the fused PBR plan moved to another context");
    }
    s.ctx = ctx;
    if (s.scene_dirty) {
        if (!s.scene_fits()) {
            Export(back);
            return false;
        }
        if (s.plan) {
            // a new scene: a new plan, with the current state
            s.pull_state();
            for (int r : kQStateRoles) {
                s.state_dirty.insert(r);
            }
            s.drop_plan();
        }
    }
    if (!s.have(kQGtAlbedo) || !s.have(kQGtMr) || !s.have(kQEnvGt)) {
        Export(back);
        return false;
    }
    if (!s.plan) {
        s.create_plan();
        s.target_dirty = true;
        for (int r : kQStateRoles) {
            s.state_dirty.insert(r);
        }
    }
    s.scene_dirty = false;
    if (s.target_dirty) {
        // set_target renders the targets through the plan; the state goes back after it
        s.pull_state();
        check_hip_rc(dressi_pbr_set_target(s.plan, s.data.at(kQGtAlbedo).data.data(),
                                           s.data.at(kQGtMr).data.data(),
                                           s.data.at(kQEnvGt).data.data()),
                     "dressi_pbr_set_target");
        s.target_dirty = false;
        for (int r : kQStateRoles) {
            s.state_dirty.insert(r);
        }
    }
    if (!s.state_dirty.empty()) {
        s.pull_state();
        s.push_state();
    }
    check_hip_rc(dressi_pbr_step(s.plan, 1), "dressi_pbr_step");
    s.steps++;
    return true;
}

bool PbrRoute::Readable(const Variable& var) const {
    const VariableNode* n = NodeAccess::Node(var).get();
    auto it = st_->serve.find(n);
    if (it != st_->serve.end()) {
        const int k = it->second;
        return k < kQServeGrad0 || k >= kQServeP0 || st_->keep_grad;
    }
    return st_->roles_of.count(n) != 0;
}

CpuImage PbrRoute::Recv(const Variable& var) {
    State& s = *st_;
    const VariableNode* n = NodeAccess::Node(var).get();
    DRESSI_CHECK(Readable(var),
                 "recvImg: the fused PBR plan does not keep this Variable (markOutput it before "
                 "the first execStep)");
    DRESSI_CHECK(s.plan && s.steps > 0, "recvImg before the first execStep()");
    auto sv = s.serve.find(n);
    if (sv == s.serve.end()) {
        s.pull_state();
        auto d = s.data.find(s.roles_of.at(n)[0]);
        DRESSI_CHECK(d != s.data.end(), "recvImg: no image was sent to this leaf");
        return d->second;
    }
    const int k = sv->second;
    if (k == kQServeLoss) {
        CpuImage out(1, 1, 1);
        check_hip_rc(dressi_pbr_read(s.plan, DRESSI_PBR_LOSS, out.data.data(), sizeof(float)),
                     "dressi_pbr_read");
        return out;
    }
    if (k >= kQServeGrad0 && k < kQServeP0) {
        const int q = k - kQServeGrad0;
        const ImgSize sz = s.size_of(q);
        std::vector<float> rgba((size_t)sz.w * sz.h * 4);
        const int which = q == 0 ? DRESSI_PBR_G_ALBEDO : q == 1 ? DRESSI_PBR_G_MR : DRESSI_PBR_G_ENV;
        check_hip_rc(dressi_pbr_read(s.plan, which, rgba.data(), rgba.size() * sizeof(float)),
                     "dressi_pbr_read");
        CpuImage out(sz.w, sz.h, 3);
        for (size_t i = 0; i < (size_t)sz.w * sz.h; i++) {
            for (int c = 0; c < 3; c++) {
                out.data[i * 3 + c] = rgba[i * 4 + c];
            }
        }
        return out;
    }
    s.pull_state();
    if (k == kQServeT) {
        return s.data.at(kQT);
    }
    if (k >= kQServeV0) {
        return s.data.at(kQV0 + (k - kQServeV0));
    }
    if (k >= kQServeM0) {
        return s.data.at(kQM0 + (k - kQServeM0));
    }
    return s.data.at(kQParamRole[k - kQServeP0]);
}

std::unique_ptr<FusedRoute> RecogniseFusedRoute(const GraphRoots& g) {
    if (auto r = SilhouetteRoute::Recognise(g)) {
        return r;
    }
    if (auto r = TextureRoute::Recognise(g)) {
        return r;
    }
    if (auto r = PbrRoute::Recognise(g)) {
        return r;
    }
    return nullptr;
}

}  // namespace dressi
