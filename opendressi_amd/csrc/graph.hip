// graph.hip -- the Dressi-AD graph API (include/dressi_graph.h): graph IR,
// reverse-mode construction, and an executor that runs any graph of the
// path's ops on one HIP device.
//
// IR (include/dressi/variable.h, function.h, src/core/node.h:42-65): a
// Variable is a shared handle to a node holding its type, image size,
// creator and (weak) users; a Function holds its op, inputs, (weak) output,
// attributes and backward builder. Ids come from one counter, so creation
// order is a topological order.
//
// Executor: the functions reachable from the roots are evaluated in id
// order, each into its own device buffer: elementwise ops by one generic
// kernel launch per node (the reference CPU evaluator's per-op float
// semantics, src/core/op_builder.cpp:25-108), the raster / gather ops by the
// library's per-op entry points. After evaluation each update value is
// copied into its leaf (DressiAD's end-of-frame copy-back,
// src/dressi_ad.cpp:317-341).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <queue>
#include <unordered_map>
#include <unordered_set>

#include "dressi_graph.h"
#include "dressi_math.h"

namespace dressi {

namespace {

enum class Op : int {
    kConst,
    kAdd, kSub, kMul, kDiv, kNeg, kSqrt, kAbs, kSign, kExp, kLog, kPow,
    kMax, kMin, kClamp, kStep, kSigmoid, kLess, kLessEq, kGreater, kGreaterEq,
    kExtract, kCompose, kDot, kCompSum, kCopy, kSumPw,
    kReduce2x2, kUpsample2x, kScreenCoord,
    kRasterize, kRasterizeFaceId, kSoftClip, kRasterizeSoft, kLookupFaces, kLookupFacesBwd,
    kFaceFetch, kFaceFetchBwd, kGatherDistGrad, kColSum, kAntiAlias, kAaBwdImg, kAaBwdVtx,
};

uint64_t g_next_id = 1;

}  // namespace

using BwdFn = std::function<Variable(const Variables& xs, const Variable& y, const Variable& gy,
                                     uint32_t idx)>;

struct VariableNode {
    uint64_t id = 0;
    VType vtype = FLOAT;
    ImgSize size;
    std::shared_ptr<FunctionNode> creator;
    std::vector<std::weak_ptr<FunctionNode>> users;
    bool req_grad = false;
};

struct FunctionNode {
    uint64_t id = 0;
    Op op = Op::kConst;
    std::string name;
    std::vector<std::shared_ptr<VariableNode>> xs;
    std::weak_ptr<VariableNode> y;
    BwdFn bwd;
    std::vector<float> cval;  // constants
    uint32_t a0 = 0, a1 = 0;  // component offset / corner / sample count
    float f0 = 0.f;           // radius
    int flag = 0;             // wide gather / peel input present
};

uint32_t NumComponents(VType t) {
    switch (t) {
        case FLOAT: return 1;
        case VEC2: return 2;
        case VEC3: return 3;
        case VEC4: return 4;
        case IVEC3: return 3;
    }
    return 1;
}

static VType vec_of(uint32_t n) {
    return n == 1 ? FLOAT : n == 2 ? VEC2 : n == 3 ? VEC3 : VEC4;
}

static void require(bool ok, const std::string& msg) {
    if (!ok) {
        throw DressiError(msg);
    }
}

// ---- Variable / Function ---------------------------------------------------

Variable::Variable(VType vtype, ImgSize img_size) : m_node(std::make_shared<VariableNode>()) {
    m_node->id = g_next_id++;
    m_node->vtype = vtype;
    m_node->size = img_size;
}
bool Variable::operator<(const Variable& o) const {
    return (m_node ? m_node->id : 0) < (o.m_node ? o.m_node->id : 0);
}
uint64_t Variable::id() const { return m_node->id; }
VType Variable::getVType() const { return m_node->vtype; }
ImgSize Variable::getImgSize() const { return m_node->size; }
Function Variable::getCreator() const { return Function(m_node->creator); }
bool Variable::getRequiresGrad() const { return m_node->req_grad; }
void Variable::setRequiresGrad(bool r) { m_node->req_grad = r; }
void Variable::setRequiresGradRecursively(bool r) {
    // this variable and everything computed downstream of it
    std::unordered_set<const VariableNode*> seen;
    std::vector<std::shared_ptr<VariableNode>> stack = {m_node};
    while (!stack.empty()) {
        auto n = stack.back();
        stack.pop_back();
        if (!n || !seen.insert(n.get()).second) {
            continue;
        }
        n->req_grad = r;
        for (const auto& wu : n->users) {
            if (auto u = wu.lock()) {
                if (auto y = u->y.lock()) {
                    stack.push_back(std::move(y));
                }
            }
        }
    }
}

uint64_t Function::id() const { return m_node->id; }
const std::string& Function::name() const { return m_node->name; }
Variables Function::getInputVars() const {
    Variables v;
    for (const auto& x : m_node->xs) {
        v.emplace_back(x);
    }
    return v;
}
Variable Function::getOutputVar() const { return Variable(m_node->y.lock()); }
Variable Function::buildBwd(const Variable& gy, uint32_t idx) const {
    if (!m_node->bwd) {
        return nullptr;
    }
    return m_node->bwd(getInputVars(), getOutputVar(), gy, idx);
}

namespace {

ImgSize common_size(const Variables& xs) {
    ImgSize s;
    for (const auto& x : xs) {
        const ImgSize xs_ = x.getImgSize();
        if (xs_.isUniform()) {
            continue;
        }
        require(s.isUniform() || s == xs_, "image size mismatch between non-uniform inputs");
        s = xs_;
    }
    return s;
}

VType widest(const Variables& xs) {
    uint32_t n = 0;
    VType t = FLOAT;
    for (const auto& x : xs) {
        const uint32_t k = NumComponents(x.getVType());
        require(k <= 1 || n <= 1 || x.getVType() == t, "vector type mismatch between inputs");
        if (k > n) {
            n = k;
            t = x.getVType();
        }
    }
    return t;
}

struct OpSpec {
    Op op;
    const char* name;
    VType vtype;
    ImgSize size;
    BwdFn bwd;
};

Variable make_op(const OpSpec& s, const Variables& xs, std::vector<float> cval = {},
                 uint32_t a0 = 0, uint32_t a1 = 0, float f0 = 0.f, int flag = 0) {
    auto fn = std::make_shared<FunctionNode>();
    fn->id = g_next_id++;
    fn->op = s.op;
    fn->name = s.name;
    fn->bwd = s.bwd;
    fn->cval = std::move(cval);
    fn->a0 = a0;
    fn->a1 = a1;
    fn->f0 = f0;
    fn->flag = flag;
    for (const auto& x : xs) {
        require((bool)x, std::string(s.name) + ": null input");
        fn->xs.push_back(x.node());
        x.node()->users.push_back(fn);
    }
    auto y = std::make_shared<VariableNode>();
    y->id = g_next_id++;
    y->vtype = s.vtype;
    y->size = s.size;
    y->creator = fn;
    fn->y = y;
    return Variable(y);
}

Variable ew(Op op, const char* name, const Variables& xs, BwdFn bwd) {
    return make_op({op, name, widest(xs), common_size(xs), std::move(bwd)}, xs);
}

Variable ew_fixed(Op op, const char* name, VType t, const Variables& xs, BwdFn bwd) {
    return make_op({op, name, t, common_size(xs), std::move(bwd)}, xs);
}

const BwdFn kNull = nullptr;

Variable const_vec(const char* name, std::vector<float> v) {
    const VType t = vec_of((uint32_t)v.size());
    return make_op({Op::kConst, name, t, {1, 1}, kNull}, {}, std::move(v));
}

Variable extract(const Variable& v, uint32_t ofs, uint32_t n);

Variable compose(const Variables& parts) {
    uint32_t total = 0;
    std::vector<uint32_t> offs, widths;
    for (const auto& p : parts) {
        offs.push_back(total);
        widths.push_back(NumComponents(p.getVType()));
        total += widths.back();
    }
    require(total >= 2 && total <= 4, "Compose: 2..4 components");
    return make_op({Op::kCompose, "Compose", vec_of(total), common_size(parts),
                    [offs, widths](const Variables&, const Variable&, const Variable& gy,
                                   uint32_t i) { return extract(gy, offs[i], widths[i]); }},
                   parts);
}

Variable replicate(const Variable& s, uint32_t n) {
    return n == 1 ? s : compose(Variables(n, s));
}

Variable extract(const Variable& v, uint32_t ofs, uint32_t n) {
    const uint32_t src_n = NumComponents(v.getVType());
    require(ofs + n <= src_n, "component extraction out of range");
    if (n == src_n) {
        return v;
    }
    return make_op({Op::kExtract, "ExtractComps", vec_of(n), v.getImgSize(),
                    [ofs, n, src_n](const Variables&, const Variable&, const Variable& gy,
                                    uint32_t) {
                        Variables parts;
                        for (uint32_t j = 0; j < src_n; j++) {
                            if (ofs <= j && j < ofs + n) {
                                parts.push_back(n == 1 ? gy : extract(gy, j - ofs, 1));
                            } else {
                                parts.push_back(F::Float(0.f));
                            }
                        }
                        return compose(parts);
                    }},
                   {v}, {}, ofs);
}

Variable unary(Op op, const char* name, const Variable& x,
               std::function<Variable(const Variable& x, const Variable& y)> dydx) {
    BwdFn b = nullptr;
    if (dydx) {
        b = [dydx](const Variables& xs, const Variable& y, const Variable& gy, uint32_t) {
            return F::Mul(gy, dydx(xs[0], y));
        };
    }
    return ew(op, name, {x}, b);
}

Variable compare(Op op, const char* name, const Variable& a, const Variable& b) {
    require(a.getVType() == FLOAT && b.getVType() == FLOAT, "comparisons take FLOAT inputs");
    return ew_fixed(op, name, FLOAT, {a, b}, kNull);
}

ImgSize half(ImgSize s) { return {(s.w + 1) / 2, (s.h + 1) / 2}; }

Variable reduce2x2(const Variable& x);

Variable upsample2x(const Variable& x, ImgSize target) {
    return make_op({Op::kUpsample2x, "UpsampleNearest2x", x.getVType(), target,
                    [](const Variables&, const Variable&, const Variable& gy, uint32_t) {
                        return reduce2x2(gy);
                    }},
                   {x});
}

Variable reduce2x2(const Variable& x) {
    const ImgSize src = x.getImgSize();
    require(!src.isUniform(), "Reduce2x2Sum of a {1,1} input");
    return make_op({Op::kReduce2x2, "Reduce2x2Sum", x.getVType(), half(src),
                    [src](const Variables&, const Variable&, const Variable& gy, uint32_t) {
                        return upsample2x(gy, src);
                    }},
                   {x});
}

Variable sum_pw_flat(const Variables& xs) {
    return ew(Op::kSumPw, "SumPixelWise", xs,
              [](const Variables&, const Variable&, const Variable& gy, uint32_t) { return gy; });
}

// Internal backward ops (not differentiable further).
Variable special(Op op, const char* name, VType t, ImgSize size, const Variables& xs,
                 uint32_t a0 = 0, uint32_t a1 = 0, float f0 = 0.f, int flag = 0) {
    return make_op({op, name, t, size, kNull}, xs, {}, a0, a1, f0, flag);
}

}  // namespace

// ---- F:: ---------------------------------------------------------------------

namespace F {

Variable Float(float v) { return const_vec("Float", {v}); }
Variable Vec2(float x, float y) { return const_vec("Vec2", {x, y}); }
Variable Vec3(float x, float y, float z) { return const_vec("Vec3", {x, y, z}); }
Variable Vec4(float x, float y, float z, float w) { return const_vec("Vec4", {x, y, z, w}); }

Variable Add(const Variable& a, const Variable& b) {
    return ew(Op::kAdd, "Add", {a, b},
              [](const Variables&, const Variable&, const Variable& gy, uint32_t) { return gy; });
}
Variable Sub(const Variable& a, const Variable& b) {
    return ew(Op::kSub, "Sub", {a, b},
              [](const Variables&, const Variable&, const Variable& gy, uint32_t i) {
                  return i == 0 ? gy : Neg(gy);
              });
}
Variable Mul(const Variable& a, const Variable& b) {
    return ew(Op::kMul, "Mul", {a, b},
              [](const Variables& xs, const Variable&, const Variable& gy, uint32_t i) {
                  return i == 0 ? Mul(gy, xs[1]) : Mul(gy, xs[0]);
              });
}
Variable Div(const Variable& a, const Variable& b) {
    return ew(Op::kDiv, "Div", {a, b},
              [](const Variables& xs, const Variable&, const Variable& gy, uint32_t i) {
                  if (i == 0) {
                      return Div(gy, xs[1]);
                  }
                  return Neg(Div(Mul(gy, xs[0]), Mul(xs[1], xs[1])));
              });
}
Variable Neg(const Variable& x) {
    return ew(Op::kNeg, "Neg", {x},
              [](const Variables&, const Variable&, const Variable& gy, uint32_t) {
                  return Neg(gy);
              });
}
Variable Sqrt(const Variable& x) {
    return unary(Op::kSqrt, "Sqrt", x,
                 [](const Variable&, const Variable& y) { return Div(Float(0.5f), y); });
}
Variable Sign(const Variable& x) { return unary(Op::kSign, "Sign", x, nullptr); }
Variable Abs(const Variable& x) {
    return unary(Op::kAbs, "Abs", x, [](const Variable& xv, const Variable&) { return Sign(xv); });
}
Variable Exp(const Variable& x) {
    return unary(Op::kExp, "Exp", x, [](const Variable&, const Variable& y) { return y; });
}
Variable Log(const Variable& x) {
    return unary(Op::kLog, "Log", x,
                 [](const Variable& xv, const Variable&) { return Div(Float(1.f), xv); });
}
Variable Pow(const Variable& x, const Variable& p) {
    return ew(Op::kPow, "Pow", {x, p},
              [](const Variables& xs, const Variable& y, const Variable& gy, uint32_t i) {
                  if (i == 0) {
                      return Mul(gy, Mul(xs[1], Pow(xs[0], Sub(xs[1], Float(1.f)))));
                  }
                  return Mul(gy, Mul(y, Log(xs[0])));
              });
}
Variable Max(const Variable& a, const Variable& b) {
    return ew(Op::kMax, "Max", {a, b},
              [](const Variables& xs, const Variable&, const Variable& gy, uint32_t i) {
                  Variable mask = Step(xs[1], xs[0]);
                  return i == 0 ? Mul(gy, mask) : Mul(gy, Sub(Float(1.f), mask));
              });
}
Variable Min(const Variable& a, const Variable& b) {
    return ew(Op::kMin, "Min", {a, b},
              [](const Variables& xs, const Variable&, const Variable& gy, uint32_t i) {
                  Variable mask = Step(xs[0], xs[1]);
                  return i == 0 ? Mul(gy, mask) : Mul(gy, Sub(Float(1.f), mask));
              });
}
Variable Clamp(const Variable& x, const Variable& lo, const Variable& hi) {
    return ew(Op::kClamp, "Clamp", {x, lo, hi},
              [](const Variables& xs, const Variable&, const Variable& gy, uint32_t i) -> Variable {
                  if (i != 0) {
                      return nullptr;  // no gradient toward the bounds
                  }
                  return Mul(gy, Mul(Step(xs[1], xs[0]), Step(xs[0], xs[2])));
              });
}
Variable Step(const Variable& edge, const Variable& x) {
    return ew(Op::kStep, "Step", {edge, x}, kNull);
}
Variable Sigmoid(const Variable& x) {
    return ew(Op::kSigmoid, "Sigmoid", {x},
              [](const Variables&, const Variable& y, const Variable& gy, uint32_t) {
                  return Mul(gy, Mul(y, Sub(Float(1.f), y)));
              });
}
Variable Less(const Variable& a, const Variable& b) { return compare(Op::kLess, "Less", a, b); }
Variable LessEqual(const Variable& a, const Variable& b) {
    return compare(Op::kLessEq, "LessEqual", a, b);
}
Variable Greater(const Variable& a, const Variable& b) {
    return compare(Op::kGreater, "Greater", a, b);
}
Variable GreaterEqual(const Variable& a, const Variable& b) {
    return compare(Op::kGreaterEq, "GreaterEqual", a, b);
}

Variable Vec2(const Variable& x, const Variable& y) { return compose({x, y}); }
Variable Vec3(const Variable& x, const Variable& y, const Variable& z) {
    return compose({x, y, z});
}
Variable Vec3(const Variable& xy, const Variable& z) { return compose({xy, z}); }
Variable Vec4(const Variable& x, const Variable& y, const Variable& z, const Variable& w) {
    return compose({x, y, z, w});
}
Variable Vec4(const Variable& xyz, const Variable& w) { return compose({xyz, w}); }
Variable GetX(const Variable& v) { return extract(v, 0, 1); }
Variable GetY(const Variable& v) { return extract(v, 1, 1); }
Variable GetZ(const Variable& v) { return extract(v, 2, 1); }
Variable GetW(const Variable& v) { return extract(v, 3, 1); }
Variable Dot(const Variable& a, const Variable& b) {
    require(a.getVType() == b.getVType() && a.getVType() != FLOAT,
            "Dot takes two equal vector types");
    return ew_fixed(Op::kDot, "Dot", FLOAT, {a, b},
                    [](const Variables& xs, const Variable&, const Variable& gy, uint32_t i) {
                        return Mul(gy, xs[i == 0 ? 1 : 0]);
                    });
}
Variable CompSum(const Variable& v) {
    if (v.getVType() == FLOAT) {
        return v;
    }
    const uint32_t n = NumComponents(v.getVType());
    return ew_fixed(Op::kCompSum, "CompSum", FLOAT, {v},
                    [n](const Variables&, const Variable&, const Variable& gy, uint32_t) {
                        return replicate(gy, n);
                    });
}

Variable Broadcast(const Variable& x, ImgSize size) {
    require(x.getImgSize().isUniform(), "Broadcast: input must be {1,1}");
    if (size.isUniform()) {
        return x;
    }
    return make_op({Op::kCopy, "Broadcast", x.getVType(), size,
                    [](const Variables&, const Variable&, const Variable& gy, uint32_t) {
                        return Sum(gy);
                    }},
                   {x});
}
Variable Sum(const Variable& x) {
    Variable cur = x;
    while (!cur.getImgSize().isUniform()) {
        cur = reduce2x2(cur);
    }
    return cur;
}
Variable Mean(const Variable& x) {
    const ImgSize s = x.getImgSize();
    const float inv = 1.f / (float(s.w) * float(s.h) * float(NumComponents(x.getVType())));
    return Mul(CompSum(Sum(x)), Float(inv));
}
Variable SumPixelWise(const Variables& xs) {
    require(!xs.empty(), "SumPixelWise needs inputs");
    Variables level = xs;
    while (level.size() > 1) {
        Variables next;
        for (size_t i = 0; i < level.size(); i += 4) {
            const size_t n = std::min<size_t>(4, level.size() - i);
            if (n == 1) {
                next.push_back(level[i]);
            } else {
                next.push_back(sum_pw_flat(Variables(level.begin() + i, level.begin() + i + n)));
            }
        }
        level = std::move(next);
    }
    return level[0];
}
Variable StopGradient(const Variable& x) {
    return make_op({Op::kCopy, "StopGradient", x.getVType(), x.getImgSize(), kNull}, {x});
}

Variable ScreenCoord(ImgSize size) {
    return make_op({Op::kScreenCoord, "ScreenCoord", VEC2, size, kNull}, {});
}
Variable Rasterize(const Variable& clip, const Variable& attr, const Variable& faces,
                   ImgSize screen) {
    require(clip.getVType() == VEC4 && clip.getImgSize().h == 1, "Rasterize: clip VEC4 {V,1}");
    return make_op({Op::kRasterize, "Rasterize", attr.getVType(), screen, kNull},
                   {clip, attr, faces});
}
Variable RasterizeFaceId(const Variable& clip, const Variable& dummy, const Variable& faces,
                         ImgSize screen) {
    return make_op({Op::kRasterizeFaceId, "RasterizeFaceId", FLOAT, screen, kNull},
                   {clip, dummy, faces});
}
Variable SoftClip(const Variable& clip, const Variable& faces, ImgSize screen, float radius) {
    const ImgSize out = {faces.getImgSize().w * 3, 1};
    return make_op({Op::kSoftClip, "SoftClip", VEC4, out, kNull}, {clip, faces}, {}, screen.w,
                   screen.h, radius);
}
static Variable rasterize_soft(const Variables& xs, ImgSize screen, float radius, bool peel) {
    BwdFn b = [radius](const Variables& in, const Variable& y, const Variable& gy,
                       uint32_t i) -> Variable {
        if (i != 3) {
            return nullptr;
        }
        const Variable& vf = in[5];
        const Variable wide = special(Op::kGatherDistGrad, "GatherDistGrad", VEC4,
                                      {in[3].getImgSize().w, vf.getImgSize().h},
                                      {gy, y, in[3], in[4], vf}, 0, 0, radius, 1);
        return special(Op::kColSum, "ColSum", VEC4, {wide.getImgSize().w, 1}, {wide});
    };
    return make_op({Op::kRasterizeSoft, "RasterizeSoft", VEC4, screen, b}, xs, {}, screen.w,
                   screen.h, radius, peel ? 1 : 0);
}
Variable RasterizeSoft(const Variable& soft, const Variable& fid, const Variable& fsoft,
                       const Variable& clip, const Variable& faces, const Variable& vf,
                       ImgSize screen, float radius) {
    return rasterize_soft({soft, fid, fsoft, clip, faces, vf}, screen, radius, false);
}
Variable RasterizeSoft(const Variable& soft, const Variable& fid, const Variable& fsoft,
                       const Variable& clip, const Variable& faces, const Variable& vf,
                       const Variable& prev, ImgSize screen, float radius) {
    return rasterize_soft({soft, fid, fsoft, clip, faces, vf, prev}, screen, radius, true);
}
Variable LookupFaces(const Variable& attr, const Variable& faces, const Variable& vf,
                     uint32_t corner) {
    require(corner < 3, "LookupFaces: corner 0..2");
    return make_op({Op::kLookupFaces, "LookupFaces", attr.getVType(), {faces.getImgSize().w, 1},
                    [corner](const Variables& xs, const Variable&, const Variable& gy,
                             uint32_t i) -> Variable {
                        if (i != 0) {
                            return nullptr;
                        }
                        return special(Op::kLookupFacesBwd, "LookupFacesBwd", gy.getVType(),
                                       xs[0].getImgSize(), {gy, xs[1], xs[2]}, corner);
                    }},
                   {attr, faces, vf}, {}, corner);
}
Variable FaceFetch(const Variable& tri, const Variable& idx, const Variable& p0,
                   const Variable& p1, const Variable& p2, const Variable& seed, float radius,
                   uint32_t n_samples) {
    return make_op({Op::kFaceFetch, "FaceFetch", tri.getVType(), idx.getImgSize(),
                    [radius, n_samples](const Variables& xs, const Variable&, const Variable& gy,
                                        uint32_t i) -> Variable {
                        if (i != 0) {
                            return nullptr;
                        }
                        return special(Op::kFaceFetchBwd, "FaceFetchBwd", gy.getVType(),
                                       xs[0].getImgSize(), {gy, xs[1], xs[2], xs[3], xs[4], xs[5]},
                                       n_samples, 0, radius);
                    }},
                   {tri, idx, p0, p1, p2, seed}, {}, n_samples, 0, radius);
}
Variable AntiAlias(const Variable& img, const Variable& tri, const Variable& clip,
                   const Variable& faces, const Variable& vf, const Variable& seed,
                   uint32_t n_samples) {
    return make_op({Op::kAntiAlias, "AntiAlias", img.getVType(), img.getImgSize(),
                    [n_samples](const Variables& xs, const Variable&, const Variable& gy,
                                uint32_t i) -> Variable {
                        if (i == 0) {
                            return special(Op::kAaBwdImg, "AntiAliasBwdImg", gy.getVType(),
                                           gy.getImgSize(), {gy, xs[1], xs[2], xs[3]});
                        }
                        if (i != 2) {
                            return nullptr;
                        }
                        const uint32_t nv = xs[2].getImgSize().w;
                        if (n_samples > 0) {
                            const Variable wide = special(
                                    Op::kAaBwdVtx, "AntiAliasBwdVtx", VEC4,
                                    {nv, xs[4].getImgSize().h},
                                    {gy, xs[0], xs[1], xs[2], xs[3], xs[4], xs[5]}, n_samples, 0,
                                    0.f, 1);
                            return special(Op::kColSum, "ColSum", VEC4, {nv, 1}, {wide});
                        }
                        return special(Op::kAaBwdVtx, "AntiAliasBwdVtx", VEC4, {nv, 1},
                                       {gy, xs[0], xs[1], xs[2], xs[3], xs[4], xs[5]}, 0);
                    }},
                   {img, tri, clip, faces, vf, seed}, {}, n_samples);
}

}  // namespace F

Variable operator+(const Variable& a, const Variable& b) { return F::Add(a, b); }
Variable operator-(const Variable& a, const Variable& b) { return F::Sub(a, b); }
Variable operator*(const Variable& a, const Variable& b) { return F::Mul(a, b); }
Variable operator/(const Variable& a, const Variable& b) { return F::Div(a, b); }
Variable operator+(const Variable& a, float b) { return F::Add(a, F::Float(b)); }
Variable operator-(const Variable& a, float b) { return F::Sub(a, F::Float(b)); }
Variable operator*(const Variable& a, float b) { return F::Mul(a, F::Float(b)); }
Variable operator/(const Variable& a, float b) { return F::Div(a, F::Float(b)); }
Variable operator+(float a, const Variable& b) { return F::Add(F::Float(a), b); }
Variable operator-(float a, const Variable& b) { return F::Sub(F::Float(a), b); }
Variable operator*(float a, const Variable& b) { return F::Mul(F::Float(a), b); }
Variable operator/(float a, const Variable& b) { return F::Div(F::Float(a), b); }
Variable operator-(const Variable& x) { return F::Neg(x); }

// ---- BuildBackward (src/core/build_backward.cpp:13-149) --------------------

namespace {

Variable sum_to_shape(const Variable& grad, const Variable& target) {
    Variable g = grad;
    const uint32_t nt = NumComponents(target.getVType());
    if (NumComponents(g.getVType()) != nt) {
        require(nt == 1, "gradient has more components than its non-scalar target");
        g = F::CompSum(g);
    }
    if (target.getImgSize().isUniform() && !g.getImgSize().isUniform()) {
        g = F::Sum(g);
    } else if (!target.getImgSize().isUniform() && g.getImgSize().isUniform()) {
        g = F::Broadcast(g, target.getImgSize());
    }
    require(g.getImgSize() == target.getImgSize(), "gradient does not reduce to its target size");
    return g;
}

// <=4-ary sequential sums, level by level, in list order
Variable sum_contribs(Variables c) {
    while (c.size() > 1) {
        Variables next;
        for (size_t i = 0; i < c.size(); i += 4) {
            const size_t n = std::min<size_t>(4, c.size() - i);
            if (n == 1) {
                next.push_back(c[i]);
            } else {
                next.push_back(sum_pw_flat(Variables(c.begin() + i, c.begin() + i + n)));
            }
        }
        c = std::move(next);
    }
    return c[0];
}

}  // namespace

std::tuple<Variables, Variables> BuildBackward(const Variable& loss) {
    require((bool)loss, "null loss");
    require(loss.getVType() != IVEC3, "the loss must be a float image");
    std::map<Variable, Variables> contribs;  // ordered by id
    auto later = [](const std::shared_ptr<FunctionNode>& a, const std::shared_ptr<FunctionNode>& b) {
        return a->id < b->id;
    };
    std::priority_queue<std::shared_ptr<FunctionNode>, std::vector<std::shared_ptr<FunctionNode>>,
                        decltype(later)>
            queue(later);
    std::unordered_set<uint64_t> seen;
    contribs[loss] = {F::Float(1.f)};
    if (loss.node()->creator) {
        queue.push(loss.node()->creator);
    }
    while (!queue.empty()) {
        Function fn(queue.top());
        queue.pop();
        if (!seen.insert(fn.id()).second) {
            continue;
        }
        const Variable y = fn.getOutputVar();
        auto it = contribs.find(y);
        if (it == contribs.end()) {
            continue;
        }
        Variable gy = sum_contribs(it->second);
        contribs.erase(it);
        const uint32_t ny = NumComponents(y.getVType());
        if (NumComponents(gy.getVType()) == 1 && ny > 1) {
            gy = F::Mul(gy, ny == 2 ? F::Vec2(1.f, 1.f)
                                    : ny == 3 ? F::Vec3(1.f, 1.f, 1.f) : F::Vec4(1.f, 1.f, 1.f, 1.f));
        }
        if (gy.getImgSize().isUniform() && !y.getImgSize().isUniform()) {
            gy = F::Broadcast(gy, y.getImgSize());
        }
        const Variables xs = fn.getInputVars();
        for (uint32_t i = 0; i < xs.size(); i++) {
            if (!xs[i].getRequiresGrad()) {
                continue;
            }
            Variable gx = fn.buildBwd(gy, i);
            if (!gx) {
                continue;
            }
            contribs[xs[i]].push_back(sum_to_shape(gx, xs[i]));
            if (xs[i].node()->creator) {
                queue.push(xs[i].node()->creator);
            }
        }
    }
    Variables leaves, grads;
    for (auto& [x, g] : contribs) {
        if (x == loss) {
            continue;
        }
        leaves.push_back(x);
        grads.push_back(sum_to_shape(sum_contribs(g), x));
    }
    return {leaves, grads};
}

// ---- device kernels -----------------------------------------------------------

namespace {

struct EwIn {
    const float* p;
    uint32_t nc;
    uint32_t uniform;
};

struct EwArgs {
    int op;
    uint32_t n_in;
    uint32_t ny;
    uint32_t a0;
    size_t n_px;
    EwIn in[4];
    float* out;
};

__device__ __forceinline__ float comp(const EwIn& x, size_t p, uint32_t c) {
    const size_t q = x.uniform ? 0 : p;
    return x.p[q * x.nc + (x.nc == 1 ? 0 : c)];
}

__device__ __forceinline__ float std_min(float a, float b) { return b < a ? b : a; }
__device__ __forceinline__ float std_max(float a, float b) { return a < b ? b : a; }

__global__ __launch_bounds__(256) void k_elementwise(EwArgs A) {
    const size_t p = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= A.n_px) {
        return;
    }
    float* y = A.out + p * A.ny;
    const Op op = (Op)A.op;
    if (op == Op::kCompose) {
        uint32_t o = 0;
        for (uint32_t i = 0; i < A.n_in; i++) {
            for (uint32_t c = 0; c < A.in[i].nc; c++) {
                y[o++] = comp(A.in[i], p, c);
            }
        }
        return;
    }
    if (op == Op::kExtract) {
        const size_t q = A.in[0].uniform ? 0 : p;
        for (uint32_t c = 0; c < A.ny; c++) {
            y[c] = A.in[0].p[q * A.in[0].nc + A.a0 + c];
        }
        return;
    }
    if (op == Op::kDot || op == Op::kCompSum) {
        float acc = 0.f;
        for (uint32_t c = 0; c < A.in[0].nc; c++) {
            acc += op == Op::kDot ? comp(A.in[0], p, c) * comp(A.in[1], p, c) : comp(A.in[0], p, c);
        }
        y[0] = acc;
        return;
    }
    for (uint32_t c = 0; c < A.ny; c++) {
        const float a = comp(A.in[0], p, c);
        const float b = A.n_in > 1 ? comp(A.in[1], p, c) : 0.f;
        float r = 0.f;
        switch (op) {
            case Op::kAdd: r = a + b; break;
            case Op::kSub: r = a - b; break;
            case Op::kMul: r = a * b; break;
            case Op::kDiv: r = a / b; break;
            case Op::kNeg: r = -a; break;
            case Op::kSqrt: r = sqrtf(a); break;
            case Op::kAbs: r = fabsf(a); break;
            case Op::kSign: r = (float)((a > 0.f) - (a < 0.f)); break;
            case Op::kExp: r = libc_expf(a); break;
            case Op::kLog: r = logf(a); break;
            case Op::kPow: r = powf(a, b); break;
            case Op::kMax: r = std_max(a, b); break;
            case Op::kMin: r = std_min(a, b); break;
            case Op::kClamp: r = std_min(std_max(a, b), comp(A.in[2], p, c)); break;
            case Op::kStep: r = b < a ? 0.f : 1.f; break;
            case Op::kSigmoid: r = 1.f / (1.f + libc_expf(-a)); break;
            case Op::kLess: r = (float)(a < b); break;
            case Op::kLessEq: r = (float)(a <= b); break;
            case Op::kGreater: r = (float)(a > b); break;
            case Op::kGreaterEq: r = (float)(a >= b); break;
            case Op::kCopy: r = a; break;
            case Op::kSumPw: {
                float acc = 0.f;
                for (uint32_t i = 0; i < A.n_in; i++) {
                    acc += comp(A.in[i], p, c);
                }
                r = acc;
                break;
            }
            default: break;
        }
        y[c] = r;
    }
}

__global__ __launch_bounds__(256) void k_fill(float* y, uint32_t n, float v0, float v1, float v2,
                                              float v3) {
    const uint32_t c = threadIdx.x;
    if (c < n) {
        y[c] = c == 0 ? v0 : c == 1 ? v1 : c == 2 ? v2 : v3;
    }
}

// Reduce2x2Sum: each output pixel sums its 2x2 source block in row order
// from 0 (the reference CPU kernel's accumulation order).
__global__ __launch_bounds__(256) void k_reduce2x2(const float* x, uint32_t sw, uint32_t sh,
                                                   uint32_t nc, uint32_t ow, uint32_t oh,
                                                   float* y) {
    const uint32_t q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= ow * oh) {
        return;
    }
    const uint32_t ox = q % ow, oy = q / ow;
    for (uint32_t c = 0; c < nc; c++) {
        float acc = 0.f;
        for (uint32_t dy = 0; dy < 2; dy++) {
            for (uint32_t dx = 0; dx < 2; dx++) {
                const uint32_t sx = 2 * ox + dx, sy = 2 * oy + dy;
                if (sx < sw && sy < sh) {
                    acc += x[((size_t)sy * sw + sx) * nc + c];
                }
            }
        }
        y[(size_t)q * nc + c] = acc;
    }
}

__global__ __launch_bounds__(256) void k_upsample2x(const float* x, uint32_t sw, uint32_t nc,
                                                    uint32_t ow, uint32_t oh, float* y) {
    const uint32_t q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= ow * oh) {
        return;
    }
    const uint32_t ox = q % ow, oy = q / ow;
    for (uint32_t c = 0; c < nc; c++) {
        y[(size_t)q * nc + c] = x[((size_t)(oy / 2) * sw + ox / 2) * nc + c];
    }
}

__global__ __launch_bounds__(256) void k_screen_coord(uint32_t w, uint32_t h, float* y) {
    const uint32_t q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= w * h) {
        return;
    }
    y[2 * (size_t)q + 0] = (float)(q % w) + 0.5f;
    y[2 * (size_t)q + 1] = (float)(q / w) + 0.5f;
}

uint32_t blocks(size_t n) { return (uint32_t)((n + 255) / 256); }

}  // namespace

// ---- DressiAD ---------------------------------------------------------------

struct DressiAD::Impl {
    dressi_ctx* ctx = nullptr;
    Variable loss;
    Optimizer optimizer;
    bool grads_built = false;
    Variables leaves, grads;
    Variables outputs;
    std::vector<std::pair<Variable, Variable>> updates;
    std::unordered_map<const VariableNode*, float*> bufs;
    std::vector<std::shared_ptr<VariableNode>> keep;  // owners of `bufs` keys
    std::vector<std::shared_ptr<FunctionNode>> plan;
    bool plan_dirty = true;

    static size_t count(const VariableNode& n) {
        return (size_t)n.size.w * n.size.h * NumComponents(n.vtype);
    }
    float* buf(const std::shared_ptr<VariableNode>& n) {
        auto it = bufs.find(n.get());
        if (it != bufs.end()) {
            return it->second;
        }
        void* p = nullptr;
        check(dressi_malloc(ctx, &p, std::max<size_t>(count(*n), 1) * sizeof(float)));
        check(dressi_memset(ctx, p, 0, std::max<size_t>(count(*n), 1) * sizeof(float)));
        bufs[n.get()] = (float*)p;
        keep.push_back(n);
        return (float*)p;
    }
    static void check(int rc) {
        if (rc != DRESSI_OK) {
            throw DressiError(std::string("HIP executor: ") + dressi_last_error());
        }
    }

    void build_grads() {
        if (grads_built || !loss) {
            return;
        }
        grads_built = true;
        std::tie(leaves, grads) = BuildBackward(loss);
        if (optimizer) {
            const Variables updated = optimizer(leaves, grads);
            require(updated.size() == leaves.size(), "the optimizer must return one value per leaf");
            for (size_t i = 0; i < leaves.size(); i++) {
                updates.emplace_back(leaves[i], updated[i]);
            }
        }
        plan_dirty = true;
    }

    void build_plan() {
        build_grads();
        std::vector<std::shared_ptr<VariableNode>> roots;
        if (loss) {
            roots.push_back(loss.node());
        }
        for (const auto& o : outputs) {
            roots.push_back(o.node());
        }
        for (const auto& u : updates) {
            roots.push_back(u.second.node());
        }
        std::unordered_set<const FunctionNode*> seen;
        std::vector<std::shared_ptr<FunctionNode>> fns;
        std::vector<std::shared_ptr<VariableNode>> stack = roots;
        while (!stack.empty()) {
            auto v = stack.back();
            stack.pop_back();
            if (!v->creator || !seen.insert(v->creator.get()).second) {
                continue;
            }
            fns.push_back(v->creator);
            for (const auto& x : v->creator->xs) {
                stack.push_back(x);
            }
        }
        std::sort(fns.begin(), fns.end(),
                  [](const auto& a, const auto& b) { return a->id < b->id; });
        plan = std::move(fns);
        for (const auto& fn : plan) {
            for (const auto& x : fn->xs) {
                buf(x);
            }
            buf(fn->y.lock());
        }
        plan_dirty = false;
    }

    void run(const FunctionNode& fn) {
        const auto y = fn.y.lock();
        float* out = buf(y);
        const uint32_t ny = NumComponents(y->vtype);
        const size_t n_px = (size_t)y->size.w * y->size.h;
        hipStream_t s = (hipStream_t)dressi_ctx_stream(ctx);
        std::vector<const float*> in;
        std::vector<const VariableNode*> xn;
        for (const auto& x : fn.xs) {
            in.push_back(buf(x));
            xn.push_back(x.get());
        }
        auto nc = [&](int i) { return NumComponents(xn[i]->vtype); };
        auto w_of = [&](int i) { return xn[i]->size.w; };
        auto h_of = [&](int i) { return xn[i]->size.h; };
        switch (fn.op) {
            case Op::kConst: {
                const auto& v = fn.cval;
                hipLaunchKernelGGL(k_fill, dim3(1), dim3(64), 0, s, out, (uint32_t)v.size(), v[0],
                                   v.size() > 1 ? v[1] : 0.f, v.size() > 2 ? v[2] : 0.f,
                                   v.size() > 3 ? v[3] : 0.f);
                break;
            }
            case Op::kReduce2x2:
                hipLaunchKernelGGL(k_reduce2x2, dim3(blocks(n_px)), dim3(256), 0, s, in[0], w_of(0),
                                   h_of(0), ny, y->size.w, y->size.h, out);
                break;
            case Op::kUpsample2x:
                hipLaunchKernelGGL(k_upsample2x, dim3(blocks(n_px)), dim3(256), 0, s, in[0],
                                   w_of(0), ny, y->size.w, y->size.h, out);
                break;
            case Op::kScreenCoord:
                hipLaunchKernelGGL(k_screen_coord, dim3(blocks(n_px)), dim3(256), 0, s, y->size.w,
                                   y->size.h, out);
                break;
            case Op::kRasterize:
                check(dressi_rasterize(ctx, in[0], w_of(0), in[1], nc(1), in[2], w_of(2), y->size.w,
                                       y->size.h, out));
                break;
            case Op::kRasterizeFaceId:
                check(dressi_rasterize_face_id(ctx, in[0], w_of(0), in[2], w_of(2), y->size.w,
                                               y->size.h, out));
                break;
            case Op::kSoftClip:
                check(dressi_soft_clip(ctx, in[0], w_of(0), in[1], w_of(1), fn.a0, fn.a1, fn.f0,
                                       out));
                break;
            case Op::kRasterizeSoft:
                check(dressi_rasterize_soft(ctx, in[0], in[1], in[2], in[3], w_of(3), in[4], w_of(4),
                                            fn.a0, fn.a1, fn.f0, fn.flag ? in[6] : nullptr, out));
                break;
            case Op::kLookupFaces:
                check(dressi_lookup_faces(ctx, in[0], nc(0), w_of(0), in[1], w_of(1), fn.a0, out));
                break;
            case Op::kLookupFacesBwd:
                check(dressi_lookup_faces_bwd(ctx, in[0], nc(0), in[1], w_of(1), in[2], w_of(2),
                                              h_of(2), fn.a0, out));
                break;
            case Op::kFaceFetch:
                check(dressi_face_fetch(ctx, in[0], nc(0), w_of(0), in[1], w_of(1), h_of(1), out));
                break;
            case Op::kFaceFetchBwd:
                check(dressi_face_fetch_bwd(ctx, in[0], nc(0), in[1], w_of(1), h_of(1), in[2], in[3],
                                            in[4], w_of(2), in[5], fn.f0, fn.a0, out));
                break;
            case Op::kGatherDistGrad:
                check(dressi_gather_dist_grad(ctx, in[0], in[1], in[2], w_of(2), in[3], w_of(3),
                                              in[4], h_of(4), fn.f0, fn.flag, w_of(1), h_of(1),
                                              out));
                break;
            case Op::kColSum:
                check(dressi_col_sum(ctx, in[0], nc(0), w_of(0), h_of(0), out));
                break;
            case Op::kAntiAlias:
                check(dressi_antialias(ctx, in[0], nc(0), in[1], in[2], w_of(2), in[3], w_of(3),
                                       w_of(0), h_of(0), out));
                break;
            case Op::kAaBwdImg:
                check(dressi_antialias_bwd_img(ctx, in[0], nc(0), in[1], in[2], w_of(2), in[3],
                                               w_of(3), w_of(0), h_of(0), out));
                break;
            case Op::kAaBwdVtx:
                check(dressi_antialias_bwd_vtx(ctx, in[0], in[1], nc(0), in[2], in[3], w_of(3),
                                               in[4], w_of(4), in[5], h_of(5), in[6], fn.a0,
                                               fn.flag, w_of(0), h_of(0), out));
                break;
            default: {
                require(fn.xs.size() <= 4, fn.name + ": more than 4 inputs");
                EwArgs A{};
                A.op = (int)fn.op;
                A.n_in = (uint32_t)fn.xs.size();
                A.ny = ny;
                A.a0 = fn.a0;
                A.n_px = n_px;
                for (size_t i = 0; i < fn.xs.size(); i++) {
                    A.in[i] = {in[i], nc((int)i), xn[i]->size.isUniform() ? 1u : 0u};
                }
                A.out = out;
                hipLaunchKernelGGL(k_elementwise, dim3(blocks(n_px)), dim3(256), 0, s, A);
                break;
            }
        }
        if (hipGetLastError() != hipSuccess) {
            throw DressiError(fn.name + ": kernel launch failed");
        }
    }
};

DressiAD::DressiAD(int device) : m_impl(new Impl) {
    Impl::check(dressi_ctx_create(device, &m_impl->ctx));
}
DressiAD::~DressiAD() {
    if (m_impl && m_impl->ctx) {
        dressi_ctx_synchronize(m_impl->ctx);
        for (auto& [n, p] : m_impl->bufs) {
            dressi_free(m_impl->ctx, p);
        }
        dressi_ctx_destroy(m_impl->ctx);
    }
}
void DressiAD::setLossVar(const Variable& loss) {
    m_impl->loss = loss;
    m_impl->grads_built = false;
    m_impl->plan_dirty = true;
}
void DressiAD::setOptimizer(const Optimizer& f) {
    m_impl->optimizer = f;
    m_impl->grads_built = false;
    m_impl->plan_dirty = true;
}
void DressiAD::markOutput(const Variable& v) {
    m_impl->outputs.push_back(v);
    m_impl->plan_dirty = true;
}
void DressiAD::addUpdate(const Variable& leaf, const Variable& value) {
    require(!leaf.node()->creator, "addUpdate: the target must be a leaf");
    require(leaf.getVType() == value.getVType() && leaf.getImgSize() == value.getImgSize(),
            "addUpdate: value and leaf shapes differ");
    m_impl->updates.emplace_back(leaf, value);
    m_impl->plan_dirty = true;
}
std::vector<std::pair<Variable, Variable>> DressiAD::inputGrads() const {
    m_impl->build_grads();
    std::vector<std::pair<Variable, Variable>> r;
    for (size_t i = 0; i < m_impl->leaves.size(); i++) {
        r.emplace_back(m_impl->leaves[i], m_impl->grads[i]);
    }
    return r;
}
size_t DressiAD::getFuncCount() const {
    if (m_impl->plan_dirty) {
        m_impl->build_plan();
    }
    return m_impl->plan.size();
}
std::string DressiAD::getDeviceName() const {
    char b[256];
    Impl::check(dressi_ctx_device_name(m_impl->ctx, b, sizeof(b)));
    return b;
}
void DressiAD::execStep() {
    if (m_impl->plan_dirty) {
        m_impl->build_plan();
    }
    for (const auto& fn : m_impl->plan) {
        m_impl->run(*fn);
    }
    for (const auto& [leaf, value] : m_impl->updates) {
        if (hipMemcpyAsync(m_impl->buf(leaf.node()), m_impl->buf(value.node()),
                           Impl::count(*leaf.node()) * sizeof(float), hipMemcpyDeviceToDevice,
                           (hipStream_t)dressi_ctx_stream(m_impl->ctx)) != hipSuccess) {
            throw DressiError("execStep: update copy failed");
        }
    }
}
void DressiAD::sendImg(const Variable& v, const float* data) {
    require(!v.node()->creator, "sendImg: only leaves take host data");
    Impl::check(dressi_memcpy_h2d(m_impl->ctx, m_impl->buf(v.node()), data,
                                  Impl::count(*v.node()) * sizeof(float)));
}
std::vector<float> DressiAD::recvImg(const Variable& v) {
    std::vector<float> out(Impl::count(*v.node()));
    Impl::check(dressi_memcpy_d2h(m_impl->ctx, out.data(), m_impl->buf(v.node()),
                                  out.size() * sizeof(float)));
    Impl::check(dressi_ctx_synchronize(m_impl->ctx));
    return out;
}
dressi_ctx* DressiAD::context() const { return m_impl->ctx; }

}  // namespace dressi
