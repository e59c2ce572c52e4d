// graph.hip -- the Dressi-AD graph API (include/dressi/*.h): graph IR,
// the F:: op catalogue with each op's backward builder, BuildBackward and
// TraverseFuncs. Host code; the executor (DressiAD) is executor.hip.
//
// IR (include/dressi/variable.h, function.h, src/core/node.h:42-65): a
// Variable is a shared handle to a node holding its type, image size,
// creator and (weak) users; a Function holds its op, inputs, (weak) output,
// attributes and backward builder. Ids come from one counter, so creation
// order is a topological order, and the backward graph's summation order
// follows the reference's (node creation order is part of the numbers).
#include <algorithm>
#include <atomic>
#include <cstring>
#include <map>
#include <queue>
#include <sstream>
#include <unordered_set>

#include "graph_ir.h"

namespace dressi {

namespace {

std::atomic<uint64_t> g_next_id{1};

uint64_t next_id() { return g_next_id.fetch_add(1); }

}  // namespace

void ThrowDressiError(const std::string& msg, const char* file, int line) {
    std::ostringstream os;
    os << msg << " (" << file << ":" << line << ")";
    throw DressiError(os.str());
}

uint32_t NumComponents(VType t) {
    switch (t) {
        case FLOAT: return 1;
        case VEC2: return 2;
        case VEC3: return 3;
        case VEC4: return 4;
        case MAT2: return 4;
        case MAT3: return 9;
        case MAT4: return 16;
        case INT: return 1;
        case IVEC2: return 2;
        case IVEC3: return 3;
        case IVEC4: return 4;
        case UINT: return 1;
    }
    DRESSI_CHECK(false, "unknown VType");
}
bool IsIntVType(VType t) { return t == INT || t == IVEC2 || t == IVEC3 || t == IVEC4 || t == UINT; }
bool IsMatrixVType(VType t) { return t == MAT2 || t == MAT3 || t == MAT4; }
bool IsVectorVType(VType t) {
    return t == VEC2 || t == VEC3 || t == VEC4 || t == IVEC2 || t == IVEC3 || t == IVEC4;
}
const char* GlslTypeName(VType t) {
    switch (t) {
        case FLOAT: return "float";
        case VEC2: return "vec2";
        case VEC3: return "vec3";
        case VEC4: return "vec4";
        case MAT2: return "mat2";
        case MAT3: return "mat3";
        case MAT4: return "mat4";
        case INT: return "int";
        case IVEC2: return "ivec2";
        case IVEC3: return "ivec3";
        case IVEC4: return "ivec4";
        case UINT: return "uint";
    }
    return "float";
}
VType VecVTypeOf(uint32_t n, bool is_int) {
    DRESSI_CHECK(n >= 1 && n <= 4, "VecVTypeOf: 1..4 components");
    if (is_int) {
        return n == 1 ? INT : n == 2 ? IVEC2 : n == 3 ? IVEC3 : IVEC4;
    }
    return n == 1 ? FLOAT : n == 2 ? VEC2 : n == 3 ? VEC3 : VEC4;
}

bool IsElementwise(Op op) {
    switch (op) {
        case Op::kAdd: case Op::kSub: case Op::kMul: case Op::kDiv: case Op::kNeg:
        case Op::kSin: case Op::kCos: case Op::kTan: case Op::kAsin: case Op::kAcos:
        case Op::kAtan: case Op::kAtan2: case Op::kExp: case Op::kExp2: case Op::kLog:
        case Op::kLog2: case Op::kSqrt: case Op::kInvSqrt: case Op::kAbs: case Op::kSign:
        case Op::kFloor: case Op::kFract: case Op::kMod: case Op::kPow: case Op::kMax:
        case Op::kMin: case Op::kClamp: case Op::kMix: case Op::kStep: case Op::kSmoothStep:
        case Op::kSigmoid: case Op::kLess: case Op::kLessEq: case Op::kGreater:
        case Op::kGreaterEq: case Op::kExtract: case Op::kCompose: case Op::kDot:
        case Op::kCompSum: case Op::kCross: case Op::kCopy: case Op::kSumPw:
        case Op::kLength: case Op::kNormalize:
            return true;
        default:
            return false;
    }
}

static void require(bool ok, const std::string& msg) {
    if (!ok) {
        throw DressiError(msg);
    }
}

// ---- Variable / Function ------------------------------------------------------

Variable::Variable(VType vtype, ImgSize img_size) : m_node(std::make_shared<VariableNode>()) {
    m_node->id = next_id();
    m_node->vtype = vtype;
    m_node->size = img_size;
}
uint64_t Variable::id() const { return m_node->id; }
VType Variable::getVType() const { return m_node->vtype; }
void Variable::setVType(VType t) { m_node->vtype = t; }
ImgSize Variable::getImgSize() const { return m_node->size; }
void Variable::setImgSize(ImgSize s) { m_node->size = s; }
Function Variable::getCreator() const { return NodeAccess::Wrap(m_node->creator); }
void Variable::setCreator(const Function& creator) { m_node->creator = NodeAccess::Node(creator); }
std::vector<Function> Variable::getUsers() const {
    std::vector<Function> out;
    for (const auto& w : m_node->users) {
        if (auto u = w.lock()) {
            out.push_back(NodeAccess::Wrap(u));
        }
    }
    return out;
}
void Variable::addUser(const Function& user) { m_node->users.push_back(NodeAccess::Node(user)); }
bool Variable::getRequiresGrad() const { return m_node->req_grad; }
void Variable::setRequiresGrad(bool r) { m_node->req_grad = r; }
bool Variable::IsDirty() const { return m_node->dirty; }
void Variable::setDirty(bool d) { m_node->dirty = d; }

// `n` and everything computed downstream of it (through the users)
template <typename Fn>
static void for_downstream(const std::shared_ptr<VariableNode>& start, Fn&& fn) {
    std::unordered_set<const VariableNode*> seen;
    std::vector<std::shared_ptr<VariableNode>> stack = {start};
    while (!stack.empty()) {
        auto n = stack.back();
        stack.pop_back();
        if (!n || !seen.insert(n.get()).second) {
            continue;
        }
        fn(*n);
        for (const auto& wu : n->users) {
            if (auto u = wu.lock()) {
                if (auto y = u->y.lock()) {
                    stack.push_back(std::move(y));
                }
            }
        }
    }
}
void Variable::setRequiresGradRecursively(bool r) {
    for_downstream(m_node, [r](VariableNode& n) { n.req_grad = r; });
}
void Variable::setDirtyRecursively(bool d) {
    for_downstream(m_node, [d](VariableNode& n) { n.dirty = d; });
}

Function::Function(const std::string& code, ShaderType type, const BwdFunc& bwd_func)
    : m_node(std::make_shared<FunctionNode>()) {
    m_node->id = next_id();
    m_node->op = Op::kCustom;
    m_node->name = code;
    m_node->shader = type;
    m_node->bwd = bwd_func;
}
uint64_t Function::id() const { return m_node->id; }
std::string Function::getFwdCode() const { return m_node->name; }
ShaderType Function::getShaderType() const { return m_node->shader; }
Variables Function::getInputVars() const {
    Variables v;
    for (const auto& x : m_node->xs) {
        v.push_back(NodeAccess::Wrap(x));
    }
    return v;
}
Variable Function::getOutputVar() const { return NodeAccess::Wrap(m_node->y.lock()); }
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
    BwdFunc bwd;
};

Variable make_op(const OpSpec& s, const Variables& xs, std::vector<float> cval = {},
                 uint32_t a0 = 0, uint32_t a1 = 0, float f0 = 0.f, int flag = 0) {
    auto fn = std::make_shared<FunctionNode>();
    fn->id = next_id();
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
        fn->xs.push_back(NodeAccess::Node(x));
        NodeAccess::Node(x)->users.push_back(fn);
    }
    auto y = std::make_shared<VariableNode>();
    y->id = next_id();
    y->vtype = s.vtype;
    y->size = s.size;
    y->creator = fn;
    fn->y = y;
    return NodeAccess::Wrap(y);
}

Variable ew(Op op, const char* name, const Variables& xs, BwdFunc bwd) {
    return make_op({op, name, widest(xs), common_size(xs), std::move(bwd)}, xs);
}

Variable ew_fixed(Op op, const char* name, VType t, const Variables& xs, BwdFunc bwd) {
    return make_op({op, name, t, common_size(xs), std::move(bwd)}, xs);
}

const BwdFunc kNull = nullptr;

Variable const_vec(const char* name, std::vector<float> v) {
    const VType t = VecVTypeOf((uint32_t)v.size());
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
    return make_op({Op::kCompose, "Compose", VecVTypeOf(total), common_size(parts),
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
    return make_op({Op::kExtract, "ExtractComps", VecVTypeOf(n), v.getImgSize(),
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
    BwdFunc b = nullptr;
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

void require_float_image(const Variable& v, const char* what) {
    require(!IsIntVType(v.getVType()) && !IsMatrixVType(v.getVType()),
            std::string(what) + " must be a float image");
}

uint32_t mat_dim(VType t) { return t == MAT2 ? 2 : t == MAT3 ? 3 : 4; }

}  // namespace

bool IsInlineConst(const Variable& v) {
    const auto& c = NodeAccess::Node(v)->creator;
    return c && c->op == Op::kConst;
}

Variable Function::buildFwd(const Variables& xs) {
    require(m_node->xs.empty() && !m_node->y.lock(), "buildFwd: the function is already connected");
    for (const auto& x : xs) {
        require((bool)x, "buildFwd: null input");
        m_node->xs.push_back(NodeAccess::Node(x));
        NodeAccess::Node(x)->users.push_back(m_node);
    }
    auto y = std::make_shared<VariableNode>();
    y->id = next_id();
    y->vtype = xs.empty() ? FLOAT : widest(xs);
    y->size = xs.empty() ? ImgSize{} : common_size(xs);
    y->creator = m_node;
    m_node->y = y;
    return NodeAccess::Wrap(y);
}

// ---- F:: ------------------------------------------------------------------------

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

// math (src/core/f_ops.cpp:262-475: derivative graphs as the reference's)
Variable Sin(const Variable& x) {
    return unary(Op::kSin, "Sin", x, [](const Variable& xv, const Variable&) { return Cos(xv); });
}
Variable Cos(const Variable& x) {
    return unary(Op::kCos, "Cos", x,
                 [](const Variable& xv, const Variable&) { return Neg(Sin(xv)); });
}
Variable Tan(const Variable& x) {
    return unary(Op::kTan, "Tan", x,
                 [](const Variable&, const Variable& y) { return Add(Float(1.f), Mul(y, y)); });
}
Variable Asin(const Variable& x) {
    return unary(Op::kAsin, "Asin", x, [](const Variable& xv, const Variable&) {
        return InverseSqrt(Sub(Float(1.f), Mul(xv, xv)));
    });
}
Variable Acos(const Variable& x) {
    return unary(Op::kAcos, "Acos", x, [](const Variable& xv, const Variable&) {
        return Neg(InverseSqrt(Sub(Float(1.f), Mul(xv, xv))));
    });
}
Variable Atan(const Variable& x) {
    return unary(Op::kAtan, "Atan", x, [](const Variable& xv, const Variable&) {
        return Div(Float(1.f), Add(Float(1.f), Mul(xv, xv)));
    });
}
Variable Atan2(const Variable& y, const Variable& x) {
    return ew(Op::kAtan2, "Atan2", {y, x},
              [](const Variables& xs, const Variable&, const Variable& gy, uint32_t i) {
                  Variable denom = Add(Mul(xs[0], xs[0]), Mul(xs[1], xs[1]));
                  if (i == 0) {
                      return Div(Mul(gy, xs[1]), denom);
                  }
                  return Neg(Div(Mul(gy, xs[0]), denom));
              });
}
Variable Exp(const Variable& x) {
    return unary(Op::kExp, "Exp", x, [](const Variable&, const Variable& y) { return y; });
}
Variable Exp2(const Variable& x) {
    return unary(Op::kExp2, "Exp2", x, [](const Variable&, const Variable& y) {
        return Mul(y, Float(0.6931471805599453f));
    });
}
Variable Log(const Variable& x) {
    return unary(Op::kLog, "Log", x,
                 [](const Variable& xv, const Variable&) { return Div(Float(1.f), xv); });
}
Variable Log2(const Variable& x) {
    return unary(Op::kLog2, "Log2", x, [](const Variable& xv, const Variable&) {
        return Div(Float(1.4426950408889634f), xv);
    });
}
Variable Sqrt(const Variable& x) {
    return unary(Op::kSqrt, "Sqrt", x,
                 [](const Variable&, const Variable& y) { return Div(Float(0.5f), y); });
}
Variable InverseSqrt(const Variable& x) {
    return unary(Op::kInvSqrt, "InverseSqrt", x, [](const Variable&, const Variable& y) {
        return Mul(Float(-0.5f), Mul(y, Mul(y, y)));
    });
}
Variable Abs(const Variable& x) {
    return unary(Op::kAbs, "Abs", x, [](const Variable& xv, const Variable&) { return Sign(xv); });
}
Variable Sign(const Variable& x) { return unary(Op::kSign, "Sign", x, nullptr); }
Variable Floor(const Variable& x) { return unary(Op::kFloor, "Floor", x, nullptr); }
Variable Fract(const Variable& x) {
    return unary(Op::kFract, "Fract", x,
                 [](const Variable&, const Variable&) { return Float(1.f); });
}
Variable Mod(const Variable& x, const Variable& m) {
    return ew(Op::kMod, "Mod", {x, m},
              [](const Variables& xs, const Variable&, const Variable& gy, uint32_t i) {
                  if (i == 0) {
                      return gy;
                  }
                  return Neg(Mul(gy, Floor(Div(xs[0], xs[1]))));
              });
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
Variable Mix(const Variable& x0, const Variable& x1, const Variable& t) {
    return ew(Op::kMix, "Mix", {x0, x1, t},
              [](const Variables& xs, const Variable&, const Variable& gy, uint32_t i) {
                  if (i == 0) {
                      return Mul(gy, Sub(Float(1.f), xs[2]));
                  }
                  if (i == 1) {
                      return Mul(gy, xs[2]);
                  }
                  return Mul(gy, Sub(xs[1], xs[0]));
              });
}
Variable Step(const Variable& edge, const Variable& x) {
    return ew(Op::kStep, "Step", {edge, x}, kNull);
}
Variable SmoothStep(const Variable& e0, const Variable& e1, const Variable& x) {
    return ew(Op::kSmoothStep, "SmoothStep", {e0, e1, x},
              [](const Variables& xs, const Variable&, const Variable& gy, uint32_t i) -> Variable {
                  if (i != 2) {
                      return nullptr;  // no gradient toward the edges
                  }
                  Variable range = Sub(xs[1], xs[0]);
                  Variable t = Clamp(Div(Sub(xs[2], xs[0]), range), Float(0.f), Float(1.f));
                  Variable dt = Div(Mul(Float(6.f), Mul(t, Sub(Float(1.f), t))), range);
                  return Mul(gy, dt);
              });
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
    require(IsVectorVType(a.getVType()) && a.getVType() == b.getVType(),
            "Dot takes two equal vector types");
    return ew_fixed(Op::kDot, "Dot", FLOAT, {a, b},
                    [](const Variables& xs, const Variable&, const Variable& gy, uint32_t i) {
                        return Mul(gy, xs[i == 0 ? 1 : 0]);
                    });
}
Variable Cross(const Variable& a, const Variable& b) {
    require(a.getVType() == VEC3 && b.getVType() == VEC3, "Cross takes VEC3 inputs");
    return ew_fixed(Op::kCross, "Cross", VEC3, {a, b},
                    [](const Variables& xs, const Variable&, const Variable& gy, uint32_t i) {
                        return i == 0 ? Cross(xs[1], gy) : Cross(gy, xs[0]);
                    });
}
Variable Length(const Variable& v) {
    require(IsVectorVType(v.getVType()) || v.getVType() == FLOAT,
            "Length takes a float vector");
    return ew_fixed(Op::kLength, "Length", FLOAT, {v},
                    [](const Variables& xs, const Variable& y, const Variable& gy, uint32_t) {
                        return Mul(Div(gy, y), xs[0]);
                    });
}
Variable Distance(const Variable& a, const Variable& b) { return Length(Sub(a, b)); }
Variable Normalize(const Variable& v) {
    // backward (gy - y dot(y, gy)) / |x| (f_ops.cpp:719-743)
    return ew(Op::kNormalize, "Normalize", {v},
              [](const Variables& xs, const Variable& y, const Variable& gy, uint32_t) {
                  return Div(Sub(gy, Mul(y, Dot(y, gy))), Length(xs[0]));
              });
}
Variable Reflect(const Variable& incident, const Variable& normal) {
    return Sub(incident, Mul(Mul(Float(2.f), Dot(normal, incident)), normal));
}
Variable CompSum(const Variable& v) {
    if (v.getVType() == FLOAT) {
        return v;
    }
    require(IsVectorVType(v.getVType()) && !IsIntVType(v.getVType()),
            "CompSum takes a float vector");
    const uint32_t n = NumComponents(v.getVType());
    return ew_fixed(Op::kCompSum, "CompSum", FLOAT, {v},
                    [n](const Variables&, const Variable&, const Variable& gy, uint32_t) {
                        return replicate(gy, n);
                    });
}

Variable MatMul(const Variable& a, const Variable& b) {
    const VType ta = a.getVType(), tb = b.getVType();
    require(IsMatrixVType(ta), "MatMul: the left operand must be a matrix");
    const uint32_t dim = mat_dim(ta);
    const bool vec_rhs = IsVectorVType(tb);
    require(vec_rhs ? NumComponents(tb) == dim : tb == ta, "MatMul: dimension mismatch");
    return make_op({Op::kMatMul, "MatMul", vec_rhs ? tb : ta, common_size({a, b}),
                    [vec_rhs](const Variables& xs, const Variable&, const Variable& gy,
                              uint32_t i) -> Variable {
                        if (vec_rhs) {
                            return i == 0 ? OuterProduct(gy, xs[1]) : MatMul(Transpose(xs[0]), gy);
                        }
                        return i == 0 ? MatMul(gy, Transpose(xs[1])) : MatMul(Transpose(xs[0]), gy);
                    }},
                   {a, b}, {}, dim, vec_rhs ? 1u : 0u);
}
Variable Transpose(const Variable& m) {
    require(IsMatrixVType(m.getVType()), "Transpose takes a matrix");
    return make_op({Op::kTranspose, "Transpose", m.getVType(), m.getImgSize(),
                    [](const Variables&, const Variable&, const Variable& gy, uint32_t) {
                        return Transpose(gy);
                    }},
                   {m}, {}, mat_dim(m.getVType()));
}
Variable OuterProduct(const Variable& col, const Variable& row) {
    const VType tc = col.getVType();
    require(IsVectorVType(tc) && row.getVType() == tc, "OuterProduct takes two equal vectors");
    const uint32_t dim = NumComponents(tc);
    return make_op({Op::kOuter, "OuterProduct", dim == 2 ? MAT2 : dim == 3 ? MAT3 : MAT4,
                    common_size({col, row}),
                    [](const Variables& xs, const Variable&, const Variable& gy, uint32_t i) {
                        return i == 0 ? MatMul(gy, xs[1]) : MatMul(Transpose(gy), xs[0]);
                    }},
                   {col, row}, {}, dim);
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
Variable SumAll(const Variable& x) {
    require_float_image(x, "SumAll: the input");
    return make_op({Op::kSumAll, "SumAll", FLOAT, {1, 1}, kNull}, {x});
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
Variable SetFragDepth(const Variable& depth) {
    return make_op({Op::kSetFragDepth, "SetFragDepth", depth.getVType(), depth.getImgSize(),
                    [](const Variables&, const Variable&, const Variable& gy, uint32_t) {
                        return gy;
                    }},
                   {depth});
}
Variable PeelDepth(const Variable& frag_depth, const Variable& prev_frag_depth) {
    return make_op({Op::kPeelDepth, "PeelDepth", FLOAT,
                    common_size({frag_depth, prev_frag_depth}), kNull},
                   {frag_depth, prev_frag_depth});
}

Variable ScreenCoord(ImgSize size) {
    return make_op({Op::kScreenCoord, "ScreenCoord", VEC2, size, kNull}, {});
}
Variable Rasterize(const Variable& clip, const Variable& attr, const Variable& faces,
                   ImgSize screen) {
    require(clip.getVType() == VEC4 && clip.getImgSize().h == 1, "Rasterize: clip VEC4 {V,1}");
    require(NumComponents(attr.getVType()) <= 4, "Rasterize: attribute of 1..4 components");
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
    BwdFunc b = [radius](const Variables& in, const Variable& y, const Variable& gy,
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

Variable PixelFetch(const Variable& tex, uint32_t x_index, const Variable& row_idx) {
    require_float_image(tex, "PixelFetch: tex");
    require(x_index < tex.getImgSize().w, "PixelFetch: x out of range");
    require(row_idx.getVType() == FLOAT && row_idx.getImgSize().isUniform(),
            "PixelFetch: row_idx must be FLOAT {1,1}");
    return make_op({Op::kPixelFetch, "PixelFetch", tex.getVType(), {1, 1}, kNull}, {tex, row_idx},
                   {}, x_index);
}
Variable TileFetch(const Variable& atlas, const Variable& tile_idx, uint32_t tile_h) {
    require_float_image(atlas, "TileFetch: atlas");
    require(tile_h > 0 && atlas.getImgSize().h % tile_h == 0,
            "TileFetch: atlas height must be a multiple of tile_h");
    require(tile_idx.getVType() == FLOAT && tile_idx.getImgSize().isUniform(),
            "TileFetch: tile_idx must be FLOAT {1,1}");
    return make_op({Op::kTileFetch, "TileFetch", atlas.getVType(),
                    {atlas.getImgSize().w, tile_h}, kNull},
                   {atlas, tile_idx}, {}, tile_h);
}

Variable VertexNeighborMean(const Variable& pos, const Variable& nbrs) {
    require(pos.getVType() == VEC3 && pos.getImgSize().h == 1,
            "VertexNeighborMean: pos must be VEC3 {V,1}");
    return make_op({Op::kVertexNeighborMean, "VertexNeighborMean", VEC3, pos.getImgSize(), kNull},
                   {pos, nbrs});
}
Variable NormalConsistencyFaceTerm(const Variable& pos, const Variable& faces,
                                   const Variable& face_adj) {
    return make_op({Op::kNcFaceTerm, "NormalConsistencyFaceTerm", VEC3,
                    {faces.getImgSize().w, 1}, kNull},
                   {pos, faces, face_adj});
}
Variable NormalConsistencyVertexGrad(const Variable& face_term, const Variable& pos,
                                     const Variable& faces, const Variable& vf) {
    return make_op({Op::kNcVertexGrad, "NormalConsistencyVertexGrad", VEC3, pos.getImgSize(),
                    kNull},
                   {face_term, pos, faces, vf});
}

// textures: the inverse-UV table is held by the backward builder, not an
// input of the forward (f_ops.cpp:2605-2639, 2736-2780)
Variable Texture(const Variable& tex, const Variable& uv, const Variable& inv_uv) {
    require_float_image(tex, "Texture: the texture");
    require(!tex.getImgSize().isUniform() && uv.getVType() == VEC2 &&
                    inv_uv.getVType() == VEC4 && inv_uv.getImgSize() == tex.getImgSize(),
            "Texture: texture image, uv VEC2, inv_uv VEC4 of the texture size");
    return make_op({Op::kTexture, "Texture", tex.getVType(), uv.getImgSize(),
                    [inv_uv](const Variables& xs, const Variable&, const Variable& gy,
                             uint32_t i) -> Variable {
                        if (i != 0) {
                            return nullptr;
                        }
                        return special(Op::kGatherInvUv, "GatherByInverseUV", gy.getVType(),
                                       inv_uv.getImgSize(), {gy, inv_uv, xs[1]});
                    }},
                   {tex, uv});
}
Variable TextureBilinear(const Variable& tex, const Variable& uv, const Variable& inv_uv) {
    require_float_image(tex, "TextureBilinear: the texture");
    require(!tex.getImgSize().isUniform() && uv.getVType() == VEC2 &&
                    inv_uv.getVType() == VEC4 && inv_uv.getImgSize() == tex.getImgSize(),
            "TextureBilinear: texture image, uv VEC2, inv_uv VEC4 of the texture size");
    return make_op({Op::kTextureBilinear, "TextureBilinear", tex.getVType(), uv.getImgSize(),
                    [inv_uv](const Variables& xs, const Variable&, const Variable& gy,
                             uint32_t i) -> Variable {
                        if (i != 0) {
                            return nullptr;
                        }
                        return special(Op::kGatherInvUvBilinear, "GatherByInverseUVBilinear",
                                       gy.getVType(), inv_uv.getImgSize(), {gy, inv_uv, xs[1]});
                    }},
                   {tex, uv});
}
Variable EquirectSample(const Variable& map, const Variable& dir) {
    require_float_image(map, "EquirectSample: the map");
    require(!map.getImgSize().isUniform() && dir.getVType() == VEC3,
            "EquirectSample: map image, dir VEC3");
    const ImgSize msz = map.getImgSize();
    return make_op({Op::kEquirectSample, "EquirectSample", map.getVType(), dir.getImgSize(),
                    [msz](const Variables& xs, const Variable&, const Variable& gy,
                          uint32_t i) -> Variable {
                        if (i != 0) {
                            return nullptr;
                        }
                        return special(Op::kEquirectSampleBwd, "EquirectSampleBwd",
                                       gy.getVType(), msz, {gy, xs[1]});
                    }},
                   {map, dir});
}
Variable IrradianceConv(const Variable& env, ImgSize out_size) {
    require_float_image(env, "IrradianceConv: env");
    require(!env.getImgSize().isUniform() && !out_size.isUniform(),
            "IrradianceConv: env and output must be images");
    const ImgSize esz = env.getImgSize();
    return make_op({Op::kIrradianceConv, "IrradianceConv", env.getVType(), out_size,
                    [esz](const Variables&, const Variable&, const Variable& gy,
                          uint32_t) -> Variable {
                        return special(Op::kIrradianceConvBwd, "IrradianceConvBwd",
                                       gy.getVType(), esz, {gy});
                    }},
                   {env});
}
Variable PrefilterEnv(const Variable& env, ImgSize out_size, float roughness,
                      uint32_t n_samples) {
    require_float_image(env, "PrefilterEnv: env");
    return make_op({Op::kPrefilterEnv, "PrefilterEnv", env.getVType(), out_size, kNull}, {env},
                   {}, n_samples, 0, roughness);
}
Variable PrefilterConv(const Variable& env, ImgSize out_size, float roughness) {
    require_float_image(env, "PrefilterConv: env");
    require(!env.getImgSize().isUniform() && !out_size.isUniform(),
            "PrefilterConv: env and output must be images");
    const ImgSize esz = env.getImgSize();
    // the static per-output normaliser (a zero-input op, as the reference's)
    Variable norm = make_op({Op::kPrefilterConv, "PrefilterConvNorm", FLOAT, out_size, kNull},
                            {}, {}, esz.w, esz.h, roughness, 1);
    return make_op({Op::kPrefilterConv, "PrefilterConv", env.getVType(), out_size,
                    [esz, roughness](const Variables& xs, const Variable&, const Variable& gy,
                                     uint32_t i) -> Variable {
                        if (i != 0) {
                            return nullptr;
                        }
                        return special(Op::kPrefilterConvBwd, "PrefilterConvBwd", gy.getVType(),
                                       esz, {gy, xs[1]}, 0, 0, roughness);
                    }},
                   {env, norm}, {}, 0, 0, roughness, 0);
}
Variable BrdfIntegrationLut(ImgSize size, uint32_t n_samples) {
    return make_op({Op::kBrdfLut, "BrdfIntegrationLut", VEC2, size, kNull}, {}, {}, n_samples);
}
Variable AvgPool2x2(const Variable& x) { return Mul(reduce2x2(x), Float(0.25f)); }

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
Variable operator<(const Variable& a, const Variable& b) { return F::Less(a, b); }
Variable operator<(float a, const Variable& b) { return F::Less(F::Float(a), b); }
Variable operator<(const Variable& a, float b) { return F::Less(a, F::Float(b)); }
Variable operator<=(const Variable& a, const Variable& b) { return F::LessEqual(a, b); }
Variable operator>(const Variable& a, const Variable& b) { return F::Greater(a, b); }
Variable operator>=(const Variable& a, const Variable& b) { return F::GreaterEqual(a, b); }

Functions TraverseFuncs(const Variables& roots) {
    Functions funcs;
    std::unordered_set<uint64_t> seen_fn, seen_var;
    std::vector<Variable> stack;
    for (const auto& r : roots) {
        if (r) {
            stack.push_back(r);
        }
    }
    while (!stack.empty()) {
        Variable v = stack.back();
        stack.pop_back();
        if (!seen_var.insert(v.id()).second) {
            continue;
        }
        Function c = v.getCreator();
        if (!c || !seen_fn.insert(c.id()).second) {
            continue;
        }
        funcs.push_back(c);
        for (const auto& x : c.getInputVars()) {
            stack.push_back(x);
        }
    }
    std::sort(funcs.begin(), funcs.end(),
              [](const Function& a, const Function& b) { return a.id() < b.id(); });
    return funcs;
}

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
    require(!IsIntVType(loss.getVType()) && !IsMatrixVType(loss.getVType()),
            "the loss must be a float image");
    std::map<Variable, Variables> contribs;  // ordered by id
    auto later = [](const std::shared_ptr<FunctionNode>& a, const std::shared_ptr<FunctionNode>& b) {
        return a->id < b->id;
    };
    std::priority_queue<std::shared_ptr<FunctionNode>, std::vector<std::shared_ptr<FunctionNode>>,
                        decltype(later)>
            queue(later);
    std::unordered_set<uint64_t> seen;
    contribs[loss] = {F::Float(1.f)};
    if (NodeAccess::Node(loss)->creator) {
        queue.push(NodeAccess::Node(loss)->creator);
    }
    while (!queue.empty()) {
        Function fn = NodeAccess::Wrap(queue.top());
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
            if (NodeAccess::Node(xs[i])->creator) {
                queue.push(NodeAccess::Node(xs[i])->creator);
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

}  // namespace dressi
