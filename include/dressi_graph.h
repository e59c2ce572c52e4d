/* dressi_graph.h -- the Dressi-AD C++ graph API on the HIP library.
 *
 * Mirrors the reference's public graph API (include/dressi/variable.h:18-49,
 * function.h:25-51, f.h:12-330, dressi_ad.h:44-131) for the ops of the
 * silhouette / antialias / soft-raster paths: build a DAG of `Variable`s
 * with `F::` ops, differentiate it with `BuildBackward`
 * (src/core/build_backward.cpp:62-149), and run it with `DressiAD`, which
 * executes every node of the graph on one HIP device: elementwise nodes
 * through one generic kernel per node, the raster / gather ops through the
 * library's per-op kernels (dressi_hip.h). Graphs are evaluated in node
 * creation order with the reference CPU evaluator's float semantics (one
 * rounding per op, no contraction), so a graph built with the same
 * expressions gives the reference's numbers.
 *
 * Layouts follow the reference: an image of W x H pixels with 1..4 float
 * components per pixel, row-major, components tight ({V,1} arrays are
 * 1-row images; IVEC3 faces are stored as float ids).
 */
#pragma once

#include <cstdint>
#include <functional>
#include <memory>
#include <stdexcept>
#include <string>
#include <tuple>
#include <utility>
#include <vector>

#include "dressi_hip.h"

namespace dressi {

enum VType { FLOAT, VEC2, VEC3, VEC4, IVEC3 };

uint32_t NumComponents(VType t);

struct ImgSize {
    uint32_t w = 1;
    uint32_t h = 1;
    bool operator==(const ImgSize& o) const { return w == o.w && h == o.h; }
    bool operator!=(const ImgSize& o) const { return !(*this == o); }
    bool isUniform() const { return w == 1 && h == 1; }
};

class DressiError : public std::runtime_error {
public:
    explicit DressiError(const std::string& msg) : std::runtime_error(msg) {}
};

struct VariableNode;
struct FunctionNode;
class Function;

class Variable {
public:
    Variable(VType vtype = FLOAT, ImgSize img_size = {1, 1});
    Variable(std::nullptr_t) {}
    explicit operator bool() const { return m_node != nullptr; }
    bool operator==(const Variable& o) const { return m_node == o.m_node; }
    bool operator!=(const Variable& o) const { return m_node != o.m_node; }
    bool operator<(const Variable& o) const;  // by id

    uint64_t id() const;
    VType getVType() const;
    ImgSize getImgSize() const;
    Function getCreator() const;
    bool getRequiresGrad() const;
    void setRequiresGrad(bool req_grad);
    void setRequiresGradRecursively(bool req_grad = true);

    const std::shared_ptr<VariableNode>& node() const { return m_node; }
    explicit Variable(std::shared_ptr<VariableNode> node) : m_node(std::move(node)) {}

private:
    std::shared_ptr<VariableNode> m_node;
};
using Variables = std::vector<Variable>;

class Function {
public:
    Function() = default;
    explicit Function(std::shared_ptr<FunctionNode> node) : m_node(std::move(node)) {}
    explicit operator bool() const { return m_node != nullptr; }
    uint64_t id() const;
    const std::string& name() const;
    Variables getInputVars() const;
    Variable getOutputVar() const;
    // The gradient w.r.t. input `idx` given the output gradient (null: none)
    Variable buildBwd(const Variable& gy, uint32_t idx) const;
    const std::shared_ptr<FunctionNode>& node() const { return m_node; }

private:
    std::shared_ptr<FunctionNode> m_node;
};

namespace F {
// constants
Variable Float(float v);
Variable Vec2(float x, float y);
Variable Vec3(float x, float y, float z);
Variable Vec4(float x, float y, float z, float w);
// arithmetic / math (component- and {1,1}-broadcasting)
Variable Add(const Variable& a, const Variable& b);
Variable Sub(const Variable& a, const Variable& b);
Variable Mul(const Variable& a, const Variable& b);
Variable Div(const Variable& a, const Variable& b);
Variable Neg(const Variable& x);
Variable Sqrt(const Variable& x);
Variable Abs(const Variable& x);
Variable Sign(const Variable& x);
Variable Exp(const Variable& x);
Variable Log(const Variable& x);
Variable Pow(const Variable& x, const Variable& p);
Variable Max(const Variable& a, const Variable& b);
Variable Min(const Variable& a, const Variable& b);
Variable Clamp(const Variable& x, const Variable& lo, const Variable& hi);
Variable Step(const Variable& edge, const Variable& x);
Variable Sigmoid(const Variable& x);
Variable Less(const Variable& a, const Variable& b);
Variable LessEqual(const Variable& a, const Variable& b);
Variable Greater(const Variable& a, const Variable& b);
Variable GreaterEqual(const Variable& a, const Variable& b);
// vectors
Variable Vec2(const Variable& x, const Variable& y);
Variable Vec3(const Variable& x, const Variable& y, const Variable& z);
Variable Vec3(const Variable& xy, const Variable& z);
Variable Vec4(const Variable& x, const Variable& y, const Variable& z, const Variable& w);
Variable Vec4(const Variable& xyz, const Variable& w);
Variable GetX(const Variable& v);
Variable GetY(const Variable& v);
Variable GetZ(const Variable& v);
Variable GetW(const Variable& v);
Variable Dot(const Variable& a, const Variable& b);
Variable CompSum(const Variable& v);
// reductions / broadcast
Variable Broadcast(const Variable& x, ImgSize size);
Variable Sum(const Variable& x);   // -> {1,1} by 2x2 block sums
Variable Mean(const Variable& x);  // -> FLOAT {1,1}
Variable SumPixelWise(const Variables& xs);
Variable StopGradient(const Variable& x);
// screen-space ops of the path
Variable ScreenCoord(ImgSize size);
Variable Rasterize(const Variable& vtx_clip_pos, const Variable& vtx_attrib,
                   const Variable& faces, ImgSize screen_size);
Variable RasterizeFaceId(const Variable& vtx_clip_pos, const Variable& vtx_attrib_dummy,
                         const Variable& faces, ImgSize screen_size);
Variable SoftClip(const Variable& vtx_clip_hard_tex, const Variable& faces_tex,
                  ImgSize screen_size, float radius_px);
Variable RasterizeSoft(const Variable& vtx_clip_soft, const Variable& face_id,
                       const Variable& faces_soft, const Variable& vtx_clip_hard_tex,
                       const Variable& faces_tex, const Variable& vtx_faces_tex,
                       ImgSize screen_size, float radius_px);
Variable RasterizeSoft(const Variable& vtx_clip_soft, const Variable& face_id,
                       const Variable& faces_soft, const Variable& vtx_clip_hard_tex,
                       const Variable& faces_tex, const Variable& vtx_faces_tex,
                       const Variable& prev_shifted_depth, ImgSize screen_size,
                       float radius_px);
Variable LookupFaces(const Variable& vtx_attr, const Variable& faces_tex,
                     const Variable& vtx_faces_tex, uint32_t corner);
Variable FaceFetch(const Variable& tri_attr, const Variable& idx_img, const Variable& tri_prj_0,
                   const Variable& tri_prj_1, const Variable& tri_prj_2, const Variable& seed,
                   float radius_px, uint32_t n_samples = 4);
Variable AntiAlias(const Variable& img, const Variable& tri_id, const Variable& vtx_clip,
                   const Variable& faces_tex, const Variable& vtx_faces_tex, const Variable& seed,
                   uint32_t n_samples = 8);
}  // namespace F

Variable operator+(const Variable& a, const Variable& b);
Variable operator-(const Variable& a, const Variable& b);
Variable operator*(const Variable& a, const Variable& b);
Variable operator/(const Variable& a, const Variable& b);
Variable operator+(const Variable& a, float b);
Variable operator-(const Variable& a, float b);
Variable operator*(const Variable& a, float b);
Variable operator/(const Variable& a, float b);
Variable operator+(float a, const Variable& b);
Variable operator-(float a, const Variable& b);
Variable operator*(float a, const Variable& b);
Variable operator/(float a, const Variable& b);
Variable operator-(const Variable& x);

// Reverse-mode graph of `loss` (any float image: every pixel and component
// is seeded with 1). Returns the requires-grad leaves and their gradients.
std::tuple<Variables, Variables> BuildBackward(const Variable& loss);

// The executor (DressiAD, include/dressi/dressi_ad.h:44-131): roots are the
// loss, the marked outputs and the update values; execStep evaluates them
// from the current leaves, then copies each update value into its leaf.
class DressiAD {
public:
    using Optimizer = std::function<Variables(Variables, Variables)>;
    explicit DressiAD(int device = 0);
    ~DressiAD();
    DressiAD(const DressiAD&) = delete;
    DressiAD& operator=(const DressiAD&) = delete;

    void setLossVar(const Variable& loss_var);
    void setOptimizer(const Optimizer& optim_func);
    void markOutput(const Variable& var);
    void addUpdate(const Variable& input_leaf, const Variable& updated);
    std::vector<std::pair<Variable, Variable>> inputGrads() const;
    size_t getFuncCount() const;
    std::string getDeviceName() const;

    void execStep();
    // host data: W * H * NumComponents(vtype) floats, row-major
    void sendImg(const Variable& var, const float* data);
    std::vector<float> recvImg(const Variable& var);
    dressi_ctx* context() const;

private:
    struct Impl;
    std::unique_ptr<Impl> m_impl;
};

}  // namespace dressi
