// graph_ir.h -- the nodes behind dressi::Variable / dressi::Function
// (include/dressi/variable.h, function.h), shared by the graph builder
// (graph.hip) and the executor (executor.hip).
//
// A VariableNode is an image (type, size), its creator and its users; a
// FunctionNode an operation: its op code, inputs, output, attributes and
// backward builder. Node ids come from one counter, so creation order is a
// topological order (the reference's src/core/node.h:42-65 contract).
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <tuple>
#include <vector>

#include "dressi/dressi.h"

namespace dressi {

enum class Op : int {
    kCustom,  // a Function made from GLSL text: not executable here
    kConst,
    // elementwise (per pixel; {1,1} and 1-component inputs broadcast)
    kAdd, kSub, kMul, kDiv, kNeg,
    kSin, kCos, kTan, kAsin, kAcos, kAtan, kAtan2,
    kExp, kExp2, kLog, kLog2, kSqrt, kInvSqrt, kAbs, kSign, kFloor, kFract, kMod, kPow,
    kMax, kMin, kClamp, kMix, kStep, kSmoothStep, kSigmoid,
    kLess, kLessEq, kGreater, kGreaterEq,
    kExtract, kCompose, kDot, kCompSum, kCross, kLength, kNormalize, kCopy, kSumPw,
    // matrices (per pixel, up to 16 components)
    kMatMul, kTranspose, kOuter,
    // image-level
    kReduce2x2, kUpsample2x, kScreenCoord, kSumAll, kPixelFetch, kTileFetch, kAvgPool, kAvgPoolBwd,
    // raster / gather ops of the path (per-op entry points of the C ABI)
    kRasterize, kRasterizeFaceId, kSoftClip, kRasterizeSoft, kLookupFaces, kLookupFacesBwd,
    kFaceFetch, kFaceFetchBwd, kGatherDistGrad, kColSum, kAntiAlias, kAaBwdImg, kAaBwdVtx,
    kTexture, kGatherInvUv, kTextureBilinear, kGatherInvUvBilinear,
    kEquirectSample, kEquirectSampleBwd, kIrradianceConv, kIrradianceConvBwd,
    kPrefilterEnv, kPrefilterConv, kPrefilterConvBwd, kBrdfLut,
    kVertexNeighborMean, kNcFaceTerm, kNcVertexGrad,
    kSetFragDepth, kPeelDepth,  // raster-pass-only ops of the reference: not executable here
};

// Per-pixel elementwise op: one fused-stage instruction
bool IsElementwise(Op op);

struct VariableNode {
    uint64_t id = 0;
    VType vtype = FLOAT;
    ImgSize size;
    std::shared_ptr<FunctionNode> creator;
    std::vector<std::weak_ptr<FunctionNode>> users;
    bool req_grad = false;
    bool dirty = false;
};

struct FunctionNode {
    uint64_t id = 0;
    Op op = Op::kConst;
    std::string name;
    ShaderType shader = FRAG;
    std::vector<std::shared_ptr<VariableNode>> xs;
    std::weak_ptr<VariableNode> y;
    BwdFunc bwd;
    std::vector<float> cval;  // constant values
    uint32_t a0 = 0, a1 = 0;  // component offset / corner / sample count / size
    float f0 = 0.f;           // radius / roughness
    int flag = 0;             // wide gather / peel input present
};

// Access to the nodes of the public handles (the reference's NodeAccess)
struct NodeAccess {
    static const std::shared_ptr<VariableNode>& Node(const Variable& v) { return v.m_node; }
    static const std::shared_ptr<FunctionNode>& Node(const Function& f) { return f.m_node; }
    static Variable Wrap(std::shared_ptr<VariableNode> n) { return Variable(std::move(n)); }
    static Function Wrap(std::shared_ptr<FunctionNode> n) { return Function(std::move(n)); }
};

// Reverse-mode graph of `loss` (every pixel and component seeded with 1):
// the requires-grad leaves in creation order and their gradients
// (src/core/build_backward.cpp:62-149)
std::tuple<Variables, Variables> BuildBackward(const Variable& loss);

// The functions needed for `roots`, in creation (topological) order
// (src/core/build_backward.cpp:151-181)
Functions TraverseFuncs(const Variables& roots);

// A {1,1} constant created by F::Float / F::VecN (executed once, inlined
// into fused stages)
bool IsInlineConst(const Variable& v);

}  // namespace dressi
