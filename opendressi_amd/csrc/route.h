// route.h -- hands a DressiAD graph that is one of the fit examples' to its
// fused plan. The silhouette fit: a graph that is the silhouette-fit example's
// (examples/silhouette_optimization/run.cpp:229-437: technique hardsoftras
// with one peel, or aa; all views each iteration; the in-graph Adam, with
// or without its regularisers at weight 0) to the fused silhouette plan
// (dressi_hsr_*), which runs the whole iteration as one replayed hipGraph.
//
// Recognition is structural: the example's graph is rebuilt with the F::
// ops from sizes and attributes read off the user's graph, and the two are
// compared from the roots down (op, attributes, constant values, input
// order, image types and sizes). The per-view MVP entries and the learning
// rate are free constants whose values the comparison reads; every other
// constant must be equal. The static leaf images the plan derives from the
// mesh (face ids, soft faces, the vertex-face table, the ones attribute)
// are checked against what the example sends before the plan is used; when
// they differ, or a later send does not fit, the route hands every leaf
// image (current optimiser state included) back to the generic executor.
#pragma once

#include <map>
#include <memory>
#include <string>
#include <utility>

#include "graph_ir.h"

typedef struct dressi_ctx dressi_ctx;

namespace dressi {

// What the executor holds after its traversal level
struct GraphRoots {
    Variable loss{nullptr};
    Variables input_vars, input_grad_vars, updated_vars;
    std::vector<std::pair<Variable, Variable>> extra_updates;  // (leaf, updated)
    Variables extra_outputs;
    bool grad_outputs = false;
    const Functions* funcs = nullptr;
};

// A fused plan standing in for the generic executor on a recognised graph.
class FusedRoute {
public:
    virtual ~FusedRoute() = default;

    virtual std::string name() const = 0;  // "fused:<plan>"
    virtual size_t kernels() const = 0;    // kernels per iteration

    // Leaf image from sendImg. false: `var` is computed by the graph (the
    // plan cannot take an image for it). Images of variables outside the
    // graph are ignored, as the generic executor never reads them.
    virtual bool Accept(const Variable& var, const CpuImageView& img) = 0;
    // One iteration on `ctx`'s stream. false: the leaf images do not fit
    // the plan; `back` then holds every leaf image the route has (current
    // optimiser state included) and the caller runs the graph itself.
    virtual bool Step(dressi_ctx* ctx, std::map<Variable, CpuImage>* back) = 0;
    // Every leaf image the route holds, current state included
    virtual void Export(std::map<Variable, CpuImage>* back) = 0;

    virtual bool Readable(const Variable& var) const = 0;
    virtual CpuImage Recv(const Variable& var) = 0;
};

// The silhouette route, else the texture route (tests/graph_tex.cpp's form
// of examples/texture_optimization/run.cpp:112-145: TextureBilinear on an
// RGBA texture, the RGB L2 image loss, the in-graph Adam, per-view clip and
// ScreenAttr images sent each step, on dressi_tex_* with
// DRESSI_TEX_EXTERNAL_CLIP), else the PBR route (tests/graph_pbr.cpp: the
// material + environment fit of examples/pbr_material_optimization/
// run.cpp:189-288 built with the examples' PBR graph builders, normal
// mapping off, AO 1, emissive 0, on dressi_pbr_* with the views' clip
// images); nullptr when none recognises the graph.
std::unique_ptr<FusedRoute> RecogniseFusedRoute(const GraphRoots& g);

class SilhouetteRoute : public FusedRoute {
public:
    // nullptr unless the graph is the example's
    static std::unique_ptr<SilhouetteRoute> Recognise(const GraphRoots& g);
    ~SilhouetteRoute() override;

    std::string name() const override;  // "fused:hardsoftras" / "fused:aa"
    size_t kernels() const override;
    bool Accept(const Variable& var, const CpuImageView& img) override;
    bool Step(dressi_ctx* ctx, std::map<Variable, CpuImage>* back) override;
    void Export(std::map<Variable, CpuImage>* back) override;
    bool Readable(const Variable& var) const override;
    CpuImage Recv(const Variable& var) override;

private:
    struct State;
    explicit SilhouetteRoute(std::unique_ptr<State> st);
    std::unique_ptr<State> st_;
};

class TextureRoute : public FusedRoute {
public:
    static std::unique_ptr<TextureRoute> Recognise(const GraphRoots& g);
    ~TextureRoute() override;

    std::string name() const override;  // "fused:texture"
    size_t kernels() const override;
    bool Accept(const Variable& var, const CpuImageView& img) override;
    bool Step(dressi_ctx* ctx, std::map<Variable, CpuImage>* back) override;
    void Export(std::map<Variable, CpuImage>* back) override;
    bool Readable(const Variable& var) const override;
    CpuImage Recv(const Variable& var) override;

private:
    struct State;
    explicit TextureRoute(std::unique_ptr<State> st);
    std::unique_ptr<State> st_;
};

class PbrRoute : public FusedRoute {
public:
    static std::unique_ptr<PbrRoute> Recognise(const GraphRoots& g);
    ~PbrRoute() override;

    std::string name() const override;  // "fused:pbr"
    size_t kernels() const override;
    bool Accept(const Variable& var, const CpuImageView& img) override;
    bool Step(dressi_ctx* ctx, std::map<Variable, CpuImage>* back) override;
    void Export(std::map<Variable, CpuImage>* back) override;
    bool Readable(const Variable& var) const override;
    CpuImage Recv(const Variable& var) override;

private:
    struct State;
    explicit PbrRoute(std::unique_ptr<State> st);
    std::unique_ptr<State> st_;
};

}  // namespace dressi
