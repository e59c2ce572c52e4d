// route.h -- hands a DressiAD graph that is the silhouette-fit example's
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

class SilhouetteRoute {
public:
    // nullptr unless the graph is the example's
    static std::unique_ptr<SilhouetteRoute> Recognise(const GraphRoots& g);
    ~SilhouetteRoute();

    std::string name() const;  // "fused:hardsoftras" / "fused:aa"
    size_t kernels() const;    // kernels per iteration

    // Leaf image from sendImg. false: `var` is computed by the graph (the
    // plan cannot take an image for it). Images of variables outside the
    // graph are ignored, as the generic executor never reads them.
    bool Accept(const Variable& var, const CpuImageView& img);
    // One iteration on `ctx`'s stream. false: the leaf images do not fit
    // the plan; `back` then holds every leaf image the route has (current
    // optimiser state included) and the caller runs the graph itself.
    bool Step(dressi_ctx* ctx, std::map<Variable, CpuImage>* back);
    // Every leaf image the route holds, current state included
    void Export(std::map<Variable, CpuImage>* back);

    bool Readable(const Variable& var) const;
    CpuImage Recv(const Variable& var);

private:
    struct State;
    explicit SilhouetteRoute(std::unique_ptr<State> st);
    std::unique_ptr<State> st_;
};

}  // namespace dressi
