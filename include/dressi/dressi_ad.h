/* dressi/dressi_ad.h -- DressiAD, the executor of the Appendix-A graph API
 * on one HIP device (the reference's include/dressi/dressi_ad.h:22-136,
 * same methods and meaning; src/dressi_ad.cpp:24-696 is the behaviour it
 * keeps).
 *
 * execStep() walks the reference's build ladder -- backward graph,
 * optimizer wiring, traversal, packing, device plan -- only as far as the
 * last change requires, then runs one iteration: the whole iteration is one
 * replayed hipGraph (the reference replays one recorded command buffer),
 * followed by the end-of-frame copy-backs (optimizer outputs and addUpdate
 * pairs into their leaves). Leaves the user has not touched since the last
 * step are static: after setRebuildCounts' fast / full counts of steps with
 * the same dirty pattern, functions whose inputs are all static and whose
 * images are already computed are pruned (the reactive cache).
 *
 * Packing: PackingMode::RSP fuses every run of consecutive elementwise
 * functions of one image size into one kernel (a per-pixel program over
 * registers, the reference's substage), and hands the recognised example
 * graphs (the HardSoftRas / AA silhouette fit) to their fused plans;
 * PackingMode::Naive runs one kernel per function (the correctness
 * baseline). */
#ifndef DRESSI_DRESSI_AD_H
#define DRESSI_DRESSI_AD_H

#include <functional>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "dressi/types.h"
#include "dressi/variable.h"

typedef struct dressi_ctx dressi_ctx;

namespace dressi {

// One HIP device and stream shared by the DressiAD instances built on it
struct HipContext;
using HipContextPtr = std::shared_ptr<HipContext>;
// the reference's name of the shared-context handle
using VkContextPtr = HipContextPtr;

class DressiAD {
public:
    // takes the requires-grad leaves and their gradients, returns the
    // updated value of each leaf
    using Optimizer = std::function<Variables(Variables xs, Variables gxs)>;

    enum InitStatus {
        BACKWARD,
        OPTIMIZER,
        TRAVERSE,
        SUBSTAGE,
        STAGE,
        VULKAN,  // the device plan (kept under the reference's name)
        FINISHED,
    };

    enum class PackingMode {
        Naive,  // one kernel per function
        RSP,    // fused elementwise stages and recognised fused plans
    };

    DressiAD();
    explicit DressiAD(VkContextPtr ctx);
    ~DressiAD();
    DressiAD(const DressiAD&) = delete;
    DressiAD& operator=(const DressiAD&) = delete;

    // A context on device 0 (`debug` is accepted; the HIP runtime has no
    // validation layers)
    static VkContextPtr createContext(bool debug = false);
    // HIP extension: a context on device `device`
    static VkContextPtr createContextOnDevice(int device);

    void setLossVar(const Variable& loss_var);
    void setOptimizer(const Optimizer& optim_func);
    void setPackingMode(PackingMode mode);
    // steps with an unchanged dirty pattern before a fast (stage-level) /
    // full (function-level) rebuild prunes static cached branches; 0
    // disables either
    void setRebuildCounts(uint32_t fast, uint32_t full);
    // keep `var` computed and readable by recvImg
    void markOutput(const Variable& var);
    // copy `updated` into the leaf `input_leaf` at the end of every step
    // (GPU-resident optimizer state); may be called from the optimizer
    void addUpdate(const Variable& input_leaf, const Variable& updated);
    // keep every requires-grad leaf's gradient computed and readable
    void setGradOutputsEnabled(bool enable);
    std::vector<std::pair<Variable, Variable>> inputGrads() const;

    size_t getFuncCount() const;      // functions of the traversed graph
    size_t getStageCount() const;     // launch groups per step (1: one fused plan)
    size_t getSubStageCount() const;  // kernels per step
    std::string getDeviceName() const;

    void execStep();
    void execStepWithSends(const std::vector<std::pair<Variable, CpuImageView>>& items);
    // uploads, one step and the stacked download ({w, h * n}) of same-shape
    // images, with one synchronisation
    CpuImage execStepWithSendsAndRecvImgsStacked(
            const std::vector<std::pair<Variable, CpuImageView>>& sends, const Variables& recvs);

    // host -> device; before the first execStep the data is kept and
    // uploaded once device images exist
    void sendImg(const Variable& var, const CpuImage& cpu_img);
    void sendImg(const Variable& var, const CpuImageView& cpu_img);
    void sendImgs(const std::vector<std::pair<Variable, CpuImageView>>& items);
    CpuImage recvImg(const Variable& var);
    std::vector<CpuImage> recvImgs(const Variables& vars);
    CpuImage recvImgsStacked(const Variables& vars);

    // HIP extensions: which plan runs the graph ("generic" or
    // "fused:hardsoftras" / "fused:aa"), and the C-ABI context
    std::string getPlanName() const;
    dressi_ctx* context() const;

private:
    struct Impl;
    std::unique_ptr<Impl> m_impl;
};

}  // namespace dressi

#endif  // DRESSI_DRESSI_AD_H
