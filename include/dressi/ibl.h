/* dressi/ibl.h -- split-sum IBL builders and lookups composed of F:: ops
 * (the reference's include/dressi/ibl.h:24-63, src/core/ibl.cpp:14-93).
 * Maps are equirectangular images; the prefiltered environment is one
 * image per roughness level. With a static environment the reactive cache
 * runs the precompute once. */
#ifndef DRESSI_IBL_H
#define DRESSI_IBL_H

#include <vector>

#include "dressi/types.h"
#include "dressi/variable.h"

namespace dressi {

// E(N) / pi of the environment pooled to at most 64 x 32
Variable BuildIrradianceSample(const Variable& env_img, ImgSize out_size = {32, 16});
// `levels` images from `top` (halving), roughness level / (levels - 1),
// GGX importance-sampled with n_samples taps (forward only)
std::vector<Variable> BuildPrefEnvironmentSample(const Variable& env_img, uint32_t levels = 5,
                                                 ImgSize top = {128, 64},
                                                 uint32_t n_samples = 256);
// the same levels by the deterministic GGX convolution (differentiable
// w.r.t. the environment), source pooled to at most 128 x 64
std::vector<Variable> BuildPrefEnvironmentSampleConv(const Variable& env_img,
                                                     uint32_t levels = 5,
                                                     ImgSize top = {128, 64});
Variable BuildBrdfIntegrationMap(ImgSize size = {256, 256}, uint32_t n_samples = 512);

Variable SampleIrradiance(const Variable& irrad, const Variable& normal);
// tent-weighted blend of the levels at lod = roughness * (levels - 1)
Variable SamplePrefEnvironment(const std::vector<Variable>& levels, const Variable& refl_dir,
                               const Variable& roughness);
Variable SampleBrdfLut(const Variable& lut, const Variable& n_dot_v, const Variable& roughness);

}  // namespace dressi

#endif  // DRESSI_IBL_H
