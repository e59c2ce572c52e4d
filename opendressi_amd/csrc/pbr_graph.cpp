// pbr_graph.cpp -- the examples' split-sum PBR rendering graph
// (include/dressi_examples/pbr_graph.h; the reference's
// examples/common/pbr_graph.cpp:19-146). Host code: every builder only
// composes F:: nodes. The node sequence of each shading term follows the
// reference's, operand for operand, because the graph's floats (and so its
// gradients) depend on the order in which the terms are combined.
#include "dressi_examples/pbr_graph.h"

#include "dressi/ibl.h"

namespace dressi_examples {

using dressi::BuildBrdfIntegrationMap;
using dressi::BuildIrradianceSample;
using dressi::BuildPrefEnvironmentSample;
using dressi::BuildPrefEnvironmentSampleConv;
using dressi::ImgSize;
using dressi::SampleBrdfLut;
using dressi::SampleIrradiance;
using dressi::SamplePrefEnvironment;
using dressi::Variable;
namespace F = dressi::F;

namespace {

constexpr float kPi = 3.14159265358979324f;

// v / |v| with a 1e-12 floor under the squared length: background pixels
// rasterize to the zero vector, and a NaN there would survive the coverage
// composite (0 * NaN)
Variable unit_or_zero(const Variable& v) { return v * F::InverseSqrt(F::Dot(v, v) + 1e-12f); }

// the material maps sampled at the G-buffer's uv
struct Surface {
    Variable albedo{nullptr}, rough{nullptr}, metal{nullptr}, ao{nullptr}, emissive{nullptr};
};

Surface sample_surface(const PbrMaterialLeaves& mat, const Variable& uv, const Variable& inv_uv) {
    Surface s;
    s.albedo = F::TextureBilinear(mat.albedo, uv, inv_uv);
    const Variable mr = F::TextureBilinear(mat.mr, uv, inv_uv);
    s.rough = F::Clamp(F::GetY(mr), F::Float(0.045f), F::Float(1.f));
    s.metal = F::GetZ(mr);
    s.ao = F::GetX(F::TextureBilinear(mat.ao, uv, inv_uv));
    s.emissive = F::TextureBilinear(mat.emissive, uv, inv_uv);
    return s;
}

// the interpolated normal, optionally perturbed by the tangent-space map
// through the Gram-Schmidt frame (t, n x t * handedness, n)
Variable shading_normal(const PbrGBuffer& g, const PbrMaterialLeaves& mat, const Variable& inv_uv,
                        bool normal_mapping) {
    const Variable n0 = unit_or_zero(g.g_n);
    if (!normal_mapping) {
        return n0;
    }
    const Variable t0 = unit_or_zero(g.g_t - n0 * F::Dot(n0, g.g_t));
    const Variable b0 = F::Cross(n0, t0) * g.handed;
    const Variable nm = F::TextureBilinear(mat.normal_map, g.uv, inv_uv) * 2.f - 1.f;
    return unit_or_zero(t0 * F::GetX(nm) + b0 * F::GetY(nm) + n0 * F::GetZ(nm));
}

// Cook-Torrance with GGX distribution, Schlick-GGX geometry (k = (r+1)^2 / 8)
// and Schlick Fresnel for the point light, times its inverse-square radiance
Variable point_light(const Surface& s, const PbrFrameLeaves& fr, const Variable& p,
                     const Variable& n, const Variable& v, const Variable& n_dot_v,
                     const Variable& f0) {
    const Variable to_light = fr.light_pos - p;
    const Variable dist2 = F::Max(F::Dot(to_light, to_light), F::Float(1e-4f));
    const Variable l = unit_or_zero(to_light);
    const Variable h = unit_or_zero(v + l);
    const Variable n_dot_l = F::Max(F::Dot(n, l), F::Float(0.f));
    const Variable n_dot_h = F::Max(F::Dot(n, h), F::Float(0.f));
    const Variable v_dot_h = F::Max(F::Dot(v, h), F::Float(0.f));

    const Variable a = s.rough * s.rough;
    const Variable a2 = a * a;
    const Variable dd = n_dot_h * n_dot_h * (a2 - 1.f) + 1.f;
    const Variable ndf = a2 / (kPi * dd * dd);
    const Variable k = (s.rough + 1.f) * (s.rough + 1.f) / 8.f;
    const Variable geo_v = n_dot_v / (n_dot_v * (1.f - k) + k);
    const Variable geo_l = F::Max(n_dot_l, F::Float(1e-4f)) /
                           (F::Max(n_dot_l, F::Float(1e-4f)) * (1.f - k) + k);
    const Variable fres = f0 + (1.f - f0) * F::Pow(1.f - v_dot_h, F::Float(5.f));
    const Variable spec = fres * (ndf * geo_v * geo_l / (4.f * n_dot_v * n_dot_l + 1e-4f));
    const Variable kd = (1.f - fres) * (1.f - s.metal);
    const Variable radiance = fr.light_col / dist2;
    return (kd * s.albedo / kPi + spec) * radiance * n_dot_l;
}

// split-sum image-based light with the roughness-aware Schlick Fresnel
// (f0 + (max(1 - r, f0) - f0) (1 - n.v)^5), scaled by the occlusion
Variable image_light(const Surface& s, const PbrIblMaps& ibl, const Variable& n, const Variable& v,
                     const Variable& n_dot_v, const Variable& f0) {
    const Variable fres = f0 + (F::Max(1.f - s.rough, f0) - f0) *
                                       F::Pow(1.f - n_dot_v, F::Float(5.f));
    const Variable kd = (1.f - fres) * (1.f - s.metal);
    const Variable diffuse = SampleIrradiance(ibl.irr, n);
    const Variable refl = F::Reflect(F::Neg(v), n);
    const Variable pref = SamplePrefEnvironment(ibl.pref, refl, s.rough);
    const Variable ab = SampleBrdfLut(ibl.lut, n_dot_v, s.rough);
    const Variable spec = pref * (f0 * F::GetX(ab) + F::GetY(ab));
    return (kd * diffuse * s.albedo + spec) * s.ao;
}

// the environment along each pixel's view ray (screen y grows downwards,
// the camera's up axis upwards)
Variable background(const PbrFrameLeaves& fr, const PbrIblMaps& ibl, ImgSize screen) {
    const Variable sc = F::ScreenCoord(screen);
    const Variable nx = F::GetX(sc) * (2.f / float(screen.w)) - 1.f;
    const Variable ny = F::GetY(sc) * (2.f / float(screen.h)) - 1.f;
    return F::EquirectSample(ibl.env, fr.cam_fwd + fr.cam_right * nx - fr.cam_up * ny);
}

}  // namespace

PbrIblMaps BuildPbrIblMaps(const Variable& env, bool differentiable_prefilter) {
    PbrIblMaps m;
    m.env = env;
    m.irr = BuildIrradianceSample(env);
    m.pref = differentiable_prefilter ? BuildPrefEnvironmentSampleConv(env)
                                      : BuildPrefEnvironmentSample(env);
    m.lut = BuildBrdfIntegrationMap();
    return m;
}

PbrGBuffer BuildPbrGBuffer(const PbrGeometryLeaves& geom, ImgSize screen) {
    const auto raster = [&](const Variable& attr) {
        return F::Rasterize(geom.clip, attr, geom.faces, screen);
    };
    PbrGBuffer g;
    const Variable uvh = raster(geom.uvh);
    g.g_n = raster(geom.normal);
    g.g_t = raster(geom.tangent);
    g.g_p = raster(geom.wpos);
    g.uv = F::Vec2(F::GetX(uvh), F::GetY(uvh));
    g.mask = F::GetZ(uvh);
    // interpolated handedness is near +-1 on a face; the 1e-6 bias makes the
    // background's 0 read as +1
    g.handed = F::Sign(F::GetW(uvh) + 1e-6f);
    return g;
}

PbrOutputs BuildPbrShade(const PbrGBuffer& gbuf, const PbrMaterialLeaves& mat,
                         const PbrFrameLeaves& frame, const PbrIblMaps& ibl,
                         const Variable& inv_uv, ImgSize screen, bool normal_mapping) {
    const Surface s = sample_surface(mat, gbuf.uv, inv_uv);
    const Variable n = shading_normal(gbuf, mat, inv_uv, normal_mapping);
    const Variable v = unit_or_zero(frame.cam_pos - gbuf.g_p);
    const Variable n_dot_v = F::Max(F::Dot(n, v), F::Float(1e-4f));
    const Variable f0 = F::Mix(F::Vec3(0.04f, 0.04f, 0.04f), s.albedo, s.metal);

    const Variable direct = point_light(s, frame, gbuf.g_p, n, v, n_dot_v, f0);
    const Variable ambient = image_light(s, ibl, n, v, n_dot_v, f0);
    const Variable bg = background(frame, ibl, screen);

    PbrOutputs out;
    const Variable surface = direct + ambient + s.emissive;
    out.hdr = gbuf.mask * surface + (1.f - gbuf.mask) * bg;
    out.mapped = out.hdr / (out.hdr + 1.f);
    out.ldr = F::Pow(out.mapped, F::Float(1.f / 2.2f));
    out.mask = gbuf.mask;
    out.uv = gbuf.uv;
    out.albedo = s.albedo;
    out.normal = n;
    return out;
}

PbrOutputs BuildPbrForward(const PbrGeometryLeaves& geom, const PbrMaterialLeaves& mat,
                           const PbrFrameLeaves& frame, const PbrIblMaps& ibl,
                           const Variable& inv_uv, ImgSize screen, bool normal_mapping) {
    return BuildPbrShade(BuildPbrGBuffer(geom, screen), mat, frame, ibl, inv_uv, screen,
                         normal_mapping);
}

}  // namespace dressi_examples
