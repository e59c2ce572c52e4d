// graph_pbr.cpp -- the PBR material + environment fit written against the
// graph API (#include "dressi/dressi.h") with the examples' PBR graph
// builders (dressi_examples/pbr_graph.h) and run by DressiAD: per view the
// G-buffer and the shading with normal mapping off (AO 1, emissive 0, the
// normal map flat), the target rendered by the same graph from the
// ground-truth maps, the L1 image loss Mean(|StopGradient(target) - pred|)
// summed over views, and in-graph Adam on albedo, mr and env with one shared
// step counter, albedo / mr clamped to [0,1] and the env to >= 0
// (examples/pbr_material_optimization/run.cpp:189-288,
// examples/pbr_envmap_optimization/run.cpp:312-317).
//
//   graph_pbr <in.bin> <out.bin>
// in.bin:  u32 V, F, N, S, tex_w, tex_h, env_w, env_h, levels, iters,
//          packing (0 RSP, 1 Naive); f32 lr; pos {V,3}, normal {V,3},
//          uv {V,2}, faces {F,3}, mvps {N,16}, frames {N,12} (cam_pos,
//          cam_fwd, cam_right, cam_up), light {6} (pos, colour),
//          gt_albedo, gt_mr {T,3}, gt_env {E,3}, albedo0, mr0 {T,3}, env0 {E,3}
// out.bin: albedo, mr {T,3}, env {E,3}, t, loss[iters], g_albedo0,
//          g_mr0 {T,3}, g_env0 {E,3} (gradients of the first iteration)
// stdout:  "graph_pbr: plan=<name> stages=<n> substages=<n> funcs=<n>"
#include <cstdio>
#include <vector>

#include "dressi/dressi.h"
#include "dressi/ibl.h"
#include "dressi/mesh_utils.h"
#include "dressi_examples/pbr_graph.h"

using namespace dressi;
using namespace dressi_examples;

namespace {

template <typename T>
void get(FILE* f, T* p, size_t n) {
    if (fread(p, sizeof(T), n, f) != n) {
        throw DressiError("short input file");
    }
}

CpuImage Read(FILE* f, uint32_t w, uint32_t h, uint32_t c) {
    CpuImage img(w, h, c);
    get(f, img.data.data(), img.data.size());
    return img;
}

// column-vector clip transform, m column-major, terms summed k = 0..3
CpuImage ClipOf(const CpuImage& pos, const float* m) {
    const uint32_t n = pos.width;
    CpuImage clip(n, 1, 4);
    for (uint32_t i = 0; i < n; i++) {
        const float p[4] = {pos.at(i, 0, 0), pos.at(i, 0, 1), pos.at(i, 0, 2), 1.f};
        for (uint32_t row = 0; row < 4; row++) {
            float acc = 0.f;
            for (int k = 0; k < 4; k++) {
                acc += m[k * 4 + row] * p[k];
            }
            clip.at(i, 0, row) = acc;
        }
    }
    return clip;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        if (argc != 3) {
            throw DressiError("usage: graph_pbr <in.bin> <out.bin>");
        }
        FILE* fi = fopen(argv[1], "rb");
        if (!fi) {
            throw DressiError("cannot open input");
        }
        uint32_t hdr[11];
        get(fi, hdr, 11);
        const uint32_t n_verts = hdr[0], n_faces = hdr[1], n_views = hdr[2], s = hdr[3];
        const uint32_t tw = hdr[4], th = hdr[5], ew = hdr[6], eh = hdr[7], levels = hdr[8];
        const uint32_t iters = hdr[9];
        const bool naive = hdr[10] != 0;
        float lr = 0.f;
        get(fi, &lr, 1);
        const CpuImage pos_img = Read(fi, n_verts, 1, 3);
        const CpuImage normal_img = Read(fi, n_verts, 1, 3);
        const CpuImage uv_img = Read(fi, n_verts, 1, 2);
        const CpuImage faces_img = Read(fi, n_faces, 1, 3);
        std::vector<float> mvps(size_t(n_views) * 16), frames(size_t(n_views) * 12);
        get(fi, mvps.data(), mvps.size());
        get(fi, frames.data(), frames.size());
        float light[6];
        get(fi, light, 6);
        const CpuImage gt_albedo_img = Read(fi, tw, th, 3);
        const CpuImage gt_mr_img = Read(fi, tw, th, 3);
        const CpuImage gt_env_img = Read(fi, ew, eh, 3);
        const CpuImage albedo0 = Read(fi, tw, th, 3);
        const CpuImage mr0 = Read(fi, tw, th, 3);
        const CpuImage env0 = Read(fi, ew, eh, 3);
        fclose(fi);

        const ImgSize screen = {s, s}, tex_size = {tw, th}, env_size = {ew, eh};
        PbrGeometryLeaves geom;
        geom.uvh = Variable(VEC4, {n_verts, 1});
        geom.normal = Variable(VEC3, {n_verts, 1});
        geom.tangent = Variable(VEC3, {n_verts, 1});
        geom.wpos = Variable(VEC3, {n_verts, 1});
        geom.faces = Variable(IVEC3, {n_faces, 1});
        PbrMaterialLeaves gt_mat;
        gt_mat.albedo = Variable(VEC3, tex_size);
        gt_mat.mr = Variable(VEC3, tex_size);
        gt_mat.normal_map = Variable(VEC3, tex_size);
        gt_mat.ao = Variable(VEC3, tex_size);
        gt_mat.emissive = Variable(VEC3, tex_size);
        Variable albedo(VEC3, tex_size), mr(VEC3, tex_size);
        PbrMaterialLeaves mat = gt_mat;
        mat.albedo = albedo;
        mat.mr = mr;
        Variable env_gt(VEC3, env_size), env(VEC3, env_size);
        // the environment is optimised: the differentiable GGX prefilter
        const auto maps_of = [&](const Variable& e) {
            PbrIblMaps m;
            m.env = e;
            m.irr = BuildIrradianceSample(e);
            m.pref = BuildPrefEnvironmentSampleConv(e, levels);
            m.lut = BuildBrdfIntegrationMap();
            return m;
        };
        const PbrIblMaps ibl_gt = maps_of(env_gt), ibl = maps_of(env);
        Variable uv_clip(VEC4, {n_verts, 1});
        Variable light_pos(VEC3, {1, 1}), light_col(VEC3, {1, 1});
        std::vector<Variable> clips, attrs;
        std::vector<PbrFrameLeaves> frs(n_views);
        Variables view_losses;
        for (uint32_t v = 0; v < n_views; v++) {
            clips.emplace_back(VEC4, ImgSize{n_verts, 1});
            attrs.emplace_back(VEC4, ImgSize{n_verts, 1});
            frs[v].cam_pos = Variable(VEC3, {1, 1});
            frs[v].cam_fwd = Variable(VEC3, {1, 1});
            frs[v].cam_right = Variable(VEC3, {1, 1});
            frs[v].cam_up = Variable(VEC3, {1, 1});
            frs[v].light_pos = light_pos;
            frs[v].light_col = light_col;
            PbrGeometryLeaves vg = geom;
            vg.clip = clips[v];
            const PbrGBuffer gb = BuildPbrGBuffer(vg, screen);
            const Variable inv_uv = F::Rasterize(uv_clip, attrs[v], geom.faces, tex_size);
            const PbrOutputs target = BuildPbrShade(gb, gt_mat, frs[v], ibl_gt, inv_uv, screen,
                                                    false);
            const PbrOutputs pred = BuildPbrShade(gb, mat, frs[v], ibl, inv_uv, screen, false);
            view_losses.push_back(F::Mean(F::Abs(F::StopGradient(target.mapped) - pred.mapped)));
        }
        Variable loss = F::SumPixelWise(view_losses);
        for (Variable leaf : {albedo, mr, env}) {
            leaf.setRequiresGradRecursively();
        }

        DressiAD ad;
        ad.setPackingMode(naive ? DressiAD::PackingMode::Naive : DressiAD::PackingMode::RSP);
        ad.setLossVar(loss);
        Variable adam_t(FLOAT, {1, 1});
        std::vector<Variable> adam_m, adam_v;  // in the order of albedo, mr, env
        for (const ImgSize& sz : {tex_size, tex_size, env_size}) {
            adam_m.emplace_back(VEC3, sz);
            adam_v.emplace_back(VEC3, sz);
        }
        bool state_registered = false;
        ad.setOptimizer([&](Variables xs, Variables gxs) {
            const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
            Variable t_new = adam_t + 1.f;
            Variable bc1 = 1.f - F::Pow(F::Float(b1), t_new);
            Variable bc2 = 1.f - F::Pow(F::Float(b2), t_new);
            Variables out;
            for (size_t i = 0; i < xs.size(); i++) {
                const size_t k = xs[i] == albedo ? 0 : xs[i] == mr ? 1 : 2;
                DRESSI_CHECK(k < 2 || xs[i] == env, "unexpected leaf");
                const Variable& g = gxs[i];
                Variable m_new = adam_m[k] * b1 + g * (1.f - b1);
                Variable v_new = adam_v[k] * b2 + g * g * (1.f - b2);
                Variable step = (m_new / bc1) / (F::Sqrt(v_new / bc2) + eps) * lr;
                out.push_back(k < 2 ? F::Clamp(xs[i] - step, F::Float(0.f), F::Float(1.f))
                                    : F::Max(xs[i] - step, F::Float(0.f)));
                if (!state_registered) {
                    ad.addUpdate(adam_m[k], m_new);
                    ad.addUpdate(adam_v[k], v_new);
                }
            }
            if (!state_registered) {
                ad.addUpdate(adam_t, t_new);
                state_registered = true;
            }
            return out;
        });
        ad.setGradOutputsEnabled(true);

        // uploads: everything but the parameters and their state is static
        CpuImage uvh_img(n_verts, 1, 4);
        for (uint32_t i = 0; i < n_verts; i++) {
            uvh_img.at(i, 0, 0) = uv_img.at(i, 0, 0);
            uvh_img.at(i, 0, 1) = uv_img.at(i, 0, 1);
            uvh_img.at(i, 0, 2) = 1.f;
            uvh_img.at(i, 0, 3) = 1.f;
        }
        ad.sendImg(geom.uvh, uvh_img);
        ad.sendImg(geom.normal, normal_img);
        ad.sendImg(geom.tangent, CpuImage(n_verts, 1, 3, 0.f));
        ad.sendImg(geom.wpos, pos_img);
        ad.sendImg(geom.faces, faces_img);
        ad.sendImg(gt_mat.albedo, gt_albedo_img);
        ad.sendImg(gt_mat.mr, gt_mr_img);
        ad.sendImg(gt_mat.normal_map, CpuImage(tw, th, 3, 0.5f));
        ad.sendImg(gt_mat.ao, CpuImage(tw, th, 3, 1.f));
        ad.sendImg(gt_mat.emissive, CpuImage(tw, th, 3, 0.f));
        ad.sendImg(env_gt, gt_env_img);
        ad.sendImg(uv_clip, UvAsClip(uv_img));
        CpuImage lp(1, 1, 3), lc(1, 1, 3);
        for (uint32_t c = 0; c < 3; c++) {
            lp.data[c] = light[c];
            lc.data[c] = light[3 + c];
        }
        ad.sendImg(light_pos, lp);
        ad.sendImg(light_col, lc);
        for (uint32_t v = 0; v < n_views; v++) {
            const CpuImage clip = ClipOf(pos_img, mvps.data() + 16 * v);
            ad.sendImg(clips[v], clip);
            ad.sendImg(attrs[v], ScreenAttr(clip, screen));
            const float* fr = frames.data() + 12 * v;
            const Variable* dst[4] = {&frs[v].cam_pos, &frs[v].cam_fwd, &frs[v].cam_right,
                                      &frs[v].cam_up};
            for (int j = 0; j < 4; j++) {
                CpuImage c3(1, 1, 3);
                for (int c = 0; c < 3; c++) {
                    c3.data[c] = fr[3 * j + c];
                }
                ad.sendImg(*dst[j], c3);
            }
        }
        ad.sendImg(albedo, albedo0);
        ad.sendImg(mr, mr0);
        ad.sendImg(env, env0);
        for (size_t k = 0; k < 3; k++) {
            const ImgSize sz = k < 2 ? tex_size : env_size;
            ad.sendImg(adam_m[k], CpuImage(sz.w, sz.h, 3, 0.f));
            ad.sendImg(adam_v[k], CpuImage(sz.w, sz.h, 3, 0.f));
        }
        ad.sendImg(adam_t, CpuImage(1, 1, 1, 0.f));

        std::vector<float> losses(iters);
        CpuImage g0[3];
        for (uint32_t it = 0; it < iters; it++) {
            const CpuImage li = ad.execStepWithSendsAndRecvImgsStacked({}, {loss});
            losses[it] = li.data.at(0);
            if (it == 0) {
                for (const auto& [x, gx] : ad.inputGrads()) {
                    const size_t k = x == albedo ? 0 : x == mr ? 1 : 2;
                    g0[k] = ad.recvImg(gx);
                }
            }
        }
        FILE* fo = fopen(argv[2], "wb");
        if (!fo) {
            throw DressiError("cannot open output");
        }
        for (const Variable& v : {albedo, mr, env, adam_t}) {
            const CpuImage d = ad.recvImg(v);
            fwrite(d.data.data(), sizeof(float), d.data.size(), fo);
        }
        fwrite(losses.data(), sizeof(float), losses.size(), fo);
        for (const CpuImage& g : g0) {
            DRESSI_CHECK(!g.data.empty(), "missing a first-iteration gradient");
            fwrite(g.data.data(), sizeof(float), g.data.size(), fo);
        }
        fclose(fo);
        printf("graph_pbr: plan=%s stages=%zu substages=%zu funcs=%zu\n",
               ad.getPlanName().c_str(), ad.getStageCount(), ad.getSubStageCount(),
               ad.getFuncCount());
    } catch (const std::exception& e) {
        fprintf(stderr, "graph_pbr: %s\n", e.what());
        return 1;
    }
    return 0;
}
