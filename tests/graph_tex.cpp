// graph_tex.cpp -- the texture fit written against the graph API
// (#include "dressi/dressi.h") and run by DressiAD: the deferred unlit
// rendering graph of examples/texture_optimization/run.cpp:112-145 with
// TextureBilinear on an RGBA texture, the RGB L2 image loss and the
// silhouette example's in-graph Adam (run.cpp:404-437), the cameras sent as
// clip / inverse-UV attribute images every iteration (the example's
// per-iteration sendImg of moving cameras).
//
//   graph_tex <in.bin> <out.bin> [warmup]
// in.bin:  u32 V, F, N, S, tex_w, tex_h, iters, n_sets, packing (0 RSP,
//          1 Naive); f32 lr; pos {V,3}, uv {V,2}, faces {F,3},
//          mvps {n_sets, N, 16}, gt_tex {T,4}, tex0 {T,4}
//          (iteration it uses camera set it % n_sets)
// out.bin: tex, m, v {T,4}, t, loss[iters] (sum of the loss image),
//          grad0 {T,4} (first iteration)
// stdout:  "graph_tex: plan=<name> stages=<n> substages=<n> funcs=<n>"
// With `warmup` (timing, the example's loop: each step sends its cameras'
// images and runs execStep, nothing is read back): `warmup` untimed steps,
// then `iters` timed ones, "graph_tex: ms_per_step=<ms>"; out.bin as above
// with the losses zero.
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "dressi/dressi.h"
#include "dressi/mesh_utils.h"
#include "dressi_examples/geometry_utils.h"

using namespace dressi;

namespace {

CpuImage ClipImage(const CpuImage& pos, const float* m) {
    dressi_examples::Mat4 r{};
    std::copy(m, m + 16, r.begin());
    return dressi_examples::TransformToClip(pos, r);
}

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

}  // namespace

int main(int argc, char** argv) {
    try {
        if (argc != 3 && argc != 4) {
            throw DressiError("usage: graph_tex <in.bin> <out.bin> [warmup]");
        }
        const int warmup = argc == 4 ? std::atoi(argv[3]) : 0;
        FILE* fi = fopen(argv[1], "rb");
        if (!fi) {
            throw DressiError("cannot open input");
        }
        uint32_t hdr[9];
        get(fi, hdr, 9);
        const uint32_t n_verts = hdr[0], n_faces = hdr[1], n_views = hdr[2], s = hdr[3];
        const uint32_t tw = hdr[4], th = hdr[5], iters = hdr[6], n_sets = hdr[7];
        const bool naive = hdr[8] != 0;
        float lr = 0.f;
        get(fi, &lr, 1);
        const CpuImage pos_img = Read(fi, n_verts, 1, 3);
        const CpuImage uv_img = Read(fi, n_verts, 1, 2);
        const CpuImage faces_img = Read(fi, n_faces, 1, 3);
        std::vector<float> mvps(size_t(n_sets) * n_views * 16);
        get(fi, mvps.data(), mvps.size());
        const CpuImage gt_img = Read(fi, tw, th, 4);
        const CpuImage tex0_img = Read(fi, tw, th, 4);
        fclose(fi);

        const ImgSize screen = {s, s};
        const ImgSize tex_size = {tw, th};
        Variable vtx_uv(VEC2, {n_verts, 1});
        Variable faces(IVEC3, {n_faces, 1});
        Variable uv_clip(VEC4, {n_verts, 1});
        Variable ones(FLOAT, {n_verts, 1});
        Variable gt_tex(VEC4, tex_size);
        Variable tex(VEC4, tex_size);
        Variable adam_m(VEC4, tex_size);
        Variable adam_v(VEC4, tex_size);
        Variable adam_t(FLOAT, {1, 1});
        std::vector<Variable> clips, attrs;
        Variables view_losses;
        const float c = 1.f / float(s * s);
        for (uint32_t v = 0; v < n_views; v++) {
            clips.emplace_back(VEC4, ImgSize{n_verts, 1});
            attrs.emplace_back(VEC4, ImgSize{n_verts, 1});
            Variable g_uv = F::Rasterize(clips[v], vtx_uv, faces, screen);
            Variable g_mask = F::Rasterize(clips[v], ones, faces, screen);
            Variable inv_uv = F::Rasterize(uv_clip, attrs[v], faces, tex_size);
            Variable target = g_mask * F::TextureBilinear(gt_tex, g_uv, inv_uv);
            Variable pred = g_mask * F::TextureBilinear(tex, g_uv, inv_uv);
            Variable diff = F::StopGradient(target) - pred;
            view_losses.push_back(diff * diff * F::Vec4(c, c, c, 0.f));
        }
        Variable loss = F::SumPixelWise(view_losses);
        Variable tex_mut = tex;
        tex_mut.setRequiresGradRecursively();

        DressiAD ad;
        ad.setPackingMode(naive ? DressiAD::PackingMode::Naive : DressiAD::PackingMode::RSP);
        ad.setLossVar(loss);
        bool state_registered = false;
        ad.setOptimizer([&](Variables xs, Variables gxs) {
            DRESSI_CHECK(xs.size() == 1 && xs[0] == tex, "expected the texture as the only leaf");
            const Variable g = gxs[0];
            const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
            Variable t_new = adam_t + 1.f;
            Variable m_new = adam_m * b1 + g * (1.f - b1);
            Variable v_new = adam_v * b2 + g * g * (1.f - b2);
            Variable bc1 = 1.f - F::Pow(F::Float(b1), t_new);
            Variable bc2 = 1.f - F::Pow(F::Float(b2), t_new);
            Variable step = (m_new / bc1) / (F::Sqrt(v_new / bc2) + eps) * lr;
            if (!state_registered) {
                ad.addUpdate(adam_m, m_new);
                ad.addUpdate(adam_v, v_new);
                ad.addUpdate(adam_t, t_new);
                state_registered = true;
            }
            return Variables{tex - step};
        });
        ad.setGradOutputsEnabled(true);

        // one-time uploads (run.cpp:146-158)
        ad.sendImg(vtx_uv, uv_img);
        ad.sendImg(faces, faces_img);
        ad.sendImg(uv_clip, UvAsClip(uv_img));
        ad.sendImg(ones, CpuImage(n_verts, 1, 1, 1.f));
        ad.sendImg(gt_tex, gt_img);
        ad.sendImg(tex, tex0_img);
        ad.sendImg(adam_m, CpuImage(tw, th, 4, 0.f));
        ad.sendImg(adam_v, CpuImage(tw, th, 4, 0.f));
        ad.sendImg(adam_t, CpuImage(1, 1, 1, 0.f));

        // iterations: each step sends its camera set's clip and inverse-UV
        // attribute images with the step
        std::vector<float> losses(iters);
        CpuImage grad0;
        std::vector<CpuImage> clip_imgs(n_views), attr_imgs(n_views);
        auto sends_of = [&](uint32_t it) {
            const float* set = mvps.data() + size_t(it % n_sets) * n_views * 16;
            std::vector<std::pair<Variable, CpuImageView>> sends;
            for (uint32_t v = 0; v < n_views; v++) {
                clip_imgs[v] = ClipImage(pos_img, set + 16 * v);
                attr_imgs[v] = ScreenAttr(clip_imgs[v], screen);
                sends.emplace_back(clips[v], CpuImageView(clip_imgs[v]));
                sends.emplace_back(attrs[v], CpuImageView(attr_imgs[v]));
            }
            return sends;
        };
        if (warmup > 0) {
            for (int it = 0; it < warmup; it++) {
                ad.execStepWithSends(sends_of((uint32_t)it));
            }
            const auto t0 = std::chrono::steady_clock::now();
            for (uint32_t it = 0; it < iters; it++) {
                ad.execStepWithSends(sends_of((uint32_t)warmup + it));
            }
            const auto t1 = std::chrono::steady_clock::now();
            printf("graph_tex: ms_per_step=%.5f\n",
                   std::chrono::duration<double, std::milli>(t1 - t0).count() / iters);
        }
        for (uint32_t it = 0; it < iters && warmup <= 0; it++) {
            const auto sends = sends_of(it);
            const CpuImage li = ad.execStepWithSendsAndRecvImgsStacked(sends, {loss});
            double acc = 0.0;
            for (float x : li.data) {
                acc += x;
            }
            losses[it] = float(acc);
            if (it == 0) {
                grad0 = ad.recvImg(ad.inputGrads().at(0).second);
            }
        }
        if (warmup > 0) {
            grad0 = CpuImage(tw, th, 4, 0.f);
        }
        FILE* fo = fopen(argv[2], "wb");
        if (!fo) {
            throw DressiError("cannot open output");
        }
        for (const Variable& v : {tex, adam_m, adam_v, adam_t}) {
            const CpuImage d = ad.recvImg(v);
            fwrite(d.data.data(), sizeof(float), d.data.size(), fo);
        }
        fwrite(losses.data(), sizeof(float), losses.size(), fo);
        fwrite(grad0.data.data(), sizeof(float), grad0.data.size(), fo);
        fclose(fo);
        printf("graph_tex: plan=%s stages=%zu substages=%zu funcs=%zu\n",
               ad.getPlanName().c_str(), ad.getStageCount(), ad.getSubStageCount(),
               ad.getFuncCount());
    } catch (const std::exception& e) {
        fprintf(stderr, "graph_tex: %s\n", e.what());
        return 1;
    }
    return 0;
}
