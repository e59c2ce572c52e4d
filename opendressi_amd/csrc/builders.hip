// builders.hip -- host-side builders of the graph API: static-topology
// images (include/dressi/mesh_utils.h; the reference's
// src/core/mesh_utils.cpp:10-203) and the split-sum IBL helpers composed of
// F:: ops (include/dressi/ibl.h; src/core/ibl.cpp:14-93). Host code only.
//
// The images are data formats the gather kernels read, so their layouts
// follow the reference exactly: a {V, max_degree} table stores entry d of
// vertex v at row d, column v; lists are in ascending face / vertex order;
// -1 pads; the maximum degree is at least 1.
#include <algorithm>
#include <cmath>
#include <tuple>

#include "dressi/f.h"
#include "dressi/ibl.h"
#include "dressi/mesh_utils.h"

namespace dressi {

namespace {

uint32_t corner(const CpuImage& faces, uint32_t f, uint32_t k) {
    return (uint32_t)faces.at(f, 0, k);
}

void check_faces(const CpuImage& faces, uint32_t n_verts) {
    DRESSI_CHECK(faces.channels == 3 && faces.height == 1, "faces must be a {F,1} x 3 image");
    for (float v : faces.data) {
        DRESSI_CHECK(v >= 0.f && (uint32_t)v < n_verts, "face vertex id out of range");
    }
}

// per-vertex lists -> {V, max(1, longest)} table, -1 padded
CpuImage lists_to_table(const std::vector<std::vector<uint32_t>>& lists) {
    size_t deg = 1;
    for (const auto& l : lists) {
        deg = std::max(deg, l.size());
    }
    const uint32_t n = (uint32_t)lists.size();
    CpuImage t(n, (uint32_t)deg, 1, -1.f);
    for (uint32_t v = 0; v < n; v++) {
        for (size_t d = 0; d < lists[v].size(); d++) {
            t.at(v, (uint32_t)d, 0) = (float)lists[v][d];
        }
    }
    return t;
}

}  // namespace

std::vector<std::vector<uint32_t>> BuildVertexAdjacency(const CpuImage& faces, uint32_t n_verts) {
    check_faces(faces, n_verts);
    std::vector<std::vector<uint32_t>> adj(n_verts);
    for (uint32_t f = 0; f < faces.width; f++) {
        for (uint32_t k = 0; k < 3; k++) {
            const uint32_t a = corner(faces, f, k);
            adj[a].push_back(corner(faces, f, (k + 1) % 3));
            adj[a].push_back(corner(faces, f, (k + 2) % 3));
        }
    }
    for (auto& l : adj) {
        std::sort(l.begin(), l.end());
        l.erase(std::unique(l.begin(), l.end()), l.end());
    }
    return adj;
}

std::vector<std::array<uint32_t, 2>> BuildFaceAdjacency(const CpuImage& faces) {
    // (edge min, edge max, face) sorted: faces grouped per edge, edges in
    // ascending (min, max) order, faces ascending within an edge
    std::vector<std::tuple<uint32_t, uint32_t, uint32_t>> edges;
    edges.reserve((size_t)faces.width * 3);
    for (uint32_t f = 0; f < faces.width; f++) {
        for (uint32_t k = 0; k < 3; k++) {
            const uint32_t a = corner(faces, f, k), b = corner(faces, f, (k + 1) % 3);
            edges.emplace_back(std::min(a, b), std::max(a, b), f);
        }
    }
    std::sort(edges.begin(), edges.end());
    std::vector<std::array<uint32_t, 2>> pairs;
    for (size_t i = 0; i < edges.size();) {
        size_t j = i;
        while (j < edges.size() && std::get<0>(edges[j]) == std::get<0>(edges[i]) &&
               std::get<1>(edges[j]) == std::get<1>(edges[i])) {
            j++;
        }
        for (size_t p = i; p < j; p++) {
            for (size_t q = p + 1; q < j; q++) {
                pairs.push_back({std::get<2>(edges[p]), std::get<2>(edges[q])});
            }
        }
        i = j;
    }
    return pairs;
}

CpuImage VertexFacesTex(const CpuImage& faces, uint32_t n_verts) {
    check_faces(faces, n_verts);
    std::vector<std::vector<uint32_t>> inc(n_verts);
    for (uint32_t f = 0; f < faces.width; f++) {
        for (uint32_t k = 0; k < 3; k++) {
            inc[corner(faces, f, k)].push_back(f);
        }
    }
    return lists_to_table(inc);
}

CpuImage VertexNeighborsTex(const CpuImage& faces, uint32_t n_verts) {
    return lists_to_table(BuildVertexAdjacency(faces, n_verts));
}

CpuImage FaceNeighborsTex(const CpuImage& faces) {
    CpuImage t(faces.width, 1, 3, -1.f);
    std::vector<uint32_t> used(faces.width, 0);
    for (const auto& pr : BuildFaceAdjacency(faces)) {
        for (int e = 0; e < 2; e++) {
            const uint32_t f = pr[e], other = pr[1 - e];
            if (used[f] < 3) {
                t.at(f, 0, used[f]++) = (float)other;
            }
        }
    }
    return t;
}

SoftGeometry BuildSoftGeometry(const CpuImage& hard_clip, const CpuImage& faces, ImgSize screen,
                               float radius_px) {
    DRESSI_CHECK(hard_clip.channels == 4, "BuildSoftGeometry: clip positions must be VEC4");
    check_faces(faces, hard_clip.width);
    const uint32_t nf = faces.width;
    const float sw = (float)screen.w, sh = (float)screen.h;
    SoftGeometry g;
    g.clip = CpuImage(nf * 3, 1, 4);
    g.face_id = CpuImage(nf * 3, 1, 1);
    g.faces = CpuImage(nf, 1, 3);
    for (uint32_t f = 0; f < nf; f++) {
        float c[3][4], px[3], py[3];
        bool front = true;
        for (uint32_t k = 0; k < 3; k++) {
            const uint32_t v = corner(faces, f, k);
            for (uint32_t q = 0; q < 4; q++) {
                c[k][q] = hard_clip.at(v, 0, q);
            }
            if (c[k][3] <= 1e-6f) {
                front = false;  // behind the camera: passed through as is
            } else {
                px[k] = (c[k][0] / c[k][3] * 0.5f + 0.5f) * sw;
                py[k] = (c[k][1] / c[k][3] * 0.5f + 0.5f) * sh;
            }
        }
        if (front) {
            // grow about the centroid so that every edge moves out by at
            // least radius_px: scale 1 + r / (closest edge distance), <= 8
            const float mx = (px[0] + px[1] + px[2]) / 3.f;
            const float my = (py[0] + py[1] + py[2]) / 3.f;
            float closest = 1e30f;
            for (uint32_t k = 0; k < 3; k++) {
                const uint32_t n = (k + 1) % 3;
                const float dx = px[n] - px[k], dy = py[n] - py[k];
                const float len = std::sqrt(dx * dx + dy * dy);
                if (len < 1e-6f) {
                    continue;
                }
                closest = std::min(closest, std::abs(dx * (my - py[k]) - dy * (mx - px[k])) / len);
            }
            const float s = closest < 1e29f
                                    ? std::min(1.f + radius_px / std::max(closest, 1e-3f), 8.f)
                                    : 1.f;
            for (uint32_t k = 0; k < 3; k++) {
                const float qx = mx + (px[k] - mx) * s;
                const float qy = my + (py[k] - my) * s;
                c[k][0] = (qx / sw * 2.f - 1.f) * c[k][3];
                c[k][1] = (qy / sh * 2.f - 1.f) * c[k][3];
            }
        }
        for (uint32_t k = 0; k < 3; k++) {
            const uint32_t v = f * 3 + k;
            for (uint32_t q = 0; q < 4; q++) {
                g.clip.at(v, 0, q) = c[k][q];
            }
            g.face_id.at(v, 0, 0) = (float)f;
            g.faces.at(f, 0, k) = (float)v;
        }
    }
    return g;
}

CpuImage UvAsClip(const CpuImage& uv) {
    DRESSI_CHECK(uv.channels == 2, "UvAsClip: uv must be VEC2");
    CpuImage c(uv.width, 1, 4);
    for (uint32_t i = 0; i < uv.width; i++) {
        c.at(i, 0, 0) = uv.at(i, 0, 0) * 2.f - 1.f;
        c.at(i, 0, 1) = uv.at(i, 0, 1) * 2.f - 1.f;
        c.at(i, 0, 2) = 0.5f;
        c.at(i, 0, 3) = 1.f;
    }
    return c;
}

CpuImage ScreenAttr(const CpuImage& clip, ImgSize screen) {
    DRESSI_CHECK(clip.channels == 4, "ScreenAttr: clip positions must be VEC4");
    CpuImage a(clip.width, 1, 4);
    for (uint32_t i = 0; i < clip.width; i++) {
        const float w = clip.at(i, 0, 3);
        a.at(i, 0, 0) = (clip.at(i, 0, 0) / w * 0.5f + 0.5f) * (float)screen.w;
        a.at(i, 0, 1) = (clip.at(i, 0, 1) / w * 0.5f + 0.5f) * (float)screen.h;
        a.at(i, 0, 2) = 1.f;
        a.at(i, 0, 3) = 0.f;
    }
    return a;
}

// ---- split-sum IBL ---------------------------------------------------------------

namespace {

// halve (2x2 mean) until the map fits max_w x max_h
Variable pool_to_fit(Variable env, uint32_t max_w, uint32_t max_h) {
    while (env.getImgSize().w > max_w || env.getImgSize().h > max_h) {
        env = F::AvgPool2x2(env);
    }
    return env;
}

ImgSize halved(ImgSize s) { return {s.w > 1 ? s.w / 2 : 1, s.h > 1 ? s.h / 2 : 1}; }

}  // namespace

Variable BuildIrradianceSample(const Variable& env_img, ImgSize out_size) {
    return F::IrradianceConv(pool_to_fit(env_img, 64, 32), out_size);
}

std::vector<Variable> BuildPrefEnvironmentSample(const Variable& env_img, uint32_t levels,
                                                 ImgSize top, uint32_t n_samples) {
    DRESSI_CHECK(levels >= 2, "BuildPrefEnvironmentSample: at least 2 levels");
    // point taps: a source pooled to twice the top level is enough
    const Variable src = pool_to_fit(env_img, top.w * 2, top.h * 2);
    std::vector<Variable> out;
    ImgSize s = top;
    for (uint32_t i = 0; i < levels; i++) {
        out.push_back(F::PrefilterEnv(src, s, (float)i / (float)(levels - 1), n_samples));
        s = halved(s);
    }
    return out;
}

std::vector<Variable> BuildPrefEnvironmentSampleConv(const Variable& env_img, uint32_t levels,
                                                     ImgSize top) {
    DRESSI_CHECK(levels >= 2, "BuildPrefEnvironmentSampleConv: at least 2 levels");
    // dense taps forward and transposed: the source is pooled to the top
    // level, and no level is larger than the source
    const Variable src = pool_to_fit(env_img, top.w, top.h);
    const ImgSize ss = src.getImgSize();
    std::vector<Variable> out;
    ImgSize s = {std::min(top.w, ss.w), std::min(top.h, ss.h)};
    for (uint32_t i = 0; i < levels; i++) {
        out.push_back(F::PrefilterConv(src, s, (float)i / (float)(levels - 1)));
        s = halved(s);
    }
    return out;
}

Variable BuildBrdfIntegrationMap(ImgSize size, uint32_t n_samples) {
    return F::BrdfIntegrationLut(size, n_samples);
}

Variable SampleIrradiance(const Variable& irrad, const Variable& normal) {
    return F::EquirectSample(irrad, normal);
}

Variable SamplePrefEnvironment(const std::vector<Variable>& levels, const Variable& refl_dir,
                               const Variable& roughness) {
    DRESSI_CHECK(levels.size() >= 2, "SamplePrefEnvironment: at least 2 levels");
    const Variable lod = roughness * (float)(levels.size() - 1);
    Variables terms;
    for (size_t i = 0; i < levels.size(); i++) {
        // tent weight of level i at the fractional level `lod`
        const Variable w = F::Clamp(1.f - F::Abs(lod - (float)i), F::Float(0.f), F::Float(1.f));
        terms.push_back(F::EquirectSample(levels[i], refl_dir) * w);
    }
    return F::SumPixelWise(terms);
}

Variable SampleBrdfLut(const Variable& lut, const Variable& n_dot_v, const Variable& roughness) {
    // the LUT is a constant: its inverse-UV table is never filled
    return F::TextureBilinear(lut, F::Vec2(n_dot_v, roughness), Variable(VEC4, lut.getImgSize()));
}

}  // namespace dressi
