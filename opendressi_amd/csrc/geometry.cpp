// geometry.cpp -- the examples' mesh and optimisation helpers
// (include/dressi_examples/geometry_utils.h; the reference's
// examples/common/geometry_utils.cpp:24-421). Host code. The sphere
// generators are the library's C-ABI ones; the float helpers evaluate
// their expressions in the reference's operation order, so that results
// are bit-identical to it under IEEE single precision without contraction.
#include <cmath>
#include <fstream>

#include "dressi_examples/geometry_utils.h"
#include "dressi_hip.h"

namespace dressi_examples {

using dressi::CpuImage;

namespace {

struct Vec3 {
    float x, y, z;
};

Vec3 sub(const Vec3& a, const Vec3& b) { return {a.x - b.x, a.y - b.y, a.z - b.z}; }
Vec3 cross(const Vec3& a, const Vec3& b) {
    return {a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x};
}
float dot(const Vec3& a, const Vec3& b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
Vec3 row3(const CpuImage& img, uint32_t i) {
    return {img.at(i, 0, 0), img.at(i, 0, 1), img.at(i, 0, 2)};
}

void check_rc(int rc, const char* what) {
    if (rc != DRESSI_OK) {
        throw std::runtime_error(std::string(what) + ": " + dressi_last_error());
    }
}

Mesh from_arrays(uint32_t nv, uint32_t nf, std::vector<float> pos, std::vector<float> uv,
                 std::vector<float> faces) {
    Mesh m;
    m.pos = CpuImage(nv, 1, 3);
    m.pos.data = std::move(pos);
    m.uv = CpuImage(nv, 1, 2, 0.f);
    if (!uv.empty()) {
        m.uv.data = std::move(uv);
    }
    m.faces = CpuImage(nf, 1, 3);
    m.faces.data = std::move(faces);
    return m;
}

// the face's three vertex ids and its edge cross product (p1 - p0) x (p2 - p0)
Vec3 face_cross(const CpuImage& pos, const CpuImage& faces, uint32_t f, uint32_t id[3]) {
    for (uint32_t k = 0; k < 3; k++) {
        id[k] = (uint32_t)faces.at(f, 0, k);
    }
    const Vec3 p0 = row3(pos, id[0]);
    return cross(sub(row3(pos, id[1]), p0), sub(row3(pos, id[2]), p0));
}

void write_v(std::ofstream& o, const Mesh& mesh) {
    for (uint32_t i = 0; i < mesh.numVertices(); i++) {
        o << "v " << mesh.pos.at(i, 0, 0) << ' ' << mesh.pos.at(i, 0, 1) << ' '
          << mesh.pos.at(i, 0, 2) << '\n';
    }
}

}  // namespace

Mesh GenerateIcosphere(uint32_t level) {
    uint32_t nv = 0, nf = 0;
    check_rc(dressi_icosphere(level, &nv, &nf, nullptr, nullptr), "GenerateIcosphere");
    std::vector<float> pos((size_t)nv * 3), faces((size_t)nf * 3);
    check_rc(dressi_icosphere(level, &nv, &nf, pos.data(), faces.data()), "GenerateIcosphere");
    return from_arrays(nv, nf, std::move(pos), {}, std::move(faces));
}

Mesh GenerateUvSphere(uint32_t stacks, uint32_t slices) {
    uint32_t nv = 0, nf = 0;
    check_rc(dressi_uv_sphere(stacks, slices, &nv, &nf, nullptr, nullptr, nullptr),
             "GenerateUvSphere");
    std::vector<float> pos((size_t)nv * 3), uv((size_t)nv * 2), faces((size_t)nf * 3);
    check_rc(dressi_uv_sphere(stacks, slices, &nv, &nf, pos.data(), uv.data(), faces.data()),
             "GenerateUvSphere");
    return from_arrays(nv, nf, std::move(pos), std::move(uv), std::move(faces));
}

CpuImage TransferDeformationByDirection(const CpuImage& ctrl_rest_pos, const CpuImage& ctrl_faces,
                                        const CpuImage& ctrl_deformed_pos,
                                        const CpuImage& dst_pos) {
    CpuImage out(dst_pos.width, 1, 3);
    for (uint32_t d = 0; d < dst_pos.width; d++) {
        const Vec3 p = row3(dst_pos, d);
        const float len = std::sqrt(p.x * p.x + p.y * p.y + p.z * p.z);
        const Vec3 dir = {p.x / len, p.y / len, p.z / len};
        // Moeller-Trumbore from the origin along dir; the nearest hit with
        // t > 1e-6, barycentrics accepted within 1e-4 of the triangle
        uint32_t hit = 0;
        float best = 1e30f, hu = 0.f, hv = 0.f;
        for (uint32_t f = 0; f < ctrl_faces.width; f++) {
            uint32_t id[3];
            for (uint32_t k = 0; k < 3; k++) {
                id[k] = (uint32_t)ctrl_faces.at(f, 0, k);
            }
            const Vec3 a = row3(ctrl_rest_pos, id[0]);
            const Vec3 e1 = sub(row3(ctrl_rest_pos, id[1]), a);
            const Vec3 e2 = sub(row3(ctrl_rest_pos, id[2]), a);
            const Vec3 pv = cross(dir, e2);
            const float det = dot(e1, pv);
            if (std::abs(det) < 1e-20f) {
                continue;
            }
            const float inv = 1.f / det;
            const Vec3 to = {-a.x, -a.y, -a.z};
            const float u = dot(to, pv) * inv;
            if (u < -1e-4f || u > 1.f + 1e-4f) {
                continue;
            }
            const Vec3 qv = cross(to, e1);
            const float v = dot(dir, qv) * inv;
            if (v < -1e-4f || u + v > 1.f + 1e-4f) {
                continue;
            }
            const float t = dot(e2, qv) * inv;
            if (t > 1e-6f && t < best) {
                best = t;
                hit = f;
                hu = u;
                hv = v;
            }
        }
        const uint32_t ia = (uint32_t)ctrl_faces.at(hit, 0, 0);
        const uint32_t ib = (uint32_t)ctrl_faces.at(hit, 0, 1);
        const uint32_t ic = (uint32_t)ctrl_faces.at(hit, 0, 2);
        const float wa = 1.f - hu - hv;
        for (uint32_t c = 0; c < 3; c++) {
            out.at(d, 0, c) = wa * ctrl_deformed_pos.at(ia, 0, c) +
                              hu * ctrl_deformed_pos.at(ib, 0, c) +
                              hv * ctrl_deformed_pos.at(ic, 0, c);
        }
    }
    return out;
}

void SaveObjMesh(const std::string& path, const Mesh& mesh) {
    std::ofstream o(path);
    if (!o) {
        return;
    }
    write_v(o, mesh);
    for (uint32_t i = 0; i < mesh.numFaces(); i++) {
        o << "f " << (int)mesh.faces.at(i, 0, 0) + 1 << ' ' << (int)mesh.faces.at(i, 0, 1) + 1
          << ' ' << (int)mesh.faces.at(i, 0, 2) + 1 << '\n';
    }
}

void SaveTexturedObjMesh(const std::string& path, const Mesh& mesh,
                         const std::string& texture_filename) {
    std::ofstream o(path);
    if (!o) {
        return;
    }
    const size_t dot_at = path.find_last_of('.');
    const std::string mtl_path =
            (dot_at == std::string::npos ? path : path.substr(0, dot_at)) + ".mtl";
    const size_t slash = mtl_path.find_last_of("/\\");
    const std::string mtl_name = slash == std::string::npos ? mtl_path : mtl_path.substr(slash + 1);
    {
        std::ofstream mtl(mtl_path);
        if (mtl) {
            mtl << "newmtl material0\nKa 0 0 0\nKd 1 1 1\nd 1\nillum 1\nmap_Kd "
                << texture_filename << '\n';
        }
    }
    o << "mtllib " << mtl_name << "\nusemtl material0\n";
    write_v(o, mesh);
    for (uint32_t i = 0; i < mesh.numVertices(); i++) {
        o << "vt " << mesh.uv.at(i, 0, 0) << ' ' << 1.f - mesh.uv.at(i, 0, 1) << '\n';
    }
    for (uint32_t i = 0; i < mesh.numFaces(); i++) {
        o << 'f';
        for (uint32_t k = 0; k < 3; k++) {
            const int id = (int)mesh.faces.at(i, 0, k) + 1;
            o << ' ' << id << '/' << id;
        }
        o << '\n';
    }
}

CpuImage UniformLaplacianGrad(const CpuImage& pos, const std::vector<std::vector<uint32_t>>& adj,
                              float lambda) {
    CpuImage g(pos.width, 1, 3, 0.f);
    for (uint32_t v = 0; v < pos.width && v < adj.size(); v++) {
        if (adj[v].empty()) {
            continue;
        }
        float sum[3] = {0.f, 0.f, 0.f};
        for (uint32_t n : adj[v]) {
            for (uint32_t c = 0; c < 3; c++) {
                sum[c] += pos.at(n, 0, c);
            }
        }
        const float inv = 1.f / (float)adj[v].size();
        for (uint32_t c = 0; c < 3; c++) {
            g.at(v, 0, c) = lambda * (pos.at(v, 0, c) - sum[c] * inv);
        }
    }
    return g;
}

CpuImage NormalConsistencyGrad(const CpuImage& pos, const CpuImage& faces,
                               const std::vector<std::array<uint32_t, 2>>& face_adj,
                               float lambda) {
    CpuImage g(pos.width, 1, 3, 0.f);
    // dE / dc for c = e1 x e2 (e1 = p1 - p0, e2 = p2 - p0) moves to the
    // vertices as p1 += e2 x gc, p2 += gc x e1, p0 -= the sum of both
    auto scatter = [&](const uint32_t id[3], const Vec3& gc) {
        const Vec3 p0 = row3(pos, id[0]);
        const Vec3 e1 = sub(row3(pos, id[1]), p0);
        const Vec3 e2 = sub(row3(pos, id[2]), p0);
        const Vec3 g1 = cross(e2, gc);
        const Vec3 g2 = cross(gc, e1);
        const float d1[3] = {g1.x, g1.y, g1.z}, d2[3] = {g2.x, g2.y, g2.z};
        for (uint32_t c = 0; c < 3; c++) {
            g.at(id[1], 0, c) += d1[c];
        }
        for (uint32_t c = 0; c < 3; c++) {
            g.at(id[2], 0, c) += d2[c];
        }
        for (uint32_t c = 0; c < 3; c++) {
            g.at(id[0], 0, c) -= d1[c] + d2[c];
        }
    };
    for (const auto& pr : face_adj) {
        uint32_t ia[3], ib[3];
        const Vec3 ca = face_cross(pos, faces, pr[0], ia);
        const Vec3 cb = face_cross(pos, faces, pr[1], ib);
        const float la = std::sqrt(dot(ca, ca));
        const float lb = std::sqrt(dot(cb, cb));
        if (la < 1e-12f || lb < 1e-12f) {
            continue;
        }
        const Vec3 na = {ca.x / la, ca.y / la, ca.z / la};
        const Vec3 nb = {cb.x / lb, cb.y / lb, cb.z / lb};
        const float d = dot(na, nb);
        // E = lambda (1 - na . nb): dE/dca = -lambda (nb - d na) / |ca|
        const Vec3 ga = {-lambda * (nb.x - d * na.x) / la, -lambda * (nb.y - d * na.y) / la,
                         -lambda * (nb.z - d * na.z) / la};
        const Vec3 gb = {-lambda * (na.x - d * nb.x) / lb, -lambda * (na.y - d * nb.y) / lb,
                         -lambda * (na.z - d * nb.z) / lb};
        scatter(ia, ga);
        scatter(ib, gb);
    }
    return g;
}

uint32_t CountFlippedFacePairs(const CpuImage& pos, const CpuImage& faces,
                               const std::vector<std::array<uint32_t, 2>>& face_adj) {
    uint32_t n = 0;
    for (const auto& pr : face_adj) {
        uint32_t ia[3], ib[3];
        if (dot(face_cross(pos, faces, pr[0], ia), face_cross(pos, faces, pr[1], ib)) < 0.f) {
            n++;
        }
    }
    return n;
}

CpuImage ChainRuleClipToPos(const CpuImage& g_clip, const Mat4& mvp) {
    CpuImage g(g_clip.width, 1, 3, 0.f);
    for (uint32_t v = 0; v < g_clip.width; v++) {
        for (uint32_t j = 0; j < 3; j++) {
            float acc = 0.f;
            for (uint32_t c = 0; c < 4; c++) {
                acc += g_clip.at(v, 0, c) * mvp[j * 4 + c];
            }
            g.at(v, 0, j) = acc;
        }
    }
    return g;
}

dressi::Variable TransformToClipVar(const dressi::Variable& pos, const Mat4& mvp) {
    using dressi::Variable;
    namespace F = dressi::F;
    const Variable x = F::GetX(pos), y = F::GetY(pos), z = F::GetZ(pos);
    const auto row = [&](size_t r) {
        return x * mvp[r] + y * mvp[4 + r] + z * mvp[8 + r] + mvp[12 + r];
    };
    return F::Vec4(row(0), row(1), row(2), row(3));
}

void AdamStep(AdamState& state, std::vector<float>& params, const std::vector<float>& grad,
              float lr) {
    if (grad.size() < params.size()) {
        throw std::runtime_error("AdamStep: gradient shorter than the parameters");
    }
    if (state.m.size() != params.size()) {
        state.m.assign(params.size(), 0.f);
        state.v.assign(params.size(), 0.f);
        state.t = 0;
    }
    state.t++;
    const float c1 = 1.f - std::pow(state.beta1, (float)state.t);
    const float c2 = 1.f - std::pow(state.beta2, (float)state.t);
    for (size_t i = 0; i < params.size(); i++) {
        const float gi = grad[i];
        state.m[i] = state.beta1 * state.m[i] + (1.f - state.beta1) * gi;
        state.v[i] = state.beta2 * state.v[i] + (1.f - state.beta2) * gi * gi;
        params[i] -= lr * (state.m[i] / c1) / (std::sqrt(state.v[i] / c2) + state.eps);
    }
}

}  // namespace dressi_examples
