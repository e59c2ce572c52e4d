// assets_cli -- a command-line driver over the examples' asset and geometry
// helpers (include/dressi_examples/*.h), for the CPU tests in
// tests/test_assets.py. Images travel as a small binary file: u32 width,
// height, channels, then width * height * channels float32.
//
//   assets_cli obj|gltf <mesh> <out prefix>       -> prefix.pos/.uv/.faces
//   assets_cli gltf_scene <file> <out prefix> [raw]  -> LoadGltfScene: prefix.pos/.uv/
//              .faces/.normal/.tangent/.base/.mr/.nmap/.occ/.emis (raw: normalize off)
//   assets_cli png_load|exr_load <file> <out>      (png_load: LoadImageRgb, PNG or JPEG)
//   assets_cli png_save|exr_save <in> <file>
//   assets_cli srgb|down <in> <out>
//   assets_cli tile <cols> <out> <in>...
//   assets_cli lookat ex ey ez cx cy cz ux uy uz <out>   (16 x 1 x 1)
//   assets_cli persp fovy aspect near far <out>
//   assets_cli mul <a> <b> <out>
//   assets_cli clip <pos> <mvp> <out>
//   assets_cli chain <g_clip> <mvp> <out>
//   assets_cli save_obj <pos> <uv> <faces> <file> [texture name]
//   assets_cli ico <level> <out prefix>; uvsphere <stacks> <slices> <out prefix>
//   assets_cli transfer <rest> <faces> <deformed> <dst> <out>
//   assets_cli lap <pos> <faces> <lambda> <out>       (vertex adjacency of faces)
//   assets_cli ncons <pos> <faces> <lambda> <out>     (face adjacency of faces;
//                                                      prints the flipped pair count)
//   assets_cli adam <params> <grads> <lr> <steps> <out>  (grads: steps x N)
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <stdexcept>

#include "dressi_examples/asset_utils.h"
#include "dressi_examples/geometry_utils.h"

using dressi::CpuImage;
using namespace dressi_examples;

namespace {

CpuImage read_img(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    uint32_t hdr[3] = {0, 0, 0};
    f.read((char*)hdr, sizeof(hdr));
    if (!f) {
        throw std::runtime_error("cannot read " + path);
    }
    CpuImage img(hdr[0], hdr[1], hdr[2]);
    f.read((char*)img.data.data(), (std::streamsize)(img.data.size() * sizeof(float)));
    if (!f) {
        throw std::runtime_error("short image file " + path);
    }
    return img;
}

void write_img(const std::string& path, const CpuImage& img) {
    std::ofstream f(path, std::ios::binary);
    const uint32_t hdr[3] = {img.width, img.height, img.channels};
    f.write((const char*)hdr, sizeof(hdr));
    f.write((const char*)img.data.data(), (std::streamsize)(img.data.size() * sizeof(float)));
    if (!f) {
        throw std::runtime_error("cannot write " + path);
    }
}

void write_mesh(const std::string& prefix, const Mesh& m) {
    write_img(prefix + ".pos", m.pos);
    write_img(prefix + ".uv", m.uv);
    write_img(prefix + ".faces", m.faces);
}

Mat4 mat_of(const CpuImage& img) {
    if (img.data.size() != 16) {
        throw std::runtime_error("a 4x4 matrix has 16 values");
    }
    Mat4 m{};
    std::memcpy(m.data(), img.data.data(), sizeof(float) * 16);
    return m;
}

CpuImage img_of(const Mat4& m) {
    CpuImage img(16, 1, 1);
    std::memcpy(img.data.data(), m.data(), sizeof(float) * 16);
    return img;
}

int run(int argc, char** argv) {
    if (argc < 2) {
        throw std::runtime_error("no command");
    }
    const std::string cmd = argv[1];
    auto arg = [&](int i) -> std::string {
        if (i >= argc) {
            throw std::runtime_error("missing argument");
        }
        return argv[i];
    };
    auto num = [&](int i) { return (float)std::strtod(arg(i).c_str(), nullptr); };
    if (cmd == "obj") {
        write_mesh(arg(3), LoadObjMesh(arg(2)));
    } else if (cmd == "gltf") {
        write_mesh(arg(3), LoadGltfMesh(arg(2)));
    } else if (cmd == "gltf_scene") {
        const GltfScene sc = LoadGltfScene(argv[2], !(argc > 4 && std::string(argv[4]) == "raw"));
        const std::string pre = argv[3];
        write_mesh(pre, sc.mesh);
        write_img(pre + ".normal", sc.normal);
        write_img(pre + ".tangent", sc.tangent);
        write_img(pre + ".base", sc.base_color);
        write_img(pre + ".mr", sc.metallic_roughness);
        write_img(pre + ".nmap", sc.normal_map);
        write_img(pre + ".occ", sc.occlusion);
        write_img(pre + ".emis", sc.emissive);
    } else if (cmd == "png_load") {
        write_img(arg(3), LoadImageRgb(arg(2)));
    } else if (cmd == "exr_load") {
        write_img(arg(3), LoadImageExr(arg(2)));
    } else if (cmd == "png_save") {
        SaveImagePng(arg(3), read_img(arg(2)));
    } else if (cmd == "exr_save") {
        SaveImageExr(arg(3), read_img(arg(2)));
    } else if (cmd == "srgb") {
        write_img(arg(3), SrgbToLinear(read_img(arg(2))));
    } else if (cmd == "down") {
        write_img(arg(3), DownsampleHalf(read_img(arg(2))));
    } else if (cmd == "tile") {
        std::vector<CpuImage> imgs;
        for (int i = 4; i < argc; i++) {
            imgs.push_back(read_img(argv[i]));
        }
        write_img(arg(3), TileImages(imgs, (uint32_t)std::atoi(arg(2).c_str())));
    } else if (cmd == "lookat") {
        write_img(arg(11), img_of(LookAt({num(2), num(3), num(4)}, {num(5), num(6), num(7)},
                                         {num(8), num(9), num(10)})));
    } else if (cmd == "persp") {
        write_img(arg(6), img_of(PerspectiveVk(num(2), num(3), num(4), num(5))));
    } else if (cmd == "mul") {
        write_img(arg(4), img_of(Mul(mat_of(read_img(arg(2))), mat_of(read_img(arg(3))))));
    } else if (cmd == "clip") {
        write_img(arg(4), TransformToClip(read_img(arg(2)), mat_of(read_img(arg(3)))));
    } else if (cmd == "chain") {
        write_img(arg(4), ChainRuleClipToPos(read_img(arg(2)), mat_of(read_img(arg(3)))));
    } else if (cmd == "save_obj") {
        Mesh m;
        m.pos = read_img(arg(2));
        m.uv = read_img(arg(3));
        m.faces = read_img(arg(4));
        if (argc > 6) {
            SaveTexturedObjMesh(arg(5), m, arg(6));
        } else {
            SaveObjMesh(arg(5), m);
        }
    } else if (cmd == "ico") {
        write_mesh(arg(3), GenerateIcosphere((uint32_t)std::atoi(arg(2).c_str())));
    } else if (cmd == "uvsphere") {
        write_mesh(arg(4), GenerateUvSphere((uint32_t)std::atoi(arg(2).c_str()),
                                            (uint32_t)std::atoi(arg(3).c_str())));
    } else if (cmd == "transfer") {
        write_img(arg(6), TransferDeformationByDirection(read_img(arg(2)), read_img(arg(3)),
                                                         read_img(arg(4)), read_img(arg(5))));
    } else if (cmd == "lap") {
        const CpuImage pos = read_img(arg(2));
        const auto adj = BuildVertexAdjacency(read_img(arg(3)), pos.width);
        write_img(arg(5), UniformLaplacianGrad(pos, adj, num(4)));
    } else if (cmd == "ncons") {
        const CpuImage pos = read_img(arg(2)), faces = read_img(arg(3));
        const auto fadj = BuildFaceAdjacency(faces);
        write_img(arg(5), NormalConsistencyGrad(pos, faces, fadj, num(4)));
        std::printf("flipped %u pairs %zu\n", CountFlippedFacePairs(pos, faces, fadj),
                    fadj.size());
    } else if (cmd == "adam") {
        const CpuImage p = read_img(arg(2)), g = read_img(arg(3));
        const int steps = std::atoi(arg(5).c_str());
        std::vector<float> params = p.data;
        AdamState st;
        for (int s = 0; s < steps; s++) {
            const size_t n = params.size();
            std::vector<float> gs(g.data.begin() + (ptrdiff_t)(s * n),
                                  g.data.begin() + (ptrdiff_t)((s + 1) * n));
            AdamStep(st, params, gs, num(4));
        }
        CpuImage out(p.width, p.height, p.channels);
        out.data = params;
        write_img(arg(6), out);
    } else {
        throw std::runtime_error("unknown command " + cmd);
    }
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        return run(argc, argv);
    } catch (const std::exception& e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 2;
    }
}
