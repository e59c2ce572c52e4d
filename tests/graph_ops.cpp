// graph_ops.cpp -- one small graph per op family of the F:: catalogue, run
// by DressiAD's generic executor (include/dressi/dressi.h); the test
// (tests/test_gpu_graph_ops.py) compares every output with the oracle's
// per-op functions or numpy.
//
//   graph_ops <case> <packing: rsp|naive> <in.bin> <out.bin>
// in.bin / out.bin: u32 count, then per image: u32 name length, name,
// u32 w, h, c, w*h*c f32. Gradients come out as "d<leaf>" for the
// upstream images "g*" fed in through a product with the output (the
// backward seeds every pixel and component with 1).
#include <cstdio>
#include <map>
#include <string>
#include <vector>

#include "dressi/dressi.h"

using namespace dressi;

namespace {

using Images = std::map<std::string, CpuImage>;

Images load(const char* path) {
    FILE* f = fopen(path, "rb");
    DRESSI_CHECK(f, "cannot open input");
    auto get = [&](void* p, size_t n) {
        DRESSI_CHECK(fread(p, 1, n, f) == n, "short input file");
    };
    uint32_t count = 0;
    get(&count, 4);
    Images out;
    for (uint32_t i = 0; i < count; i++) {
        uint32_t len = 0, whc[3];
        get(&len, 4);
        std::string name(len, ' ');
        get(&name[0], len);
        get(whc, 12);
        CpuImage img(whc[0], whc[1], whc[2]);
        get(img.data.data(), img.data.size() * 4);
        out[name] = std::move(img);
    }
    fclose(f);
    return out;
}

void save(const char* path, const Images& imgs) {
    FILE* f = fopen(path, "wb");
    DRESSI_CHECK(f, "cannot open output");
    const uint32_t count = (uint32_t)imgs.size();
    fwrite(&count, 4, 1, f);
    for (const auto& [name, img] : imgs) {
        const uint32_t len = (uint32_t)name.size();
        const uint32_t whc[3] = {img.width, img.height, img.channels};
        fwrite(&len, 4, 1, f);
        fwrite(name.data(), 1, len, f);
        fwrite(whc, 4, 3, f);
        fwrite(img.data.data(), 4, img.data.size(), f);
    }
    fclose(f);
}

VType vtype_of(uint32_t channels) {
    switch (channels) {
        case 1: return FLOAT;
        case 2: return VEC2;
        case 3: return VEC3;
        case 4: return VEC4;
        case 16: return MAT4;
        default: throw DressiError("no VType with that many channels");
    }
}

// One graph: leaves from the input images, named outputs, gradients of
// the leaves marked requires-grad.
struct Case {
    Images in;
    std::map<std::string, Variable> leaves;
    std::map<std::string, Variable> outs;
    Variables losses;
    Variables grad_leaves;

    Variable leaf(const std::string& name, bool grad = false) {
        auto it = leaves.find(name);
        if (it != leaves.end()) {
            return it->second;  // one leaf per input image
        }
        const CpuImage& img = in.at(name);
        Variable v(vtype_of(img.channels), img.getImgSize());
        if (grad) {
            grad_leaves.push_back(v);
        }
        leaves.emplace(name, v);
        return v;
    }
    float param(size_t i) const { return in.at("params").data.at(i); }
    uint32_t uparam(size_t i) const { return (uint32_t)param(i); }
    // output y; with an upstream image g, y * g joins the loss
    void out(const std::string& name, const Variable& y, const char* upstream = nullptr) {
        outs.emplace(name, y);
        if (upstream) {
            losses.push_back(y * leaf(upstream));
        }
    }
};

void build(const std::string& which, Case& c) {
    if (which == "texture") {
        Variable tex = c.leaf("tex", true), uv = c.leaf("uv"), inv = c.leaf("inv_uv");
        c.out("bilinear", F::TextureBilinear(tex, uv, inv), "g");
        Variable tex2 = c.leaf("tex2", true);
        c.out("nearest", F::Texture(tex2, uv, inv), "g2");
    } else if (which == "equirect") {
        Variable map = c.leaf("map", true), dir = c.leaf("dir");
        c.out("y", F::EquirectSample(map, dir), "g");
    } else if (which == "conv") {
        // one environment leaf per differentiated op: each gradient is one VJP
        const ImgSize o = {c.uparam(0), c.uparam(1)};
        c.out("irr", F::IrradianceConv(c.leaf("env1", true), o), "g_irr");
        c.out("pref", F::PrefilterConv(c.leaf("env2", true), o, c.param(2)), "g_pref");
        c.out("pool", F::AvgPool2x2(c.leaf("env3", true)), "g_pool");
        c.out("prefenv", F::PrefilterEnv(c.leaf("env"), o, c.param(2), c.uparam(3)));
        c.out("lut", F::BrdfIntegrationLut({c.uparam(4), c.uparam(5)}, c.uparam(6)));
    } else if (which == "matrix") {
        Variable a = c.leaf("a", true), b = c.leaf("b", true), v = c.leaf("v", true);
        Variable a2 = c.leaf("a2", true), a3 = c.leaf("a3", true), v2 = c.leaf("v2", true);
        c.out("ab", F::MatMul(a, b), "g_ab");
        c.out("av", F::MatMul(a2, v), "g_av");
        // a3's gradient: two matrix contributions (an elementwise matrix sum)
        c.out("at", F::Transpose(a3), "g_at");
        c.out("a3x2", a3 * 2.f, "g_a3x2");
        c.out("vv", F::OuterProduct(v2, v2), "g_vv");
    } else if (which == "math") {
        Variable x = c.leaf("x", true), y = c.leaf("y", true), z = c.leaf("z");
        Variable p = c.leaf("p", true), q = c.leaf("q", true);
        c.out("sin", F::Sin(x), "g");
        c.out("cos", F::Cos(x), "g");
        c.out("tan", F::Tan(x), "g");
        c.out("asin", F::Asin(x), "g");
        c.out("acos", F::Acos(x), "g");
        c.out("atan", F::Atan(x), "g");
        c.out("atan2", F::Atan2(x, y), "g");
        c.out("exp", F::Exp(x), "g");
        c.out("exp2", F::Exp2(x), "g");
        c.out("log", F::Log(y), "g");
        c.out("log2", F::Log2(y), "g");
        c.out("sqrt", F::Sqrt(y), "g");
        c.out("rsqrt", F::InverseSqrt(y), "g");
        c.out("abs", F::Abs(z));
        c.out("sign", F::Sign(z));
        c.out("floor", F::Floor(z));
        c.out("fract", F::Fract(z));
        c.out("mod", F::Mod(z, y));
        c.out("pow", F::Pow(y, x), "g");
        c.out("max", F::Max(x, y), "g");
        c.out("min", F::Min(x, y), "g");
        c.out("clamp", F::Clamp(z, F::Float(-0.5f), F::Float(0.5f)));
        c.out("mix", F::Mix(x, y, F::Float(0.25f)), "g");
        c.out("step", F::Step(x, y));
        c.out("smooth", F::SmoothStep(F::Float(0.2f), F::Float(0.8f), x));
        c.out("sigmoid", F::Sigmoid(z), "g");
        c.out("less", F::Less(x, y));
        c.out("gequal", F::GreaterEqual(x, y));
        c.out("dot", F::Dot(p, q), "g");
        c.out("cross", F::Cross(p, q), "g3");
        c.out("length", F::Length(p), "g");
        c.out("normalize", F::Normalize(p), "g3");
        c.out("reflect", F::Reflect(p, F::Normalize(q)), "g3");
        c.out("distance", F::Distance(p, q), "g");
        c.out("compsum", F::CompSum(p), "g");
        c.out("mean", F::Mean(p));
        c.out("sumall", F::SumAll(p));
        c.out("sum", F::Sum(x));
    } else if (which == "fetch") {
        Variable tex = c.leaf("tex"), row = c.leaf("row"), atlas = c.leaf("atlas");
        c.out("pixel", F::PixelFetch(tex, c.uparam(0), row));
        c.out("tile", F::TileFetch(atlas, row, c.uparam(1)));
    } else if (which == "regular") {
        Variable pos = c.leaf("pos"), nbrs = c.leaf("nbrs"), faces = c.leaf("faces");
        Variable fadj = c.leaf("fadj"), vf = c.leaf("vf");
        c.out("mean", F::VertexNeighborMean(pos, nbrs));
        Variable term = F::NormalConsistencyFaceTerm(pos, faces, fadj);
        c.out("term", term);
        c.out("grad", F::NormalConsistencyVertexGrad(term, pos, faces, vf));
    } else {
        throw DressiError("unknown case " + which);
    }
}

// Re-setting the loss after a step: the optimizer (momentum SGD whose state
// m is carried by addUpdate from inside it) runs again for the new graph. A:
// one step on loss 1, then two on loss 2 in the same DressiAD; B: a fresh
// DressiAD on loss 2 from A's state after its first step, two steps. A and
// B must agree on x, m and the function count (no stale update pairs).
int run_rebuild(const char* packing, const char* in_path, const char* out_path) {
    const Images in = load(in_path);
    const CpuImage& x0 = in.at("x");
    const CpuImage& tgt0 = in.at("tgt");
    const ImgSize sz = x0.getImgSize();
    struct Net {
        Variable x{VEC3, {1, 1}}, m{VEC3, {1, 1}}, tgt{VEC3, {1, 1}}, loss1, loss2;
    };
    auto make = [&]() {
        Net n;
        n.x = Variable(VEC3, sz);
        n.m = Variable(VEC3, sz);
        n.tgt = Variable(VEC3, sz);
        const Variable d1 = n.x - n.tgt;
        n.loss1 = F::Sum(F::CompSum(d1 * d1));
        const Variable d2 = n.x * 2.f - n.tgt;
        n.loss2 = F::Sum(F::CompSum(d2 * d2 * 0.5f));
        n.x.setRequiresGradRecursively();
        return n;
    };
    const auto mode = std::string(packing) == "naive" ? DressiAD::PackingMode::Naive
                                                      : DressiAD::PackingMode::RSP;
    auto setup = [&](DressiAD& ad, Net& n, const Variable& loss) {
        ad.setPackingMode(mode);
        ad.setLossVar(loss);
        ad.setOptimizer([&ad, &n](Variables xs, Variables gs) {
            const Variable m_new = n.m * 0.9f + gs[0];
            ad.addUpdate(n.m, m_new);
            return Variables{xs[0] - m_new * 0.1f};
        });
    };
    Images out;
    Net a = make();
    DressiAD ad_a(DressiAD::createContext());
    setup(ad_a, a, a.loss1);
    ad_a.sendImg(a.x, x0);
    ad_a.sendImg(a.m, CpuImage(sz.w, sz.h, 3, 0.f));
    ad_a.sendImg(a.tgt, tgt0);
    ad_a.execStep();
    const CpuImage x1 = ad_a.recvImg(a.x), m1 = ad_a.recvImg(a.m);
    ad_a.setLossVar(a.loss2);
    ad_a.execStep();
    ad_a.execStep();
    out["xa"] = ad_a.recvImg(a.x);
    out["ma"] = ad_a.recvImg(a.m);
    Net b = make();
    DressiAD ad_b(DressiAD::createContext());
    setup(ad_b, b, b.loss2);
    ad_b.sendImg(b.x, x1);
    ad_b.sendImg(b.m, m1);
    ad_b.sendImg(b.tgt, tgt0);
    ad_b.execStep();
    ad_b.execStep();
    out["xb"] = ad_b.recvImg(b.x);
    out["mb"] = ad_b.recvImg(b.m);
    save(out_path, out);
    printf("graph_ops rebuild: funcs_a=%zu funcs_b=%zu plan=%s\n", ad_a.getFuncCount(),
           ad_b.getFuncCount(), ad_a.getPlanName().c_str());
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 5) {
        fprintf(stderr, "usage: graph_ops <case> <rsp|naive> in.bin out.bin\n");
        return 2;
    }
    try {
        if (std::string(argv[1]) == "rebuild") {
            return run_rebuild(argv[2], argv[3], argv[4]);
        }
        Case c;
        c.in = load(argv[3]);
        build(argv[1], c);
        // the loss: every upstream product reduced to one FLOAT (components
        // summed, a matrix through its product with (1,1,1,1)), then over
        // the image; the backward hands each output exactly its upstream
        // image. Without gradients, the first output.
        Variable loss = c.outs.begin()->second;
        if (!c.losses.empty()) {
            Variables scalars;
            for (const auto& p : c.losses) {
                Variable x = p;
                if (IsMatrixVType(x.getVType())) {
                    x = F::MatMul(x, F::Vec4(1.f, 1.f, 1.f, 1.f));
                }
                if (NumComponents(x.getVType()) > 1) {
                    x = F::CompSum(x);
                }
                scalars.push_back(F::Sum(x));
            }
            loss = F::SumPixelWise(scalars);
        }
        // once the whole graph exists, as the reference examples do (the
        // flag reaches only nodes that already exist)
        for (auto& v : c.grad_leaves) {
            v.setRequiresGradRecursively();
        }
        DressiAD ad(DressiAD::createContext());
        ad.setPackingMode(std::string(argv[2]) == "naive" ? DressiAD::PackingMode::Naive
                                                          : DressiAD::PackingMode::RSP);
        ad.setLossVar(loss);
        for (const auto& [name, v] : c.outs) {
            ad.markOutput(v);
        }
        ad.setGradOutputsEnabled(!c.losses.empty());
        for (const auto& [name, v] : c.leaves) {
            ad.sendImg(v, c.in.at(name));
        }
        ad.execStep();
        Images out;
        for (const auto& [name, v] : c.outs) {
            out[name] = ad.recvImg(v);
        }
        if (!c.losses.empty()) {
            for (const auto& [leaf, grad] : ad.inputGrads()) {
                for (const auto& [name, v] : c.leaves) {
                    if (v == leaf) {
                        out["d" + name] = ad.recvImg(grad);
                    }
                }
            }
        }
        save(argv[4], out);
        printf("graph_ops %s: plan=%s stages=%zu substages=%zu funcs=%zu\n", argv[1],
               ad.getPlanName().c_str(), ad.getStageCount(), ad.getSubStageCount(),
               ad.getFuncCount());
    } catch (const std::exception& e) {
        fprintf(stderr, "graph_ops: %s\n", e.what());
        return 1;
    }
    return 0;
}
