// jpeg.cpp -- JPEG decoding for LoadImageRgb and LoadGltfScene's textures:
// the sequential DCT modes of ITU-T T.81 (baseline SOF0 and extended
// sequential SOF1), Huffman-coded, 8-bit samples, 1 or 3 components with
// sampling factors 1..4, restart intervals included. Progressive,
// lossless, hierarchical and arithmetic-coded files are rejected. Host code.
//
// The reference decodes JPEG through stb_image, a third-party library that
// is not part of its sources. What T.81 fixes -- the marker syntax, the
// Huffman and DC / AC decoding, dequantisation -- is decoded here as the
// standard specifies. The rest is a choice of each decoder, made here as
// follows: the inverse DCT is evaluated from its definition (T.81 A.3.3)
// in double precision and rounded to nearest; chroma subsampled 2x1 or 2x2
// is upsampled with the triangle ("fancy") filter of the IJG's libjpeg
// (other factors replicate); YCbCr -> RGB is the JFIF transform rounded to
// nearest (no transform for an Adobe APP14 marker with transform 0, or for
// components named 'R', 'G', 'B'). A decoder with an integer IDCT or other
// upsampling can differ from these samples by a few units.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>

#include "image_codecs.h"

namespace dressi_examples {
namespace codec {

namespace {

[[noreturn]] void bad(const std::string& what, const std::string& why) {
    throw std::runtime_error("Failed to load image: " + what + " (JPEG: " + why + ")");
}

// natural (row-major) index of the k-th coefficient in zig-zag order
// (T.81 Figure 5)
constexpr uint8_t kZigzag[64] = {0,  1,  8,  16, 9,  2,  3,  10, 17, 24, 32, 25, 18, 11, 4,  5,
                                 12, 19, 26, 33, 40, 48, 41, 34, 27, 20, 13, 6,  7,  14, 21, 28,
                                 35, 42, 49, 56, 57, 50, 43, 36, 29, 22, 15, 23, 30, 37, 44, 51,
                                 58, 59, 52, 45, 38, 31, 39, 46, 53, 60, 61, 54, 47, 55, 62, 63};

// A Huffman table in the form of T.81 F.2.2.3's DECODE: per code length l,
// the largest code of that length (-1: none), the index of its first value
// and its first code.
struct Huffman {
    bool defined = false;
    int32_t maxcode[17] = {};
    int32_t valptr[17] = {};
    int32_t mincode[17] = {};
    uint8_t vals[256] = {};
};

void build_huffman(Huffman& h, const uint8_t* counts, const uint8_t* vals, size_t nvals,
                   const std::string& what) {
    std::memcpy(h.vals, vals, nvals);
    int32_t code = 0;
    int32_t k = 0;
    for (int l = 1; l <= 16; l++) {
        const int32_t n = counts[l - 1];
        if (n) {
            h.valptr[l] = k;
            h.mincode[l] = code;
            code += n;
            k += n;
            h.maxcode[l] = code - 1;
            if (code > (1 << l)) {
                bad(what, "over-subscribed Huffman table");
            }
        } else {
            h.maxcode[l] = -1;
        }
        code <<= 1;
    }
    h.defined = true;
}

// The entropy-coded bytes of a scan, MSB first, with 0xFF 0x00 stuffing
// removed. At a marker the reader stays in front of it and supplies zero
// bits.
struct BitReader {
    const uint8_t* p;
    const uint8_t* end;
    uint32_t buf = 0;
    int n = 0;
    bool at_marker = false;

    void fill() {
        uint32_t b = 0;
        if (!at_marker && p < end) {
            b = *p;
            if (b == 0xFFu) {
                if (p + 1 < end && p[1] == 0x00) {
                    p += 2;
                } else {
                    at_marker = true;
                    b = 0;
                }
            } else {
                p++;
            }
        }
        buf = (buf << 8) | b;
        n += 8;
    }
    uint32_t bit() {
        if (n == 0) {
            fill();
        }
        n--;
        return (buf >> n) & 1u;
    }
    uint32_t bits(int s) {
        uint32_t v = 0;
        for (int i = 0; i < s; i++) {
            v = (v << 1) | bit();
        }
        return v;
    }
    int decode(const Huffman& h, const std::string& what) {
        int32_t code = (int32_t)bit();
        for (int l = 1; l <= 16; l++) {
            if (h.maxcode[l] >= 0 && code <= h.maxcode[l] && code >= h.mincode[l]) {
                return h.vals[h.valptr[l] + code - h.mincode[l]];
            }
            code = (code << 1) | (int32_t)bit();
        }
        bad(what, "bad Huffman code");
    }
    // T.81 F.2.2.1 EXTEND of a RECEIVE(s)
    int32_t receive_extend(int s) {
        if (s == 0) {
            return 0;
        }
        const int32_t v = (int32_t)bits(s);
        return v < (1 << (s - 1)) ? v - (1 << s) + 1 : v;
    }
};

struct Component {
    uint8_t id = 0;
    int h = 1, v = 1, tq = 0, td = 0, ta = 0;
    uint32_t bw = 0, bh = 0;     // blocks across / down of the plane (whole MCUs)
    std::vector<uint8_t> plane;  // bw * 8 x bh * 8 samples
    int32_t pred = 0;
    bool scanned = false;
};

// cos table of the inverse DCT: t[x][u] = C(u) / 2 cos((2x + 1) u pi / 16)
struct IdctTable {
    double t[8][8];
    IdctTable() {
        const double pi = 3.14159265358979323846;
        for (int x = 0; x < 8; x++) {
            for (int u = 0; u < 8; u++) {
                const double cu = u == 0 ? 1.0 / std::sqrt(2.0) : 1.0;
                t[x][u] = 0.5 * cu * std::cos((2.0 * x + 1.0) * u * pi / 16.0);
            }
        }
    }
};

// s(y, x) = sum_v sum_u t[y][v] t[x][u] S(v, u) + 128, rounded and clamped
void idct_block(const int32_t* coef, uint8_t* dst, size_t stride) {
    static const IdctTable T;
    double tmp[8][8];  // [v][x]
    for (int v = 0; v < 8; v++) {
        for (int x = 0; x < 8; x++) {
            double s = 0.0;
            for (int u = 0; u < 8; u++) {
                s += T.t[x][u] * (double)coef[v * 8 + u];
            }
            tmp[v][x] = s;
        }
    }
    for (int y = 0; y < 8; y++) {
        for (int x = 0; x < 8; x++) {
            double s = 0.0;
            for (int v = 0; v < 8; v++) {
                s += T.t[y][v] * tmp[v][x];
            }
            const double r = std::floor(s + 128.0 + 0.5);
            dst[(size_t)y * stride + x] = (uint8_t)(r < 0.0 ? 0.0 : (r > 255.0 ? 255.0 : r));
        }
    }
}

uint8_t clamp8(int v) { return (uint8_t)(v < 0 ? 0 : (v > 255 ? 255 : v)); }

// Upsamples one component plane (cw x ch valid samples) by (fx, fy) to
// out_w x out_h: the libjpeg triangle filter for 2x1 and 2x2, else
// replication.
std::vector<uint8_t> upsample(const Component& c, uint32_t cw, uint32_t ch, int fx, int fy,
                              uint32_t out_w, uint32_t out_h) {
    const size_t stride = (size_t)c.bw * 8;
    auto at = [&](uint32_t x, uint32_t y) -> int {
        x = std::min(x, cw - 1);
        y = std::min(y, ch - 1);
        return c.plane[(size_t)y * stride + x];
    };
    std::vector<uint8_t> out((size_t)out_w * out_h);
    if (fx == 1 && fy == 1) {
        for (uint32_t y = 0; y < out_h; y++) {
            for (uint32_t x = 0; x < out_w; x++) {
                out[(size_t)y * out_w + x] = (uint8_t)at(x, y);
            }
        }
    } else if (fx == 2 && fy == 1) {
        // out(2i) = (3 in(i) + in(i - 1) + 1) >> 2, out(2i + 1) = (3 in(i) + in(i + 1) + 2) >> 2,
        // the row's first and last outputs copied
        for (uint32_t y = 0; y < out_h; y++) {
            for (uint32_t x = 0; x < out_w; x++) {
                const uint32_t i = x / 2;
                int v;
                if (cw == 1) {
                    v = at(0, y);
                } else if (x == 0) {
                    v = at(0, y);
                } else if (i == cw - 1 && (x & 1u)) {
                    v = at(cw - 1, y);
                } else if ((x & 1u) == 0) {
                    v = (3 * at(i, y) + at(i - 1, y) + 1) >> 2;
                } else {
                    v = (3 * at(i, y) + at(i + 1, y) + 2) >> 2;
                }
                out[(size_t)y * out_w + x] = (uint8_t)v;
            }
        }
    } else if (fx == 2 && fy == 2) {
        // per output row: col(i) = 3 near(i) + far(i) (far: the input row
        // above for an even output row, below for an odd one, the edge row
        // itself at the borders), then out(2i) = (3 col(i) + col(i - 1) +
        // 8) >> 4, out(2i + 1) = (3 col(i) + col(i + 1) + 7) >> 4; the
        // row's first / last output (4 col + 8) >> 4 / (4 col + 7) >> 4
        std::vector<int> col(cw);
        for (uint32_t y = 0; y < out_h; y++) {
            const uint32_t j = y / 2;
            const uint32_t far = (y & 1u) ? (j + 1 < ch ? j + 1 : j) : (j > 0 ? j - 1 : 0);
            for (uint32_t i = 0; i < cw; i++) {
                col[i] = 3 * at(i, j) + at(i, far);
            }
            for (uint32_t x = 0; x < out_w; x++) {
                const uint32_t i = std::min(x / 2, cw - 1);
                int v;
                if (cw == 1) {
                    v = (x & 1u) ? (4 * col[0] + 7) >> 4 : (4 * col[0] + 8) >> 4;
                } else if (x == 0) {
                    v = (4 * col[0] + 8) >> 4;
                } else if (i == cw - 1 && (x & 1u)) {
                    v = (4 * col[cw - 1] + 7) >> 4;
                } else if ((x & 1u) == 0) {
                    v = (3 * col[i] + col[i - 1] + 8) >> 4;
                } else {
                    v = (3 * col[i] + col[i + 1] + 7) >> 4;
                }
                out[(size_t)y * out_w + x] = (uint8_t)v;
            }
        }
    } else {
        for (uint32_t y = 0; y < out_h; y++) {
            for (uint32_t x = 0; x < out_w; x++) {
                out[(size_t)y * out_w + x] = (uint8_t)at(x / (uint32_t)fx, y / (uint32_t)fy);
            }
        }
    }
    return out;
}

}  // namespace

Image8 DecodeJpeg(const uint8_t* data, size_t n, const std::string& what) {
    if (n < 4 || data[0] != 0xFF || data[1] != 0xD8) {
        bad(what, "no SOI marker");
    }
    uint16_t qt[4][64] = {};  // zig-zag order
    bool qdef[4] = {false, false, false, false};
    Huffman hdc[4], hac[4];
    std::vector<Component> comps;
    uint32_t X = 0, Y = 0;
    int hmax = 1, vmax = 1;
    uint32_t mcux = 0, mcuy = 0;
    uint32_t restart = 0;
    bool frame = false, adobe_rgb = false, eoi = false;
    size_t pos = 2;
    auto be16 = [&](size_t at) -> uint32_t {
        if (at + 2 > n) {
            bad(what, "truncated segment");
        }
        return ((uint32_t)data[at] << 8) | data[at + 1];
    };
    while (pos < n && !eoi) {
        // a marker: 0xFF (fill bytes allowed) then its code
        if (data[pos] != 0xFF) {
            bad(what, "expected a marker");
        }
        while (pos < n && data[pos] == 0xFF) {
            pos++;
        }
        if (pos >= n) {
            bad(what, "truncated marker");
        }
        const uint8_t m = data[pos++];
        if (m == 0xD9) {
            eoi = true;
            break;
        }
        if (m >= 0xD0 && m <= 0xD7) {
            continue;  // a stray restart marker
        }
        const uint32_t len = be16(pos);
        if (len < 2 || pos + len > n) {
            bad(what, "truncated segment");
        }
        const uint8_t* seg = data + pos + 2;
        const size_t slen = len - 2;
        const size_t next = pos + len;
        switch (m) {
            case 0xDB: {  // DQT
                size_t o = 0;
                while (o < slen) {
                    const int pq = seg[o] >> 4, tq = seg[o] & 15;
                    o++;
                    if (tq > 3 || pq > 1 || o + (pq ? 128u : 64u) > slen) {
                        bad(what, "bad quantisation table");
                    }
                    for (int k = 0; k < 64; k++) {
                        qt[tq][k] = pq ? (uint16_t)((seg[o + 2 * k] << 8) | seg[o + 2 * k + 1])
                                       : seg[o + k];
                    }
                    o += pq ? 128u : 64u;
                    qdef[tq] = true;
                }
                break;
            }
            case 0xC4: {  // DHT
                size_t o = 0;
                while (o < slen) {
                    if (o + 17 > slen) {
                        bad(what, "bad Huffman table");
                    }
                    const int tc = seg[o] >> 4, th = seg[o] & 15;
                    const uint8_t* counts = seg + o + 1;
                    size_t nv = 0;
                    for (int l = 0; l < 16; l++) {
                        nv += counts[l];
                    }
                    if (tc > 1 || th > 3 || nv > 256 || o + 17 + nv > slen) {
                        bad(what, "bad Huffman table");
                    }
                    build_huffman(tc ? hac[th] : hdc[th], counts, seg + o + 17, nv, what);
                    o += 17 + nv;
                }
                break;
            }
            case 0xC0:
            case 0xC1: {  // SOF0 / SOF1: sequential DCT, Huffman
                if (frame) {
                    bad(what, "more than one frame");
                }
                if (slen < 6 || seg[0] != 8) {
                    bad(what, "only 8-bit samples are supported");
                }
                Y = (uint32_t)((seg[1] << 8) | seg[2]);
                X = (uint32_t)((seg[3] << 8) | seg[4]);
                const int nf = seg[5];
                if (X == 0 || Y == 0) {
                    bad(what, "zero image size (DNL) is not supported");
                }
                if ((nf != 1 && nf != 3) || slen < 6u + 3u * (size_t)nf) {
                    bad(what, "only 1 or 3 components are supported");
                }
                comps.resize((size_t)nf);
                for (int i = 0; i < nf; i++) {
                    Component& c = comps[(size_t)i];
                    c.id = seg[6 + 3 * i];
                    c.h = seg[7 + 3 * i] >> 4;
                    c.v = seg[7 + 3 * i] & 15;
                    c.tq = seg[8 + 3 * i];
                    if (c.h < 1 || c.h > 4 || c.v < 1 || c.v > 4 || c.tq > 3) {
                        bad(what, "bad component parameters");
                    }
                    hmax = std::max(hmax, c.h);
                    vmax = std::max(vmax, c.v);
                }
                mcux = (X + 8u * (uint32_t)hmax - 1u) / (8u * (uint32_t)hmax);
                mcuy = (Y + 8u * (uint32_t)vmax - 1u) / (8u * (uint32_t)vmax);
                if ((uint64_t)mcux * mcuy * 64u * (uint64_t)hmax * (uint64_t)vmax > (1ull << 31)) {
                    bad(what, "image too large");
                }
                for (Component& c : comps) {
                    c.bw = mcux * (uint32_t)c.h;
                    c.bh = mcuy * (uint32_t)c.v;
                    c.plane.assign((size_t)c.bw * 8 * c.bh * 8, 0);
                }
                frame = true;
                break;
            }
            case 0xC2:
            case 0xC3:
            case 0xC5:
            case 0xC6:
            case 0xC7:
            case 0xC9:
            case 0xCA:
            case 0xCB:
            case 0xCD:
            case 0xCE:
            case 0xCF: bad(what, "only sequential Huffman-coded (baseline) files are supported");
            case 0xDD:  // DRI
                if (slen < 2) {
                    bad(what, "bad restart interval");
                }
                restart = (uint32_t)((seg[0] << 8) | seg[1]);
                break;
            case 0xEE:  // APP14 (Adobe): transform 0 = components stored as RGB
                if (slen >= 12 && std::memcmp(seg, "Adobe", 5) == 0) {
                    adobe_rgb = seg[11] == 0;
                }
                break;
            case 0xDA: {  // SOS, then the entropy-coded segment
                if (!frame) {
                    bad(what, "scan before the frame header");
                }
                const int ns = slen ? seg[0] : 0;
                if (ns < 1 || ns > 4 || slen < 4u + 2u * (size_t)ns) {
                    bad(what, "bad scan header");
                }
                std::vector<Component*> sc;
                for (int i = 0; i < ns; i++) {
                    Component* c = nullptr;
                    for (Component& k : comps) {
                        if (k.id == seg[1 + 2 * i]) {
                            c = &k;
                        }
                    }
                    if (!c) {
                        bad(what, "scan names an unknown component");
                    }
                    c->td = seg[2 + 2 * i] >> 4;
                    c->ta = seg[2 + 2 * i] & 15;
                    if (c->td > 3 || c->ta > 3 || !hdc[c->td].defined || !hac[c->ta].defined ||
                        !qdef[c->tq]) {
                        bad(what, "scan uses an undefined table");
                    }
                    c->pred = 0;
                    c->scanned = true;
                    sc.push_back(c);
                }
                const uint8_t ss = seg[1 + 2 * ns], se = seg[2 + 2 * ns], a = seg[3 + 2 * ns];
                if (ss != 0 || se != 63 || a != 0) {
                    bad(what, "spectral selection in a sequential scan");
                }
                BitReader br{data + next, data + n};
                // one block: DC difference, AC run / size codes (T.81 F.2.2)
                auto block = [&](Component& c, uint32_t bx, uint32_t by) {
                    int32_t coef[64] = {};
                    const uint16_t* q = qt[c.tq];
                    const int t = br.decode(hdc[c.td], what);
                    if (t > 15) {
                        bad(what, "bad DC code");
                    }
                    c.pred += br.receive_extend(t);
                    coef[0] = c.pred * (int32_t)q[0];
                    for (int k = 1; k < 64;) {
                        const int rs = br.decode(hac[c.ta], what);
                        const int r = rs >> 4, s = rs & 15;
                        if (s == 0) {
                            if (r != 15) {
                                break;  // EOB
                            }
                            k += 16;
                            continue;
                        }
                        k += r;
                        if (k > 63) {
                            bad(what, "AC coefficients past the block");
                        }
                        coef[kZigzag[k]] = br.receive_extend(s) * (int32_t)q[k];
                        k++;
                    }
                    const size_t stride = (size_t)c.bw * 8;
                    idct_block(coef, &c.plane[(size_t)by * 8 * stride + (size_t)bx * 8], stride);
                };
                // restart: byte-align, step over the RSTn marker, reset the
                // DC predictions
                auto restart_here = [&]() {
                    br.n = 0;
                    br.buf = 0;
                    const uint8_t* p = br.p;
                    while (p + 1 < br.end && !(p[0] == 0xFF && p[1] >= 0xD0 && p[1] <= 0xD7)) {
                        p++;
                    }
                    br.p = p + 1 < br.end ? p + 2 : br.end;
                    br.at_marker = false;
                    for (Component* c : sc) {
                        c->pred = 0;
                    }
                };
                uint64_t units = 0;
                if (ns == 1) {
                    // non-interleaved: the component's own blocks in raster order
                    Component& c = *sc[0];
                    const uint32_t cw = (X * (uint32_t)c.h + (uint32_t)hmax - 1) / (uint32_t)hmax;
                    const uint32_t chh = (Y * (uint32_t)c.v + (uint32_t)vmax - 1) / (uint32_t)vmax;
                    const uint32_t nbx = (cw + 7) / 8, nby = (chh + 7) / 8;
                    for (uint32_t by = 0; by < nby; by++) {
                        for (uint32_t bx = 0; bx < nbx; bx++) {
                            if (restart && units && units % restart == 0) {
                                restart_here();
                            }
                            block(c, bx, by);
                            units++;
                        }
                    }
                } else {
                    for (uint32_t my = 0; my < mcuy; my++) {
                        for (uint32_t mx = 0; mx < mcux; mx++) {
                            if (restart && units && units % restart == 0) {
                                restart_here();
                            }
                            for (Component* c : sc) {
                                for (int by = 0; by < c->v; by++) {
                                    for (int bx = 0; bx < c->h; bx++) {
                                        block(*c, mx * (uint32_t)c->h + (uint32_t)bx,
                                              my * (uint32_t)c->v + (uint32_t)by);
                                    }
                                }
                            }
                            units++;
                        }
                    }
                }
                // the next marker after the entropy-coded data
                const uint8_t* p = br.p;
                while (p + 1 < br.end &&
                       !(p[0] == 0xFF && p[1] != 0x00 && !(p[1] >= 0xD0 && p[1] <= 0xD7))) {
                    p++;
                }
                pos = (size_t)(p - data);
                if (p + 1 >= br.end) {
                    pos = n;
                }
                continue;
            }
            default: break;  // APPn, COM and others: skipped
        }
        pos = next;
    }
    if (!frame) {
        bad(what, "no frame header");
    }
    for (const Component& c : comps) {
        if (!c.scanned) {
            bad(what, "a component has no scan (truncated file?)");
        }
    }
    Image8 img;
    img.width = X;
    img.height = Y;
    img.comp = (uint32_t)comps.size();
    img.px.assign((size_t)X * Y * img.comp, 0);
    std::vector<std::vector<uint8_t>> full;
    for (Component& c : comps) {
        const uint32_t cw = (X * (uint32_t)c.h + (uint32_t)hmax - 1) / (uint32_t)hmax;
        const uint32_t chh = (Y * (uint32_t)c.v + (uint32_t)vmax - 1) / (uint32_t)vmax;
        if (hmax % c.h || vmax % c.v) {
            bad(what, "non-integral sampling ratio");
        }
        full.push_back(upsample(c, cw, chh, hmax / c.h, vmax / c.v, X, Y));
    }
    const size_t np = (size_t)X * Y;
    if (img.comp == 1) {
        img.px = full[0];
        return img;
    }
    const bool rgb_ids = comps[0].id == 'R' && comps[1].id == 'G' && comps[2].id == 'B';
    for (size_t i = 0; i < np; i++) {
        const double y = full[0][i], cb = (double)full[1][i] - 128.0, cr = (double)full[2][i] - 128.0;
        if (adobe_rgb || rgb_ids) {
            img.px[i * 3 + 0] = full[0][i];
            img.px[i * 3 + 1] = full[1][i];
            img.px[i * 3 + 2] = full[2][i];
            continue;
        }
        // JFIF: R = Y + 1.402 Cr, G = Y - 0.344136 Cb - 0.714136 Cr, B = Y + 1.772 Cb
        img.px[i * 3 + 0] = clamp8((int)std::floor(y + 1.402 * cr + 0.5));
        img.px[i * 3 + 1] = clamp8((int)std::floor(y - 0.344136 * cb - 0.714136 * cr + 0.5));
        img.px[i * 3 + 2] = clamp8((int)std::floor(y + 1.772 * cb + 0.5));
    }
    return img;
}

Image8 DecodeImage(const uint8_t* data, size_t n, const std::string& what) {
    static const uint8_t png_sig[8] = {137, 80, 78, 71, 13, 10, 26, 10};
    if (n >= 8 && std::memcmp(data, png_sig, 8) == 0) {
        return DecodePng(data, n, what);
    }
    if (n >= 2 && data[0] == 0xFF && data[1] == 0xD8) {
        return DecodeJpeg(data, n, what);
    }
    throw std::runtime_error("Failed to load image: " + what + " (neither PNG nor JPEG)");
}

}  // namespace codec
}  // namespace dressi_examples
