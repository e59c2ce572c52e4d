// assets.cpp -- the examples' asset and matrix helpers
// (include/dressi_examples/asset_utils.h; the reference's
// examples/common/asset_utils.cpp:41-782 and geometry_utils.cpp:199-213).
// Host code; zlib for the deflate streams of PNG and OpenEXR.
//
// The reference reads these formats through third-party libraries that
// are not part of its sources (tinyobjloader, tinygltf, tinyexr, stb_image
// / stb_image_write); what they return for the files the examples use is
// fixed by the formats themselves, which this file reads directly. The
// mesh post-processing (unwelding, the v flip, the normalisation) follows
// the reference's code, operation for operation.
#include <zlib.h>

#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <sstream>
#include <stdexcept>

#include "dressi_examples/asset_utils.h"
#include "image_codecs.h"
#include "dressi_hip.h"

namespace dressi_examples {

using dressi::CpuImage;

namespace {

[[noreturn]] void fail(const std::string& what) { throw std::runtime_error(what); }

std::vector<uint8_t> read_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) {
        fail("cannot open " + path);
    }
    return std::vector<uint8_t>((std::istreambuf_iterator<char>(f)),
                                std::istreambuf_iterator<char>());
}

void write_file(const std::string& path, const std::vector<uint8_t>& bytes, const char* what) {
    std::ofstream f(path, std::ios::binary);
    f.write((const char*)bytes.data(), (std::streamsize)bytes.size());
    if (!f) {
        fail(what + path);
    }
}

std::vector<uint8_t> inflate_all(const uint8_t* src, size_t n, size_t expect) {
    std::vector<uint8_t> out(expect);
    uLongf len = (uLongf)expect;
    if (uncompress(out.data(), &len, src, (uLong)n) != Z_OK || len != expect) {
        fail("corrupt deflate stream");
    }
    return out;
}

// a zlib stream of unknown decompressed size (PNG's IDAT)
std::vector<uint8_t> inflate_stream(const std::vector<uint8_t>& src) {
    z_stream zs{};
    if (inflateInit(&zs) != Z_OK) {
        fail("zlib init failed");
    }
    std::vector<uint8_t> out;
    std::vector<uint8_t> buf(1 << 16);
    zs.next_in = (Bytef*)src.data();
    zs.avail_in = (uInt)src.size();
    int rc = Z_OK;
    while (rc != Z_STREAM_END) {
        zs.next_out = buf.data();
        zs.avail_out = (uInt)buf.size();
        rc = inflate(&zs, Z_NO_FLUSH);
        if (rc != Z_OK && rc != Z_STREAM_END) {
            inflateEnd(&zs);
            fail("corrupt deflate stream");
        }
        out.insert(out.end(), buf.begin(), buf.begin() + (buf.size() - zs.avail_out));
        if (rc == Z_OK && zs.avail_in == 0 && zs.avail_out != 0) {
            inflateEnd(&zs);
            fail("truncated deflate stream");
        }
    }
    inflateEnd(&zs);
    return out;
}

std::vector<uint8_t> deflate_all(const uint8_t* src, size_t n) {
    uLongf len = compressBound((uLong)n);
    std::vector<uint8_t> out(len);
    if (compress2(out.data(), &len, src, (uLong)n, Z_DEFAULT_COMPRESSION) != Z_OK) {
        fail("deflate failed");
    }
    out.resize(len);
    return out;
}

// ---- mesh normalisation -------------------------------------------------------

// glTF (asset_utils.cpp:41-61): extent floored at 1e-12, (p - c) / extent
void normalise_divide(Mesh& m) {
    float lo[3] = {1e30f, 1e30f, 1e30f}, hi[3] = {-1e30f, -1e30f, -1e30f};
    for (uint32_t v = 0; v < m.numVertices(); v++) {
        for (uint32_t c = 0; c < 3; c++) {
            lo[c] = std::min(lo[c], m.pos.at(v, 0, c));
            hi[c] = std::max(hi[c], m.pos.at(v, 0, c));
        }
    }
    float ext = 1e-12f;
    for (uint32_t c = 0; c < 3; c++) {
        ext = std::max(ext, hi[c] - lo[c]);
    }
    for (uint32_t v = 0; v < m.numVertices(); v++) {
        for (uint32_t c = 0; c < 3; c++) {
            m.pos.at(v, 0, c) = (m.pos.at(v, 0, c) - 0.5f * (lo[c] + hi[c])) / ext;
        }
    }
}

// ---- a small JSON reader (glTF) ---------------------------------------------------

struct Json {
    enum Kind { kNull, kBool, kNum, kStr, kArr, kObj } kind = kNull;
    double num = 0.0;
    bool flag = false;
    std::string str;
    std::vector<Json> arr;
    std::map<std::string, Json> obj;

    const Json* get(const std::string& k) const {
        if (kind != kObj) {
            return nullptr;
        }
        auto it = obj.find(k);
        return it == obj.end() ? nullptr : &it->second;
    }
    const Json& at(const std::string& k) const {
        const Json* j = get(k);
        if (!j) {
            fail("glTF: missing \"" + k + "\"");
        }
        return *j;
    }
    const Json& at(size_t i) const {
        if (kind != kArr || i >= arr.size()) {
            fail("glTF: index out of range");
        }
        return arr[i];
    }
    double number(double fallback) const { return kind == kNum ? num : fallback; }
};

class JsonParser {
public:
    JsonParser(const char* p, const char* end) : p_(p), end_(end) {}
    Json parse() {
        Json j = value();
        ws();
        if (p_ != end_) {
            fail("glTF: trailing characters in JSON");
        }
        return j;
    }

private:
    const char* p_;
    const char* end_;

    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) {
            p_++;
        }
    }
    char peek() {
        ws();
        if (p_ >= end_) {
            fail("glTF: unexpected end of JSON");
        }
        return *p_;
    }
    void expect(char c) {
        if (peek() != c) {
            fail(std::string("glTF: expected '") + c + "' in JSON");
        }
        p_++;
    }
    static void put_utf8(std::string& s, uint32_t cp) {
        if (cp < 0x80) {
            s += (char)cp;
        } else if (cp < 0x800) {
            s += (char)(0xc0 | (cp >> 6));
            s += (char)(0x80 | (cp & 0x3f));
        } else if (cp < 0x10000) {
            s += (char)(0xe0 | (cp >> 12));
            s += (char)(0x80 | ((cp >> 6) & 0x3f));
            s += (char)(0x80 | (cp & 0x3f));
        } else {
            s += (char)(0xf0 | (cp >> 18));
            s += (char)(0x80 | ((cp >> 12) & 0x3f));
            s += (char)(0x80 | ((cp >> 6) & 0x3f));
            s += (char)(0x80 | (cp & 0x3f));
        }
    }
    uint32_t hex4() {
        if (end_ - p_ < 4) {
            fail("glTF: bad \\u escape");
        }
        uint32_t v = 0;
        for (int i = 0; i < 4; i++) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else fail("glTF: bad \\u escape");
        }
        return v;
    }
    std::string string() {
        expect('"');
        std::string s;
        while (true) {
            if (p_ >= end_) {
                fail("glTF: unterminated string");
            }
            const char c = *p_++;
            if (c == '"') {
                return s;
            }
            if (c != '\\') {
                s += c;
                continue;
            }
            if (p_ >= end_) {
                fail("glTF: unterminated string");
            }
            const char e = *p_++;
            switch (e) {
                case '"': s += '"'; break;
                case '\\': s += '\\'; break;
                case '/': s += '/'; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'n': s += '\n'; break;
                case 'r': s += '\r'; break;
                case 't': s += '\t'; break;
                case 'u': {
                    uint32_t cp = hex4();
                    if (cp >= 0xd800 && cp < 0xdc00 && end_ - p_ >= 6 && p_[0] == '\\' &&
                        p_[1] == 'u') {
                        p_ += 2;
                        const uint32_t lo = hex4();
                        cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
                    }
                    put_utf8(s, cp);
                    break;
                }
                default: fail("glTF: bad escape in string");
            }
        }
    }
    Json value() {
        Json j;
        const char c = peek();
        if (c == '{') {
            p_++;
            j.kind = Json::kObj;
            if (peek() == '}') {
                p_++;
                return j;
            }
            while (true) {
                std::string k = string();
                expect(':');
                j.obj[k] = value();
                const char d = peek();
                p_++;
                if (d == '}') {
                    return j;
                }
                if (d != ',') {
                    fail("glTF: expected ',' or '}' in JSON");
                }
            }
        }
        if (c == '[') {
            p_++;
            j.kind = Json::kArr;
            if (peek() == ']') {
                p_++;
                return j;
            }
            while (true) {
                j.arr.push_back(value());
                const char d = peek();
                p_++;
                if (d == ']') {
                    return j;
                }
                if (d != ',') {
                    fail("glTF: expected ',' or ']' in JSON");
                }
            }
        }
        if (c == '"') {
            j.kind = Json::kStr;
            j.str = string();
            return j;
        }
        auto word = [&](const char* w) {
            const size_t n = std::strlen(w);
            if ((size_t)(end_ - p_) >= n && std::strncmp(p_, w, n) == 0) {
                p_ += n;
                return true;
            }
            return false;
        };
        if (word("true")) {
            j.kind = Json::kBool;
            j.flag = true;
            return j;
        }
        if (word("false")) {
            j.kind = Json::kBool;
            return j;
        }
        if (word("null")) {
            return j;
        }
        const char* start = p_;
        while (p_ < end_ && (std::isdigit((unsigned char)*p_) || *p_ == '-' || *p_ == '+' ||
                             *p_ == '.' || *p_ == 'e' || *p_ == 'E')) {
            p_++;
        }
        if (p_ == start) {
            fail("glTF: bad JSON value");
        }
        j.kind = Json::kNum;
        j.num = std::strtod(std::string(start, p_).c_str(), nullptr);
        return j;
    }
};

std::vector<uint8_t> base64_decode(const std::string& s) {
    auto val = [](char c) -> int {
        if (c >= 'A' && c <= 'Z') return c - 'A';
        if (c >= 'a' && c <= 'z') return c - 'a' + 26;
        if (c >= '0' && c <= '9') return c - '0' + 52;
        if (c == '+') return 62;
        if (c == '/') return 63;
        return -1;
    };
    std::vector<uint8_t> out;
    uint32_t acc = 0;
    int bits = 0;
    for (char c : s) {
        if (c == '=') {
            break;
        }
        const int v = val(c);
        if (v < 0) {
            continue;  // whitespace
        }
        acc = (acc << 6) | (uint32_t)v;
        bits += 6;
        if (bits >= 8) {
            bits -= 8;
            out.push_back((uint8_t)((acc >> bits) & 0xffu));
        }
    }
    return out;
}

// %XX escapes of a relative URI
std::string uri_decode(const std::string& u) {
    std::string out;
    for (size_t i = 0; i < u.size(); i++) {
        if (u[i] == '%' && i + 2 < u.size() && std::isxdigit((unsigned char)u[i + 1]) &&
            std::isxdigit((unsigned char)u[i + 2])) {
            out += (char)std::stoi(u.substr(i + 1, 2), nullptr, 16);
            i += 2;
        } else {
            out += u[i];
        }
    }
    return out;
}

std::string dir_of(const std::string& path) {
    const size_t s = path.find_last_of("/\\");
    return s == std::string::npos ? std::string() : path.substr(0, s + 1);
}

struct Gltf {
    Json doc;
    std::vector<std::vector<uint8_t>> buffers;
};

Gltf load_gltf(const std::string& path) {
    const std::vector<uint8_t> file = read_file(path);
    Gltf g;
    std::vector<uint8_t> glb_bin;
    bool glb = false;
    if (file.size() >= 12 && std::memcmp(file.data(), "glTF", 4) == 0) {
        glb = true;
        uint32_t version = 0, total = 0;
        std::memcpy(&version, file.data() + 4, 4);
        std::memcpy(&total, file.data() + 8, 4);
        if (version != 2 || total > file.size()) {
            fail("glTF: unsupported .glb header in " + path);
        }
        size_t off = 12;
        bool have_json = false;
        while (off + 8 <= total) {
            uint32_t len = 0, type = 0;
            std::memcpy(&len, file.data() + off, 4);
            std::memcpy(&type, file.data() + off + 4, 4);
            off += 8;
            if (off + len > total) {
                fail("glTF: truncated .glb chunk in " + path);
            }
            if (type == 0x4E4F534Au) {  // JSON
                g.doc = JsonParser((const char*)file.data() + off,
                                   (const char*)file.data() + off + len)
                                .parse();
                have_json = true;
            } else if (type == 0x004E4942u) {  // BIN
                glb_bin.assign(file.begin() + (ptrdiff_t)off, file.begin() + (ptrdiff_t)(off + len));
            }
            off += (len + 3u) & ~3u;
        }
        if (!have_json) {
            fail("glTF: no JSON chunk in " + path);
        }
    } else {
        g.doc = JsonParser((const char*)file.data(), (const char*)file.data() + file.size()).parse();
    }
    if (const Json* bufs = g.doc.get("buffers")) {
        for (size_t i = 0; i < bufs->arr.size(); i++) {
            const Json& b = bufs->arr[i];
            const Json* uri = b.get("uri");
            std::vector<uint8_t> data;
            if (!uri) {
                if (!glb) {
                    fail("glTF: buffer without uri in " + path);
                }
                data = glb_bin;
            } else if (uri->str.rfind("data:", 0) == 0) {
                const size_t comma = uri->str.find(',');
                if (comma == std::string::npos ||
                    uri->str.substr(0, comma).find(";base64") == std::string::npos) {
                    fail("glTF: unsupported data uri in " + path);
                }
                data = base64_decode(uri->str.substr(comma + 1));
            } else {
                data = read_file(dir_of(path) + uri_decode(uri->str));
            }
            const size_t need = (size_t)b.at("byteLength").number(0.0);
            if (data.size() < need) {
                fail("glTF: buffer shorter than its byteLength in " + path);
            }
            g.buffers.push_back(std::move(data));
        }
    }
    return g;
}

// element i, component c of an accessor as float (asset_utils.cpp:65-99)
struct Accessor {
    const uint8_t* base = nullptr;
    size_t stride = 0, count = 0, comp_size = 0;
    uint32_t n_comp = 0, comp_type = 0;

    float read(size_t i, uint32_t c) const {
        if (i >= count || c >= n_comp) {
            fail("glTF: accessor read out of range");
        }
        const uint8_t* p = base + i * stride + c * comp_size;
        switch (comp_type) {
            case 5126: {
                float f;
                std::memcpy(&f, p, 4);
                return f;
            }
            case 5125: {
                uint32_t u;
                std::memcpy(&u, p, 4);
                return (float)u;
            }
            case 5123: {
                uint16_t u;
                std::memcpy(&u, p, 2);
                return (float)u;
            }
            case 5121: return (float)*p;
            default: fail("glTF: unsupported component type");
        }
    }
};

Accessor accessor(const Gltf& g, size_t idx) {
    const Json& acc = g.doc.at("accessors").at(idx);
    Accessor a;
    a.comp_type = (uint32_t)acc.at("componentType").number(0.0);
    a.count = (size_t)acc.at("count").number(0.0);
    const std::string& type = acc.at("type").str;
    a.n_comp = type == "SCALAR" ? 1 : type == "VEC2" ? 2 : type == "VEC3" ? 3
               : type == "VEC4" ? 4 : type == "MAT2" ? 4 : type == "MAT3" ? 9
               : type == "MAT4" ? 16 : 0;
    a.comp_size = a.comp_type == 5126 || a.comp_type == 5125 ? 4
                  : a.comp_type == 5123 || a.comp_type == 5122 ? 2
                  : a.comp_type == 5121 || a.comp_type == 5120 ? 1 : 0;
    if (!a.n_comp || !a.comp_size) {
        fail("glTF: unsupported accessor type");
    }
    const Json* bvi = acc.get("bufferView");
    if (!bvi) {
        fail("glTF: sparse / bufferView-less accessors are not supported");
    }
    const Json& bv = g.doc.at("bufferViews").at((size_t)bvi->number(0.0));
    const size_t buf = (size_t)bv.at("buffer").number(0.0);
    if (buf >= g.buffers.size()) {
        fail("glTF: bufferView names a missing buffer");
    }
    auto offset_of = [](const Json& j) {
        const Json* o = j.get("byteOffset");
        return o ? (size_t)o->number(0.0) : (size_t)0;
    };
    const size_t off = offset_of(bv) + offset_of(acc);
    const size_t elem = (size_t)a.n_comp * a.comp_size;
    a.stride = bv.get("byteStride") ? (size_t)bv.get("byteStride")->number(0.0) : elem;
    if (a.stride == 0) {
        a.stride = elem;
    }
    if (a.count && off + (a.count - 1) * a.stride + elem > g.buffers[buf].size()) {
        fail("glTF: accessor reads past its buffer");
    }
    a.base = g.buffers[buf].data() + off;
    return a;
}

// ---- OpenEXR ------------------------------------------------------------------------

float half_to_float(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = s;
        } else {  // subnormal: normalise
            uint32_t mm = m;
            int ee = -1;
            do {
                ee++;
                mm <<= 1;
            } while (!(mm & 0x400u));
            bits = s | (uint32_t)(127 - 15 - ee) << 23 | (mm & 0x3ffu) << 13;
        }
    } else if (e == 31) {
        bits = s | 0x7f800000u | m << 13;
    } else {
        bits = s | (e + 112u) << 23 | m << 13;
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// float -> half as the reference's writer converts (tinyexr v1.0.9 uses
// the ISPC reference conversion): the mantissa is truncated and then
// rounded up when the first dropped bit is set (ties round away from
// zero), a carry may overflow into the exponent (up to infinity); float
// subnormals become zero, exponents past the half range infinity, NaN a
// quiet NaN.
uint16_t float_to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t exp = (x >> 23) & 0xffu;
    const uint32_t mant = x & 0x7fffffu;
    uint32_t h = 0;
    if (exp == 0) {
        h = 0;
    } else if (exp == 255) {
        h = 0x7c00u | (mant ? 0x200u : 0u);
    } else {
        const int e = (int)exp - 127 + 15;
        if (e >= 31) {
            h = 0x7c00u;
        } else if (e <= 0) {
            if (14 - e <= 24) {
                const uint32_t m = mant | 0x800000u;
                h = m >> (14 - e);
                if ((m >> (13 - e)) & 1u) {
                    h++;
                }
            }
        } else {
            h = (uint32_t)e << 10 | mant >> 13;
            if (mant & 0x1000u) {
                h++;
            }
        }
    }
    return (uint16_t)(sign | h);
}

struct ExrChannel {
    std::string name;
    int type;  // 0 uint, 1 half, 2 float
    int xs, ys;
};

// OpenEXR's run-length code: a signed count byte, -n: n literal bytes
// follow; n >= 0: the next byte repeats n + 1 times
std::vector<uint8_t> rle_decode(const uint8_t* src, size_t n, size_t expect) {
    std::vector<uint8_t> out;
    out.reserve(expect);
    size_t i = 0;
    while (i < n) {
        const int c = (int8_t)src[i++];
        if (c < 0) {
            if (i + (size_t)(-c) > n) {
                fail("corrupt RLE block");
            }
            out.insert(out.end(), src + i, src + i + (-c));
            i += (size_t)(-c);
        } else {
            if (i >= n) {
                fail("corrupt RLE block");
            }
            out.insert(out.end(), (size_t)c + 1, src[i++]);
        }
        if (out.size() > expect) {
            fail("corrupt RLE block");
        }
    }
    if (out.size() != expect) {
        fail("corrupt RLE block");
    }
    return out;
}

// EXR's zip pre-processing: bytes split into even / odd halves, then a
// running-difference predictor; this undoes it
std::vector<uint8_t> exr_unzip_reorder(const std::vector<uint8_t>& raw) {
    std::vector<uint8_t> t = raw;
    for (size_t i = 1; i < t.size(); i++) {
        t[i] = (uint8_t)(t[i - 1] + t[i] - 128);
    }
    std::vector<uint8_t> out(t.size());
    const size_t half = (t.size() + 1) / 2;
    for (size_t i = 0; i < t.size(); i++) {
        out[i] = (i & 1u) ? t[half + i / 2] : t[i / 2];
    }
    return out;
}

std::vector<uint8_t> exr_zip_reorder(const std::vector<uint8_t>& src) {
    std::vector<uint8_t> t(src.size());
    const size_t half = (src.size() + 1) / 2;
    for (size_t i = 0; i < src.size(); i++) {
        if (i & 1u) {
            t[half + i / 2] = src[i];
        } else {
            t[i / 2] = src[i];
        }
    }
    for (size_t i = t.size(); i-- > 1;) {
        t[i] = (uint8_t)(t[i] - t[i - 1] + 128);
    }
    return t;
}

template <typename T>
void put(std::vector<uint8_t>& b, T v) {
    const size_t o = b.size();
    b.resize(o + sizeof(T));
    std::memcpy(b.data() + o, &v, sizeof(T));
}

void put_attr(std::vector<uint8_t>& b, const std::string& name, const std::string& type,
              const std::vector<uint8_t>& value) {
    b.insert(b.end(), name.begin(), name.end());
    b.push_back(0);
    b.insert(b.end(), type.begin(), type.end());
    b.push_back(0);
    put<int32_t>(b, (int32_t)value.size());
    b.insert(b.end(), value.begin(), value.end());
}

// ---- PNG ----------------------------------------------------------------------------------

uint32_t be32(const uint8_t* p) {
    return (uint32_t)p[0] << 24 | (uint32_t)p[1] << 16 | (uint32_t)p[2] << 8 | p[3];
}

void put_be32(std::vector<uint8_t>& b, uint32_t v) {
    b.push_back((uint8_t)(v >> 24));
    b.push_back((uint8_t)(v >> 16));
    b.push_back((uint8_t)(v >> 8));
    b.push_back((uint8_t)v);
}

void put_chunk(std::vector<uint8_t>& b, const char* type, const std::vector<uint8_t>& data) {
    put_be32(b, (uint32_t)data.size());
    const size_t start = b.size();
    b.insert(b.end(), type, type + 4);
    b.insert(b.end(), data.begin(), data.end());
    const uint32_t crc = (uint32_t)crc32(0L, b.data() + start, (uInt)(b.size() - start));
    put_be32(b, crc);
}

uint8_t paeth(int a, int b, int c) {
    const int p = a + b - c;
    const int pa = std::abs(p - a), pb = std::abs(p - b), pc = std::abs(p - c);
    if (pa <= pb && pa <= pc) return (uint8_t)a;
    if (pb <= pc) return (uint8_t)b;
    return (uint8_t)c;
}

}  // namespace

// ---- meshes -------------------------------------------------------------------------

Mesh LoadObjMesh(const std::string& path) {
    std::ifstream f(path);
    if (!f) {
        fail("Failed to load OBJ: " + path + " cannot open");
    }
    std::vector<float> v_pos, v_tex;
    // faces as (position index, texcoord index or -1) corners, triangulated
    std::vector<std::pair<int, int>> corners;
    std::string line;
    size_t line_no = 0;
    auto bad = [&](const char* what) {
        fail("Failed to load OBJ: " + path + " " + what + " at line " + std::to_string(line_no));
    };
    auto resolve = [&](long i, size_t n) -> int {
        // 1-based, or negative: relative to the records read so far
        const long r = i > 0 ? i - 1 : (long)n + i;
        if (i == 0 || r < 0 || r >= (long)n) {
            bad("bad index");
        }
        return (int)r;
    };
    // a number is read in double precision and stored as float, as the
    // reference's parser (tinyobjloader) stores its reals
    auto real = [](std::istringstream& ss) -> float {
        std::string t;
        if (!(ss >> t)) {
            return 0.f;
        }
        return (float)std::strtod(t.c_str(), nullptr);
    };
    auto index = [&](const std::string& t) -> long {
        char* end = nullptr;
        const long v = std::strtol(t.c_str(), &end, 10);
        if (t.empty() || *end != '\0') {
            bad("bad face index");
        }
        return v;
    };
    while (std::getline(f, line)) {
        line_no++;
        std::istringstream ss(line);
        std::string tag;
        if (!(ss >> tag) || tag[0] == '#') {
            continue;
        }
        if (tag == "v") {
            const float x = real(ss), y = real(ss), z = real(ss);
            v_pos.insert(v_pos.end(), {x, y, z});
        } else if (tag == "vt") {
            const float u = real(ss), w = real(ss);
            v_tex.insert(v_tex.end(), {u, w});
        } else if (tag == "f") {
            std::vector<std::pair<int, int>> poly;
            std::string tok;
            while (ss >> tok) {
                const size_t s1 = tok.find('/');
                const int pi = resolve(index(tok.substr(0, s1)), v_pos.size() / 3);
                int ti = -1;
                if (s1 != std::string::npos) {
                    const size_t s2 = tok.find('/', s1 + 1);
                    const std::string t = tok.substr(s1 + 1, s2 == std::string::npos
                                                                     ? std::string::npos
                                                                     : s2 - s1 - 1);
                    if (!t.empty()) {
                        ti = resolve(index(t), v_tex.size() / 2);
                    }
                }
                poly.emplace_back(pi, ti);
            }
            auto tri = [&](size_t a, size_t b, size_t c) {
                corners.push_back(poly[a]);
                corners.push_back(poly[b]);
                corners.push_back(poly[c]);
            };
            if (poly.size() == 4) {
                // a quad splits along its shorter diagonal (0-2 when strictly
                // shorter, else 1-3), squared lengths in float: the rule of
                // tinyobjloader v2.0.0rc13's triangulation
                auto d2 = [&](size_t a, size_t b) {
                    float acc = 0.f;
                    for (int c = 0; c < 3; c++) {
                        const float e = v_pos[(size_t)poly[b].first * 3 + c] -
                                        v_pos[(size_t)poly[a].first * 3 + c];
                        acc = acc + e * e;
                    }
                    return acc;
                };
                if (d2(0, 2) < d2(1, 3)) {
                    tri(0, 1, 2);
                    tri(0, 2, 3);
                } else {
                    tri(0, 1, 3);
                    tri(1, 2, 3);
                }
            } else {
                for (size_t k = 2; k < poly.size(); k++) {  // fan
                    tri(0, k - 1, k);
                }
            }
        }
    }
    // unweld: one vertex per unique (position, texcoord) pair
    std::map<std::pair<int, int>, uint32_t> unique;
    std::vector<float> pos, uv;
    std::vector<uint32_t> idx;
    for (const auto& key : corners) {
        auto it = unique.find(key);
        if (it == unique.end()) {
            it = unique.emplace(key, (uint32_t)(pos.size() / 3)).first;
            for (int c = 0; c < 3; c++) {
                pos.push_back(v_pos[(size_t)key.first * 3 + c]);
            }
            if (key.second >= 0) {
                uv.push_back(v_tex[(size_t)key.second * 2]);
                uv.push_back(1.f - v_tex[(size_t)key.second * 2 + 1]);  // origin bottom-left
            } else {
                uv.push_back(0.f);
                uv.push_back(0.f);
            }
        }
        idx.push_back(it->second);
    }
    if (idx.empty()) {
        fail("OBJ has no triangles: " + path);
    }
    // centre on the origin, maximum extent 1 (asset_utils.cpp:563-579)
    float lo[3] = {1e30f, 1e30f, 1e30f}, hi[3] = {-1e30f, -1e30f, -1e30f};
    for (size_t i = 0; i < pos.size(); i += 3) {
        for (int c = 0; c < 3; c++) {
            lo[c] = std::min(lo[c], pos[i + c]);
            hi[c] = std::max(hi[c], pos[i + c]);
        }
    }
    const float ext = std::max({hi[0] - lo[0], hi[1] - lo[1], hi[2] - lo[2]});
    const float scale = 1.f / ext;
    for (size_t i = 0; i < pos.size(); i += 3) {
        for (int c = 0; c < 3; c++) {
            pos[i + c] = (pos[i + c] - 0.5f * (lo[c] + hi[c])) * scale;
        }
    }
    Mesh m;
    const uint32_t nv = (uint32_t)(pos.size() / 3), nf = (uint32_t)(idx.size() / 3);
    m.pos = CpuImage(nv, 1, 3);
    m.pos.data = std::move(pos);
    m.uv = CpuImage(nv, 1, 2);
    m.uv.data = std::move(uv);
    m.faces = CpuImage(nf, 1, 3);
    for (size_t i = 0; i < idx.size(); i++) {
        m.faces.data[i] = (float)idx[i];
    }
    return m;
}

Mesh LoadGltfMesh(const std::string& path) {
    Gltf g;
    try {
        g = load_gltf(path);
    } catch (const std::runtime_error& e) {
        fail("Failed to load glTF: " + path + " " + e.what());
    }
    const Json* meshes = g.doc.get("meshes");
    if (!meshes || meshes->arr.empty() || !meshes->arr[0].get("primitives") ||
        meshes->arr[0].at("primitives").arr.empty()) {
        fail("glTF has no mesh primitives: " + path);
    }
    const Json& prim = meshes->arr[0].at("primitives").at(0);
    const Json* attrs = prim.get("attributes");
    const Json* pos_i = attrs ? attrs->get("POSITION") : nullptr;
    const Json* idx_i = prim.get("indices");
    if (!pos_i || !idx_i) {
        fail("glTF primitive needs POSITION + indices");
    }
    const Accessor pa = accessor(g, (size_t)pos_i->number(0.0));
    const Accessor ia = accessor(g, (size_t)idx_i->number(0.0));
    const uint32_t nv = (uint32_t)pa.count, nf = (uint32_t)(ia.count / 3);
    Mesh m;
    m.pos = CpuImage(nv, 1, 3);
    m.uv = CpuImage(nv, 1, 2, 0.f);
    m.faces = CpuImage(nf, 1, 3);
    for (uint32_t v = 0; v < nv; v++) {
        for (uint32_t c = 0; c < 3; c++) {
            m.pos.at(v, 0, c) = pa.read(v, c);
        }
    }
    if (const Json* uv_i = attrs->get("TEXCOORD_0")) {
        const Accessor ua = accessor(g, (size_t)uv_i->number(0.0));
        for (uint32_t v = 0; v < nv; v++) {
            m.uv.at(v, 0, 0) = ua.read(v, 0);
            m.uv.at(v, 0, 1) = 1.f - ua.read(v, 1);
        }
    }
    for (uint32_t fi = 0; fi < nf; fi++) {
        for (uint32_t k = 0; k < 3; k++) {
            m.faces.at(fi, 0, k) = ia.read((size_t)fi * 3 + k, 0);
        }
    }
    normalise_divide(m);
    return m;
}

namespace {

// Column-major node-local matrix: `matrix`, else T * R * S from
// translation, rotation (unit quaternion x, y, z, w) and scale
// (asset_utils.cpp:177-213).
Mat4 node_local_matrix(const Json& node) {
    Mat4 m{};
    if (const Json* mat = node.get("matrix")) {
        if (mat->arr.size() == 16) {
            for (size_t i = 0; i < 16; i++) {
                m[i] = (float)mat->arr[i].number(0.0);
            }
            return m;
        }
    }
    m[0] = m[5] = m[10] = m[15] = 1.f;
    if (const Json* r = node.get("rotation")) {
        if (r->arr.size() == 4) {
            const float x = (float)r->arr[0].number(0.0), y = (float)r->arr[1].number(0.0);
            const float z = (float)r->arr[2].number(0.0), w = (float)r->arr[3].number(0.0);
            m[0] = 1.f - 2.f * (y * y + z * z);
            m[1] = 2.f * (x * y + z * w);
            m[2] = 2.f * (x * z - y * w);
            m[4] = 2.f * (x * y - z * w);
            m[5] = 1.f - 2.f * (x * x + z * z);
            m[6] = 2.f * (y * z + x * w);
            m[8] = 2.f * (x * z + y * w);
            m[9] = 2.f * (y * z - x * w);
            m[10] = 1.f - 2.f * (x * x + y * y);
        }
    }
    if (const Json* sc = node.get("scale")) {
        if (sc->arr.size() == 3) {
            for (int col = 0; col < 3; col++) {
                const float k = (float)sc->arr[(size_t)col].number(1.0);
                for (int row = 0; row < 3; row++) {
                    m[(size_t)(col * 4 + row)] *= k;
                }
            }
        }
    }
    if (const Json* t = node.get("translation")) {
        if (t->arr.size() == 3) {
            m[12] = (float)t->arr[0].number(0.0);
            m[13] = (float)t->arr[1].number(0.0);
            m[14] = (float)t->arr[2].number(0.0);
        }
    }
    return m;
}

// Inverse transpose of the upper-left 3x3 of m (the normal matrix),
// column-major, by cofactors; a zero determinant divides by 1e-12
// (asset_utils.cpp:215-231).
std::array<float, 9> normal_matrix(const Mat4& m) {
    const float a = m[0], b = m[4], c = m[8];
    const float d = m[1], e = m[5], f = m[9];
    const float g = m[2], h = m[6], i = m[10];
    const float det = a * (e * i - f * h) - b * (d * i - f * g) + c * (d * h - e * g);
    const float inv = 1.f / (det == 0.f ? 1e-12f : det);
    return {(e * i - f * h) * inv, (c * h - b * i) * inv, (b * f - c * e) * inv,
            (f * g - d * i) * inv, (a * i - c * g) * inv, (c * d - a * f) * inv,
            (d * h - e * g) * inv, (b * g - a * h) * inv, (a * e - b * d) * inv};
}

std::array<float, 3> cross3(const std::array<float, 3>& a, const std::array<float, 3>& b) {
    return {a[1] * b[2] - a[2] * b[1], a[2] * b[0] - a[0] * b[2], a[0] * b[1] - a[1] * b[0]};
}

float dot3(const std::array<float, 3>& a, const std::array<float, 3>& b) {
    return a[0] * b[0] + a[1] * b[1] + a[2] * b[2];
}

std::array<float, 3> unit3(const std::array<float, 3>& v) {
    const float len = std::sqrt(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
    return {v[0] / len, v[1] / len, v[2] / len};
}

// The bytes of glTF image `i`: a file next to the asset, a base64 data
// URI, or a bufferView.
std::vector<uint8_t> gltf_image_bytes(const Gltf& g, size_t i, const std::string& path) {
    const Json& im = g.doc.at("images").at(i);
    if (const Json* uri = im.get("uri")) {
        if (uri->str.rfind("data:", 0) == 0) {
            const size_t comma = uri->str.find(',');
            if (comma == std::string::npos ||
                uri->str.substr(0, comma).find(";base64") == std::string::npos) {
                fail("glTF: unsupported image data uri in " + path);
            }
            return base64_decode(uri->str.substr(comma + 1));
        }
        return read_file(dir_of(path) + uri_decode(uri->str));
    }
    const Json& bv = g.doc.at("bufferViews").at((size_t)im.at("bufferView").number(0.0));
    const size_t buf = (size_t)bv.at("buffer").number(0.0);
    const size_t off = bv.get("byteOffset") ? (size_t)bv.get("byteOffset")->number(0.0) : 0;
    const size_t len = (size_t)bv.at("byteLength").number(0.0);
    if (buf >= g.buffers.size() || off + len > g.buffers[buf].size()) {
        fail("glTF: image bufferView out of range in " + path);
    }
    return std::vector<uint8_t>(g.buffers[buf].begin() + (ptrdiff_t)off,
                                g.buffers[buf].begin() + (ptrdiff_t)(off + len));
}

// Texture `tex` decoded to 3 channels in [0, 1]: channel c reads the
// image's component min(c, components - 1) (asset_utils.cpp:233-260);
// empty when the slot or its source is absent; 16-bit images are refused.
CpuImage gltf_texture(const Gltf& g, int tex, const std::string& path) {
    if (tex < 0) {
        return CpuImage();
    }
    const Json& t = g.doc.at("textures").at((size_t)tex);
    const Json* src = t.get("source");
    if (!src || src->number(-1.0) < 0.0) {
        return CpuImage();
    }
    const size_t idx = (size_t)src->number(0.0);
    const std::vector<uint8_t> bytes = gltf_image_bytes(g, idx, path);
    const codec::Image8 d =
            codec::DecodeImage(bytes.data(), bytes.size(), path + " image " + std::to_string(idx));
    if (d.bits != 8) {
        fail("glTF: only 8-bit textures supported");
    }
    CpuImage out(d.width, d.height, 3);
    const size_t np = (size_t)d.width * d.height;
    for (size_t p = 0; p < np; p++) {
        for (uint32_t c = 0; c < 3; c++) {
            out.data[p * 3 + c] = (float)d.px[p * d.comp + std::min(c, d.comp - 1)] / 255.f;
        }
    }
    return out;
}

int texture_index(const Json* slot) {
    if (!slot) {
        return -1;
    }
    const Json* i = slot->get("index");
    return i ? (int)i->number(-1.0) : -1;
}

}  // namespace

GltfScene LoadGltfScene(const std::string& path, bool normalize) {
    Gltf g;
    try {
        g = load_gltf(path);
    } catch (const std::runtime_error& e) {
        fail("Failed to load glTF: " + path + " " + e.what());
    }
    // the first node with a mesh (its own transform; parents are not
    // composed), else mesh 0 untransformed (asset_utils.cpp:280-294)
    int mesh_idx = -1;
    Mat4 xform{};
    xform[0] = xform[5] = xform[10] = xform[15] = 1.f;
    if (const Json* nodes = g.doc.get("nodes")) {
        for (const Json& node : nodes->arr) {
            const Json* mi = node.get("mesh");
            if (mi && mi->number(-1.0) >= 0.0) {
                mesh_idx = (int)mi->number(0.0);
                xform = node_local_matrix(node);
                break;
            }
        }
    }
    const Json* meshes = g.doc.get("meshes");
    if (mesh_idx < 0 && meshes && !meshes->arr.empty()) {
        mesh_idx = 0;
    }
    if (mesh_idx < 0 || !meshes || (size_t)mesh_idx >= meshes->arr.size() ||
        !meshes->arr[(size_t)mesh_idx].get("primitives") ||
        meshes->arr[(size_t)mesh_idx].at("primitives").arr.empty()) {
        fail("glTF has no mesh primitives: " + path);
    }
    const Json& prim = meshes->arr[(size_t)mesh_idx].at("primitives").at(0);
    const Json* attrs = prim.get("attributes");
    const Json* pos_i = attrs ? attrs->get("POSITION") : nullptr;
    const Json* idx_i = prim.get("indices");
    if (!pos_i || !idx_i) {
        fail("glTF primitive needs POSITION + indices");
    }
    const Accessor pa = accessor(g, (size_t)pos_i->number(0.0));
    const Accessor ia = accessor(g, (size_t)idx_i->number(0.0));
    const uint32_t nv = (uint32_t)pa.count, nf = (uint32_t)(ia.count / 3);
    GltfScene sc;
    Mesh& m = sc.mesh;
    m.pos = CpuImage(nv, 1, 3);
    m.uv = CpuImage(nv, 1, 2, 0.f);
    m.faces = CpuImage(nf, 1, 3);
    sc.normal = CpuImage(nv, 1, 3, 0.f);
    sc.tangent = CpuImage(nv, 1, 4, 0.f);
    for (uint32_t v = 0; v < nv; v++) {
        for (uint32_t c = 0; c < 3; c++) {
            m.pos.at(v, 0, c) = pa.read(v, c);
        }
    }
    if (const Json* uv_i = attrs->get("TEXCOORD_0")) {
        const Accessor ua = accessor(g, (size_t)uv_i->number(0.0));
        for (uint32_t v = 0; v < nv; v++) {
            m.uv.at(v, 0, 0) = ua.read(v, 0);  // glTF's V: no flip
            m.uv.at(v, 0, 1) = ua.read(v, 1);
        }
        // whole-period offsets (REPEAT-wrapped coordinates) removed per axis
        for (uint32_t c = 0; c < 2; c++) {
            float lo = 1e30f;
            for (uint32_t v = 0; v < nv; v++) {
                lo = std::min(lo, m.uv.at(v, 0, c));
            }
            const float shift = std::floor(lo);
            if (shift != 0.f) {
                for (uint32_t v = 0; v < nv; v++) {
                    m.uv.at(v, 0, c) -= shift;
                }
            }
        }
    }
    for (uint32_t fi = 0; fi < nf; fi++) {
        for (uint32_t k = 0; k < 3; k++) {
            m.faces.at(fi, 0, k) = ia.read((size_t)fi * 3 + k, 0);
        }
    }
    auto corner = [&](uint32_t fi, uint32_t k) {
        const float x = m.faces.at(fi, 0, k);
        if (!(x >= 0.f) || x >= (float)nv) {
            fail("glTF: face index out of range in " + path);
        }
        return (uint32_t)x;
    };
    if (const Json* n_i = attrs->get("NORMAL")) {
        const Accessor na = accessor(g, (size_t)n_i->number(0.0));
        for (uint32_t v = 0; v < nv; v++) {
            for (uint32_t c = 0; c < 3; c++) {
                sc.normal.at(v, 0, c) = na.read(v, c);
            }
        }
    } else {
        // area-weighted: each face's (p1 - p0) x (p2 - p0) added to its corners
        for (uint32_t fi = 0; fi < nf; fi++) {
            uint32_t vi[3];
            std::array<float, 3> p[3];
            for (uint32_t k = 0; k < 3; k++) {
                vi[k] = corner(fi, k);
                for (uint32_t c = 0; c < 3; c++) {
                    p[k][c] = m.pos.at(vi[k], 0, c);
                }
            }
            const std::array<float, 3> e1 = {p[1][0] - p[0][0], p[1][1] - p[0][1], p[1][2] - p[0][2]};
            const std::array<float, 3> e2 = {p[2][0] - p[0][0], p[2][1] - p[0][1], p[2][2] - p[0][2]};
            const std::array<float, 3> fn = cross3(e1, e2);
            for (uint32_t k = 0; k < 3; k++) {
                for (uint32_t c = 0; c < 3; c++) {
                    sc.normal.at(vi[k], 0, c) += fn[c];
                }
            }
        }
    }
    if (const Json* t_i = attrs->get("TANGENT")) {
        const Accessor ta = accessor(g, (size_t)t_i->number(0.0));
        for (uint32_t v = 0; v < nv; v++) {
            for (uint32_t c = 0; c < 4; c++) {
                sc.tangent.at(v, 0, c) = ta.read(v, c);
            }
        }
    } else {
        // Lengyel's per-face tangent / bitangent from the uv gradients,
        // summed per vertex, Gram-Schmidt against the normal, w the
        // handedness (asset_utils.cpp:401-463)
        std::vector<float> tan((size_t)nv * 3, 0.f), bit((size_t)nv * 3, 0.f);
        for (uint32_t fi = 0; fi < nf; fi++) {
            uint32_t vi[3];
            std::array<float, 3> p[3];
            float tu[3], tv[3];
            for (uint32_t k = 0; k < 3; k++) {
                vi[k] = corner(fi, k);
                for (uint32_t c = 0; c < 3; c++) {
                    p[k][c] = m.pos.at(vi[k], 0, c);
                }
                tu[k] = m.uv.at(vi[k], 0, 0);
                tv[k] = m.uv.at(vi[k], 0, 1);
            }
            const float du1 = tu[1] - tu[0], dv1 = tv[1] - tv[0];
            const float du2 = tu[2] - tu[0], dv2 = tv[2] - tv[0];
            const float det = du1 * dv2 - du2 * dv1;
            if (std::fabs(det) < 1e-12f) {
                continue;
            }
            const float r = 1.f / det;
            for (uint32_t c = 0; c < 3; c++) {
                const float e1 = p[1][c] - p[0][c];
                const float e2 = p[2][c] - p[0][c];
                const float tc = (e1 * dv2 - e2 * dv1) * r;
                const float bc = (e2 * du1 - e1 * du2) * r;
                for (uint32_t k = 0; k < 3; k++) {
                    tan[(size_t)vi[k] * 3 + c] += tc;
                    bit[(size_t)vi[k] * 3 + c] += bc;
                }
            }
        }
        for (uint32_t v = 0; v < nv; v++) {
            const std::array<float, 3> n = {sc.normal.at(v, 0, 0), sc.normal.at(v, 0, 1),
                                            sc.normal.at(v, 0, 2)};
            std::array<float, 3> t = {tan[(size_t)v * 3], tan[(size_t)v * 3 + 1],
                                      tan[(size_t)v * 3 + 2]};
            const float ndt = dot3(n, t);
            for (uint32_t c = 0; c < 3; c++) {
                t[c] -= n[c] * ndt;
            }
            const float len = std::sqrt(dot3(t, t));
            if (len < 1e-12f) {
                // degenerate uv: a unit vector perpendicular to n
                t = std::fabs(n[0]) < 0.9f ? unit3(cross3(n, {1.f, 0.f, 0.f}))
                                           : unit3(cross3(n, {0.f, 1.f, 0.f}));
            } else {
                for (uint32_t c = 0; c < 3; c++) {
                    t[c] /= len;
                }
            }
            const std::array<float, 3> b = {bit[(size_t)v * 3], bit[(size_t)v * 3 + 1],
                                            bit[(size_t)v * 3 + 2]};
            for (uint32_t c = 0; c < 3; c++) {
                sc.tangent.at(v, 0, c) = t[c];
            }
            sc.tangent.at(v, 0, 3) = dot3(cross3(n, t), b) < 0.f ? -1.f : 1.f;
        }
    }
    // the node transform: positions by M, normals by its normal matrix,
    // tangent xyz by M as a direction; normals and tangents renormalised
    const std::array<float, 9> nm = normal_matrix(xform);
    for (uint32_t v = 0; v < nv; v++) {
        const float p[3] = {m.pos.at(v, 0, 0), m.pos.at(v, 0, 1), m.pos.at(v, 0, 2)};
        const float n[3] = {sc.normal.at(v, 0, 0), sc.normal.at(v, 0, 1), sc.normal.at(v, 0, 2)};
        const float t[3] = {sc.tangent.at(v, 0, 0), sc.tangent.at(v, 0, 1), sc.tangent.at(v, 0, 2)};
        std::array<float, 3> np{}, nn{}, nt{};
        for (uint32_t r = 0; r < 3; r++) {
            np[r] = xform[0 * 4 + r] * p[0] + xform[1 * 4 + r] * p[1] + xform[2 * 4 + r] * p[2] +
                    xform[3 * 4 + r];
            nn[r] = nm[0 * 3 + r] * n[0] + nm[1 * 3 + r] * n[1] + nm[2 * 3 + r] * n[2];
            nt[r] = xform[0 * 4 + r] * t[0] + xform[1 * 4 + r] * t[1] + xform[2 * 4 + r] * t[2];
        }
        nn = unit3(nn);
        nt = unit3(nt);
        for (uint32_t c = 0; c < 3; c++) {
            m.pos.at(v, 0, c) = np[c];
            sc.normal.at(v, 0, c) = nn[c];
            sc.tangent.at(v, 0, c) = nt[c];
        }
    }
    if (normalize) {
        normalise_divide(m);
    }
    if (const Json* mi = prim.get("material")) {
        const Json& mat = g.doc.at("materials").at((size_t)mi->number(0.0));
        const Json* pbr = mat.get("pbrMetallicRoughness");
        sc.base_color = gltf_texture(g, texture_index(pbr ? pbr->get("baseColorTexture") : nullptr),
                                     path);
        sc.metallic_roughness = gltf_texture(
                g, texture_index(pbr ? pbr->get("metallicRoughnessTexture") : nullptr), path);
        sc.normal_map = gltf_texture(g, texture_index(mat.get("normalTexture")), path);
        sc.occlusion = gltf_texture(g, texture_index(mat.get("occlusionTexture")), path);
        sc.emissive = gltf_texture(g, texture_index(mat.get("emissiveTexture")), path);
    }
    return sc;
}

// ---- images -----------------------------------------------------------------------------

codec::Image8 codec::DecodePng(const uint8_t* fdata, size_t fsize, const std::string& path) {
    static const uint8_t sig[8] = {137, 80, 78, 71, 13, 10, 26, 10};
    if (fsize < 8 || std::memcmp(fdata, sig, 8) != 0) {
        fail("Failed to load image: " + path + " (not a PNG)");
    }
    const std::vector<uint8_t> f(fdata, fdata + fsize);
    uint32_t w = 0, h = 0;
    int depth = 0, color = -1, interlace = 0;
    std::vector<uint8_t> idat, palette;
    size_t off = 8;
    while (off + 12 <= f.size()) {
        const uint32_t len = be32(&f[off]);
        if (off + 12 + (size_t)len > f.size()) {
            fail("Failed to load image: " + path + " truncated chunk");
        }
        const std::string type((const char*)&f[off + 4], 4);
        const uint8_t* d = &f[off + 8];
        if (type == "IHDR" && len >= 13) {
            w = be32(d);
            h = be32(d + 4);
            depth = d[8];
            color = d[9];
            interlace = d[12];
        } else if (type == "PLTE") {
            palette.assign(d, d + len);
        } else if (type == "IDAT") {
            idat.insert(idat.end(), d, d + len);
        } else if (type == "IEND") {
            break;
        }
        off += 12 + (size_t)len;
    }
    const int chans = color == 0 ? 1 : color == 2 ? 3 : color == 3 ? 1 : color == 4 ? 2
                      : color == 6 ? 4 : 0;
    const bool depth_ok = (color == 0 && (depth == 1 || depth == 2 || depth == 4 || depth == 8 ||
                                          depth == 16)) ||
                          (color == 3 && (depth == 1 || depth == 2 || depth == 4 || depth == 8)) ||
                          ((color == 2 || color == 4 || color == 6) && (depth == 8 || depth == 16));
    if (!w || !h || w > (1u << 24) || h > (1u << 24) || !chans || !depth_ok || interlace > 1 ||
        (color == 3 && palette.size() < 3)) {
        fail("Failed to load image: " + path + " (unsupported PNG layout)");
    }
    const size_t bits = (size_t)chans * (size_t)depth;  // per pixel
    const size_t bpp = std::max<size_t>(1, bits / 8);    // filter distance
    const std::vector<uint8_t> raw = inflate_stream(idat);
    size_t pos = 0;
    // native components: gray, gray + alpha, RGB (also palette), RGBA
    const uint32_t out_c = color == 3 ? 3u : (uint32_t)chans;
    codec::Image8 img;
    img.width = w;
    img.height = h;
    img.comp = out_c;
    img.bits = (uint32_t)depth;
    img.px.assign((size_t)w * h * out_c, 0);
    // one (sub-)image: rows filtered and packed at `bits` per pixel;
    // pixel (i, j) lands on (x0 + i dx, y0 + j dy)
    auto decode = [&](uint32_t x0, uint32_t y0, uint32_t dx, uint32_t dy) {
        const uint32_t pw = w > x0 ? (w - x0 + dx - 1) / dx : 0;
        const uint32_t ph = h > y0 ? (h - y0 + dy - 1) / dy : 0;
        if (!pw || !ph) {
            return;
        }
        const size_t row = ((size_t)pw * bits + 7) / 8;
        if (raw.size() < pos + (row + 1) * ph) {
            fail("Failed to load image: " + path + " short image data");
        }
        std::vector<uint8_t> cur(row), prev(row, 0);
        for (uint32_t j = 0; j < ph; j++) {
            const uint8_t filter = raw[pos];
            const uint8_t* in = &raw[pos + 1];
            pos += row + 1;
            for (size_t i = 0; i < row; i++) {
                const int a = i >= bpp ? cur[i - bpp] : 0;
                const int b = prev[i];
                const int c = i >= bpp ? prev[i - bpp] : 0;
                int v = in[i];
                switch (filter) {
                    case 0: break;
                    case 1: v += a; break;
                    case 2: v += b; break;
                    case 3: v += (a + b) / 2; break;
                    case 4: v += paeth(a, b, c); break;
                    default: fail("Failed to load image: " + path + " bad PNG filter");
                }
                cur[i] = (uint8_t)v;
            }
            for (uint32_t i = 0; i < pw; i++) {
                // 8-bit samples; 16-bit ones keep their high byte, gray
                // below 8 bits scales to the full range (x 255 / (2^d - 1))
                auto sample = [&](int ch) -> uint32_t {
                    if (depth >= 8) {
                        return cur[((size_t)i * chans + (size_t)ch) * (size_t)(depth / 8)];
                    }
                    const size_t bit = (size_t)i * (size_t)depth;
                    return (uint32_t)(cur[bit >> 3] >> (8 - depth - (int)(bit & 7))) &
                           ((1u << depth) - 1u);
                };
                uint8_t* o = &img.px[((size_t)(y0 + j * dy) * w + (x0 + i * dx)) * out_c];
                if (color == 3) {
                    const size_t e = (size_t)sample(0) * 3;
                    if (e + 2 >= palette.size()) {
                        fail("Failed to load image: " + path + " palette index out of range");
                    }
                    o[0] = palette[e];
                    o[1] = palette[e + 1];
                    o[2] = palette[e + 2];
                } else {
                    const uint32_t scale = depth == 1 ? 0xffu : depth == 2 ? 0x55u
                                           : depth == 4 ? 0x11u : 1u;
                    for (int c = 0; c < chans; c++) {
                        o[c] = (uint8_t)(sample(c) * (depth < 8 ? scale : 1u));
                    }
                }
            }
            std::swap(cur, prev);
        }
    };
    if (interlace == 0) {
        decode(0, 0, 1, 1);
    } else {  // Adam7
        static const uint32_t pass[7][4] = {{0, 0, 8, 8}, {4, 0, 8, 8}, {0, 4, 4, 8}, {2, 0, 4, 4},
                                            {0, 2, 2, 4}, {1, 0, 2, 2}, {0, 1, 1, 2}};
        for (const auto& q : pass) {
            decode(q[0], q[1], q[2], q[3]);
        }
    }
    return img;
}


// stb_image's 8-bit load with 3 components asked for (what the reference
// calls, asset_utils.cpp:598-609): gray and gray + alpha replicate the gray
// sample, RGBA drops alpha; 16-bit PNG samples keep their high byte.
CpuImage LoadImageRgb(const std::string& path) {
    const std::vector<uint8_t> f = read_file(path);
    const codec::Image8 d = codec::DecodeImage(f.data(), f.size(), path);
    CpuImage img(d.width, d.height, 3);
    const size_t np = (size_t)d.width * d.height;
    for (size_t p = 0; p < np; p++) {
        for (uint32_t c = 0; c < 3; c++) {
            const uint32_t src = d.comp <= 2 ? 0u : c;
            img.data[p * 3 + c] = (float)d.px[p * d.comp + src] / 255.f;
        }
    }
    return img;
}

void SaveImagePng(const std::string& path, const CpuImage& img) {
    if (!(img.channels == 1 || img.channels >= 3) || !img.width || !img.height) {
        fail("Failed to save image: " + path + " (1-channel or >= 3-channel image expected)");
    }
    std::vector<uint8_t> raw;
    raw.reserve(((size_t)img.width * 3 + 1) * img.height);
    for (uint32_t y = 0; y < img.height; y++) {
        raw.push_back(0);  // filter: none
        for (uint32_t x = 0; x < img.width; x++) {
            for (uint32_t c = 0; c < 3; c++) {
                const float v = img.at(x, y, img.channels == 1 ? 0 : c);
                raw.push_back((uint8_t)(std::clamp(v, 0.f, 1.f) * 255.f + 0.5f));
            }
        }
    }
    std::vector<uint8_t> out = {137, 80, 78, 71, 13, 10, 26, 10};
    std::vector<uint8_t> ihdr;
    put_be32(ihdr, img.width);
    put_be32(ihdr, img.height);
    ihdr.insert(ihdr.end(), {8, 2, 0, 0, 0});  // 8-bit RGB, deflate, no interlace
    put_chunk(out, "IHDR", ihdr);
    put_chunk(out, "IDAT", deflate_all(raw.data(), raw.size()));
    put_chunk(out, "IEND", {});
    write_file(path, out, "Failed to save image: ");
}

CpuImage LoadImageExr(const std::string& path) {
    const std::vector<uint8_t> f = read_file(path);
    if (f.size() < 8 || be32(f.data()) != 0x762f3101u) {
        fail("Failed to load EXR: " + path + " not an OpenEXR file");
    }
    uint32_t version;
    std::memcpy(&version, f.data() + 4, 4);
    if ((version & 0xffu) != 2u || (version & 0x1e00u) != 0u) {
        fail("Failed to load EXR: " + path + " only single-part scanline files are read");
    }
    size_t off = 8;
    std::vector<ExrChannel> chans;
    int compression = -1;
    int32_t dw[4] = {0, 0, -1, -1};
    auto cstr = [&](size_t& o) {
        const size_t s = o;
        while (o < f.size() && f[o]) {
            o++;
        }
        if (o >= f.size()) {
            fail("Failed to load EXR: " + path + " truncated header");
        }
        return std::string((const char*)&f[s], o++ - s);
    };
    while (true) {
        const std::string name = cstr(off);
        if (name.empty()) {
            break;
        }
        const std::string type = cstr(off);
        if (off + 4 > f.size()) {
            fail("Failed to load EXR: " + path + " truncated header");
        }
        int32_t size;
        std::memcpy(&size, &f[off], 4);
        off += 4;
        if (size < 0 || off + (size_t)size > f.size()) {
            fail("Failed to load EXR: " + path + " truncated header");
        }
        const uint8_t* v = &f[off];
        if (name == "channels" && type == "chlist") {
            size_t o = off;
            while (o < off + (size_t)size && f[o]) {
                ExrChannel ch;
                ch.name = cstr(o);
                if (o + 16 > off + (size_t)size) {
                    fail("Failed to load EXR: " + path + " bad channel list");
                }
                std::memcpy(&ch.type, &f[o], 4);
                std::memcpy(&ch.xs, &f[o + 8], 4);
                std::memcpy(&ch.ys, &f[o + 12], 4);
                o += 16;
                chans.push_back(ch);
            }
        } else if (name == "compression") {
            compression = v[0];
        } else if (name == "dataWindow" && size == 16) {
            std::memcpy(dw, v, 16);
        }
        off += (size_t)size;
    }
    const int64_t w = (int64_t)dw[2] - dw[0] + 1, h = (int64_t)dw[3] - dw[1] + 1;
    if (w <= 0 || h <= 0 || w > (1 << 20) || h > (1 << 20) || chans.empty()) {
        fail("Failed to load EXR: " + path + " bad data window or no channels");
    }
    if (!(compression >= 0 && compression <= 3)) {
        fail("Failed to load EXR: " + path + " compression " + std::to_string(compression) +
             " is not supported (NONE, RLE, ZIPS, ZIP)");
    }
    for (const auto& c : chans) {
        if (c.xs != 1 || c.ys != 1 || c.type < 0 || c.type > 2) {
            fail("Failed to load EXR: " + path + " subsampled or unknown channel types");
        }
    }
    // pixel data follows the header's channel order
    const uint32_t lines = compression == 3 ? 16u : 1u;
    const uint32_t n_blocks = (uint32_t)((h + lines - 1) / lines);
    if (off + (size_t)n_blocks * 8 > f.size()) {
        fail("Failed to load EXR: " + path + " truncated offset table");
    }
    size_t line_bytes = 0;
    for (const auto& c : chans) {
        line_bytes += (size_t)w * (c.type == 1 ? 2 : 4);
    }
    // Channel selection of the reference's reader (tinyexr v1.0.9 LoadEXR,
    // no layer): a file with one channel is gray, replicated; otherwise R,
    // G and B are looked up among the first four channels by the part of
    // their name after the last '.', and each must be there.
    int src[3] = {-1, -1, -1};
    if (chans.size() == 1) {
        src[0] = src[1] = src[2] = 0;
    } else {
        for (size_t i = 0; i < std::min<size_t>(chans.size(), 4); i++) {
            const size_t dot = chans[i].name.find_last_of('.');
            const std::string n = dot == std::string::npos ? chans[i].name
                                                           : chans[i].name.substr(dot + 1);
            const int k = n == "R" ? 0 : n == "G" ? 1 : n == "B" ? 2 : -1;
            if (k >= 0) {
                src[k] = (int)i;
            }
        }
        for (int k = 0; k < 3; k++) {
            if (src[k] < 0) {
                fail("Failed to load EXR: " + path + " " + "RGB"[k] + " channel not found");
            }
        }
    }
    CpuImage img((uint32_t)w, (uint32_t)h, 3);
    for (uint32_t b = 0; b < n_blocks; b++) {
        uint64_t pos;
        std::memcpy(&pos, &f[off + (size_t)b * 8], 8);
        if (pos + 8 > f.size()) {
            fail("Failed to load EXR: " + path + " bad block offset");
        }
        int32_t y0, size;
        std::memcpy(&y0, &f[pos], 4);
        std::memcpy(&size, &f[pos + 4], 4);
        if (size < 0 || pos + 8 + (uint64_t)size > f.size()) {
            fail("Failed to load EXR: " + path + " bad block size");
        }
        const int64_t first = (int64_t)y0 - dw[1];
        const uint32_t n_lines = (uint32_t)std::min<int64_t>(lines, h - first);
        if (first < 0 || first >= h) {
            fail("Failed to load EXR: " + path + " block outside the data window");
        }
        const size_t expect = line_bytes * n_lines;
        const uint8_t* data = &f[pos + 8];
        std::vector<uint8_t> block;
        if (compression == 0 || (size_t)size == expect) {
            if ((size_t)size != expect) {
                fail("Failed to load EXR: " + path + " bad block size");
            }
            block.assign(data, data + size);
        } else {
            block = exr_unzip_reorder(compression == 1 ? rle_decode(data, (size_t)size, expect)
                                                       : inflate_all(data, (size_t)size, expect));
        }
        size_t o = 0;
        for (uint32_t l = 0; l < n_lines; l++) {
            const uint32_t y = (uint32_t)first + l;
            for (size_t ci = 0; ci < chans.size(); ci++) {
                const int t = chans[ci].type;
                for (int64_t x = 0; x < w; x++) {
                    float v;
                    if (t == 1) {
                        uint16_t hv;
                        std::memcpy(&hv, &block[o], 2);
                        v = half_to_float(hv);
                        o += 2;
                    } else if (t == 2) {
                        std::memcpy(&v, &block[o], 4);
                        o += 4;
                    } else {
                        uint32_t u;
                        std::memcpy(&u, &block[o], 4);
                        v = (float)u;
                        o += 4;
                    }
                    for (int c = 0; c < 3; c++) {
                        if (src[c] == (int)ci) {
                            img.at((uint32_t)x, y, (uint32_t)c) = v;
                        }
                    }
                }
            }
        }
    }
    return img;
}

void SaveImageExr(const std::string& path, const CpuImage& img) {
    if (img.channels != 3) {
        throw std::runtime_error("SaveImageExr: expected 3 channels");
    }
    const uint32_t w = img.width, h = img.height;
    std::vector<uint8_t> out;
    put<uint32_t>(out, 20000630u);
    put<uint32_t>(out, 2u);
    std::vector<uint8_t> chl;
    for (const char* n : {"B", "G", "R"}) {  // name order
        chl.push_back((uint8_t)n[0]);
        chl.push_back(0);
        put<int32_t>(chl, 1);  // HALF
        put<uint8_t>(chl, 0);  // pLinear
        chl.insert(chl.end(), {0, 0, 0});
        put<int32_t>(chl, 1);
        put<int32_t>(chl, 1);
    }
    chl.push_back(0);
    put_attr(out, "channels", "chlist", chl);
    // ZIP (16 lines per block); images under 16 x 16 are stored
    // uncompressed, as the reference's writer does
    const bool zip = !(w < 16 && h < 16);
    put_attr(out, "compression", "compression", {(uint8_t)(zip ? 3 : 0)});
    std::vector<uint8_t> win;
    for (int32_t v : {0, 0, (int32_t)w - 1, (int32_t)h - 1}) {
        put<int32_t>(win, v);
    }
    put_attr(out, "dataWindow", "box2i", win);
    put_attr(out, "displayWindow", "box2i", win);
    put_attr(out, "lineOrder", "lineOrder", {0});
    std::vector<uint8_t> par;
    put<float>(par, 1.f);
    put_attr(out, "pixelAspectRatio", "float", par);
    std::vector<uint8_t> sc;
    put<float>(sc, 0.f);
    put<float>(sc, 0.f);
    put_attr(out, "screenWindowCenter", "v2f", sc);
    std::vector<uint8_t> sw;
    put<float>(sw, 1.f);
    put_attr(out, "screenWindowWidth", "float", sw);
    out.push_back(0);
    const uint32_t per = zip ? 16u : 1u;
    const uint32_t n_blocks = (h + per - 1) / per;
    const size_t table = out.size();
    out.resize(table + (size_t)n_blocks * 8);
    for (uint32_t b = 0; b < n_blocks; b++) {
        const uint32_t y0 = b * per, n_lines = std::min(per, h - y0);
        std::vector<uint8_t> raw;
        raw.reserve((size_t)w * 6 * n_lines);
        for (uint32_t y = y0; y < y0 + n_lines; y++) {
            for (int c : {2, 1, 0}) {
                for (uint32_t x = 0; x < w; x++) {
                    put<uint16_t>(raw, float_to_half(img.at(x, y, (uint32_t)c)));
                }
            }
        }
        std::vector<uint8_t> z;
        if (zip) {
            z = deflate_all(exr_zip_reorder(raw).data(), raw.size());
        }
        const bool keep_raw = !zip || z.size() >= raw.size();  // as is when not smaller
        const uint64_t pos = out.size();
        std::memcpy(&out[table + (size_t)b * 8], &pos, 8);
        put<int32_t>(out, (int32_t)y0);
        put<int32_t>(out, (int32_t)(keep_raw ? raw.size() : z.size()));
        const std::vector<uint8_t>& d = keep_raw ? raw : z;
        out.insert(out.end(), d.begin(), d.end());
    }
    write_file(path, out, "Failed to save EXR: ");
}

CpuImage SrgbToLinear(const CpuImage& img) {
    CpuImage out = img;
    for (float& v : out.data) {
        v = std::pow(std::max(v, 0.f), 2.2f);
    }
    return out;
}

CpuImage DownsampleHalf(const CpuImage& img) {
    const uint32_t w = std::max(1u, (img.width + 1) / 2), h = std::max(1u, (img.height + 1) / 2);
    CpuImage out(w, h, img.channels);
    for (uint32_t y = 0; y < h; y++) {
        for (uint32_t x = 0; x < w; x++) {
            for (uint32_t c = 0; c < img.channels; c++) {
                float acc = 0.f;
                for (uint32_t dy = 0; dy < 2; dy++) {
                    for (uint32_t dx = 0; dx < 2; dx++) {
                        acc += img.at(std::min(2 * x + dx, img.width - 1),
                                      std::min(2 * y + dy, img.height - 1), c);
                    }
                }
                out.at(x, y, c) = acc * 0.25f;
            }
        }
    }
    return out;
}

CpuImage TileImages(const std::vector<CpuImage>& imgs, uint32_t cols) {
    if (imgs.empty()) {
        return CpuImage();
    }
    const uint32_t w = imgs[0].width, h = imgs[0].height;
    const uint32_t rows = ((uint32_t)imgs.size() + cols - 1) / cols;
    CpuImage t(w * cols, h * rows, 3);
    for (size_t i = 0; i < imgs.size(); i++) {
        const uint32_t ox = (uint32_t)(i % cols) * w, oy = (uint32_t)(i / cols) * h;
        const bool gray = imgs[i].channels == 1;
        for (uint32_t y = 0; y < h; y++) {
            for (uint32_t x = 0; x < w; x++) {
                for (uint32_t c = 0; c < 3; c++) {
                    t.at(ox + x, oy + y, c) = imgs[i].at(x, y, gray ? 0 : c);
                }
            }
        }
    }
    return t;
}

// ---- matrices -------------------------------------------------------------------------------

// the library's C-ABI matrix routines (one implementation for both surfaces)
Mat4 Mul(const Mat4& a, const Mat4& b) {
    Mat4 r{};
    dressi_mat4_mul(a.data(), b.data(), r.data());
    return r;
}

Mat4 LookAt(const std::array<float, 3>& eye, const std::array<float, 3>& center,
            const std::array<float, 3>& up) {
    Mat4 m{};
    dressi_look_at(eye.data(), center.data(), up.data(), m.data());
    return m;
}

Mat4 PerspectiveVk(float fovy_rad, float aspect, float z_near, float z_far) {
    Mat4 m{};
    dressi_perspective_vk(fovy_rad, aspect, z_near, z_far, m.data());
    return m;
}

CpuImage TransformToClip(const CpuImage& pos, const Mat4& mvp) {
    CpuImage clip(pos.width, 1, 4);
    for (uint32_t i = 0; i < pos.width; i++) {
        const float p[4] = {pos.at(i, 0, 0), pos.at(i, 0, 1), pos.at(i, 0, 2), 1.f};
        for (int row = 0; row < 4; row++) {
            float acc = 0.f;
            for (int k = 0; k < 4; k++) {
                acc += mvp[k * 4 + row] * p[k];
            }
            clip.at(i, 0, (uint32_t)row) = acc;
        }
    }
    return clip;
}

}  // namespace dressi_examples
