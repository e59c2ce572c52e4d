/* dressi/types.h -- value types of the Dressi-AD graph API on the HIP
 * library (the reference's include/dressi/types.h:1-135, same names and
 * signatures so reference user code compiles unchanged).
 *
 * An image is W x H pixels of one VType; on the host it is a CpuImage:
 * row-major, the logical components of each pixel packed together (a VEC3
 * pixel is 3 floats). Integer-typed images (INT, IVEC3, ...) hold their
 * values as floats on the host, as in the reference. */
#ifndef DRESSI_TYPES_H
#define DRESSI_TYPES_H

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

namespace dressi {

// Element type of a Variable's image
enum VType {
    FLOAT,
    VEC2,
    VEC3,
    VEC4,
    MAT2,
    MAT3,
    MAT4,
    INT,
    IVEC2,
    IVEC3,
    IVEC4,
    UINT,
};

// Kind of pass a Function runs in (kept for source compatibility; the HIP
// executor schedules every function as a kernel of its own kind)
enum ShaderType {
    FRAG,
    COMP,
    RASTER,
};

struct ImgSize {
    uint32_t w = 1;
    uint32_t h = 1;
    bool operator==(const ImgSize& o) const { return w == o.w && h == o.h; }
    bool operator!=(const ImgSize& o) const { return !(*this == o); }
    bool isUniform() const { return w == 1 && h == 1; }
};

// 2-D layout of very long 1-D images (the reference stores an {N,1} image
// wider than a device's image-dimension limit as {W, ceil(N / W)} with W the
// largest power of two within the limit; linear element i sits at
// (i mod W, i / W)). Device buffers here are linear, so nothing is tiled;
// the helpers keep their meaning for code that computes layouts.
inline uint32_t TileWidth(uint32_t max_dim) {
    uint32_t w = 1;
    while (w <= max_dim / 2) {
        w *= 2;
    }
    return w;
}
inline bool NeedsTiling(ImgSize s, uint32_t max_dim) {
    return max_dim > 0 && s.h == 1 && s.w > max_dim;
}
inline ImgSize PhysImgSize(ImgSize logical, uint32_t max_dim) {
    if (!NeedsTiling(logical, max_dim)) {
        return logical;
    }
    const uint32_t w = TileWidth(max_dim);
    return ImgSize{w, (logical.w + w - 1) / w};
}

// Host image: row-major, `channels` floats per pixel
struct CpuImage {
    uint32_t width = 0;
    uint32_t height = 0;
    uint32_t channels = 0;
    std::vector<float> data;

    CpuImage() = default;
    CpuImage(uint32_t w, uint32_t h, uint32_t c, float fill = 0.f)
        : width(w), height(h), channels(c), data((size_t)w * h * c, fill) {}
    ImgSize getImgSize() const { return ImgSize{width, height}; }
    float& at(uint32_t x, uint32_t y, uint32_t c) {
        return data[((size_t)y * width + x) * channels + c];
    }
    float at(uint32_t x, uint32_t y, uint32_t c) const {
        return data[((size_t)y * width + x) * channels + c];
    }
};

// Borrowed host image with CpuImage's layout; read only during the call it
// is passed to
struct CpuImageView {
    const float* data = nullptr;
    uint32_t width = 0;
    uint32_t height = 0;
    uint32_t channels = 0;

    CpuImageView() = default;
    CpuImageView(const float* d, uint32_t w, uint32_t h, uint32_t c)
        : data(d), width(w), height(h), channels(c) {}
    explicit CpuImageView(const CpuImage& img)
        : data(img.data.data()), width(img.width), height(img.height), channels(img.channels) {}
    size_t numElems() const { return (size_t)width * height * channels; }
};

class DressiError : public std::runtime_error {
public:
    explicit DressiError(const std::string& msg) : std::runtime_error(msg) {}
};

// Throws DressiError("msg (file:line)")
[[noreturn]] void ThrowDressiError(const std::string& msg, const char* file, int line);

#define DRESSI_CHECK(cond, msg)                                    \
    do {                                                           \
        if (!(cond)) {                                             \
            ::dressi::ThrowDressiError((msg), __FILE__, __LINE__); \
        }                                                          \
    } while (false)

uint32_t NumComponents(VType vtype);
bool IsIntVType(VType vtype);
bool IsMatrixVType(VType vtype);
bool IsVectorVType(VType vtype);  // VEC2..VEC4, IVEC2..IVEC4
// The reference's GLSL type name of a VType ("float", "vec3", "ivec3", ...)
const char* GlslTypeName(VType vtype);
VType VecVTypeOf(uint32_t n_components, bool is_int = false);

}  // namespace dressi

#endif  // DRESSI_TYPES_H
