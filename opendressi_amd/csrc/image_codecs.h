// image_codecs.h -- in-memory decoders of the 8-bit image formats the
// examples read (PNG in assets.cpp, JPEG in jpeg.cpp), shared by
// LoadImageRgb and LoadGltfScene's texture decoding. Host code.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace dressi_examples {
namespace codec {

// A decoded image in its own components (1 gray, 2 gray + alpha, 3 RGB,
// 4 RGBA), 8-bit samples row-major; `bits` is the file's sample depth
// (16-bit PNG samples keep their high byte here).
struct Image8 {
    uint32_t width = 0, height = 0, comp = 0, bits = 8;
    std::vector<uint8_t> px;  // width * height * comp
};

// `what` names the source in error messages (std::runtime_error).
Image8 DecodePng(const uint8_t* data, size_t n, const std::string& what);
Image8 DecodeJpeg(const uint8_t* data, size_t n, const std::string& what);
// By signature: PNG or JPEG.
Image8 DecodeImage(const uint8_t* data, size_t n, const std::string& what);

}  // namespace codec
}  // namespace dressi_examples
