// Weight matrices on the device (matrix.hpp:9-19 of the reference) with the
// gfx950 panel layout added as a format.
#ifndef VOXCPM_AMD_HOST_MATRIX_HPP_
#define VOXCPM_AMD_HOST_MATRIX_HPP_

#include <cstdint>

namespace gufo::models::voxcpm {

/// How a weight matrix is stored on the device.
enum class WeightFormat : std::uint8_t {
  kBf16,        // bfloat16 [out][in], row-major
  kBf16Tiles,   // the reference's gfx11 bfloat16 tiles (not served)
  kQ8Tiles,     // the reference's gfx11 Q8_0 tiles (not served)
  kQ8Panels,    // GGML Q8_0 in gfx950 MFMA panels (vx_q8_pack)
  kBf16Panels,  // bfloat16 in gfx950 MFMA panels (vx_bf16_pack)
};

/// A weight matrix [out][in] on the device.
struct Matrix {
  WeightFormat format = WeightFormat::kQ8Panels;
  const void* data = nullptr;
};

}  // namespace gufo::models::voxcpm

#endif  // VOXCPM_AMD_HOST_MATRIX_HPP_
