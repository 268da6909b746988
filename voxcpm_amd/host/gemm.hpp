// The product operator of the reference (gemm.hpp:49-72): Bf16Gemm::Linear
// with float32 outputs that can accumulate, here over the voxcpm_amd C ABI.
#ifndef VOXCPM_AMD_HOST_GEMM_HPP_
#define VOXCPM_AMD_HOST_GEMM_HPP_

#include <hip/hip_runtime.h>
#include <hipblas/hipblas.h>

#include <cstddef>
#include <memory>

#include "matrix.hpp"

namespace gufo::models::voxcpm {

/// Products of bfloat16 activations with the generator's weights, float32
/// accumulation and output. Q8_0 panels up to 128 rows keep the Q8_0
/// arithmetic exact (a float32 sum per block, scaled per block); more rows
/// use bf16(scale * q) as the reference's expansion does, on the matrix
/// cores without leaving Q8_0 in HBM. bf16 panels and bf16 rows sum the
/// blocks' products on the matrix cores (bf16 rows beyond 32 activation
/// rows are packed into panels in the operator's scratch first, where the
/// reference unpacks for hipBLASLt, gemm.cpp:296-303). The reference's gfx11
/// tile formats are not served and throw GpuError.
class Bf16Gemm {
public:
  /// `fallback` is accepted for the reference's signature (gemm.hpp:51)
  /// and unused: no product falls back to hipBLAS here.
  Bf16Gemm(hipblasHandle_t fallback, hipStream_t stream);
  ~Bf16Gemm();
  Bf16Gemm(const Bf16Gemm&) = delete;
  Bf16Gemm& operator=(const Bf16Gemm&) = delete;

  /// y[rows][out] (+)= x[rows][in] * w[out][in]^T (gemm.hpp:56-58).
  void Linear(const void* x, const Matrix& w, float* y, std::size_t rows,
              std::size_t in, std::size_t out, bool accumulate);

  [[nodiscard]] hipStream_t stream() const { return stream_; }

private:
  struct State;
  std::unique_ptr<State> state_;
  hipStream_t stream_ = nullptr;
};

}  // namespace gufo::models::voxcpm

#endif  // VOXCPM_AMD_HOST_GEMM_HPP_
