#include "gemm.hpp"

#include <string>

#include "device.hpp"
#include "voxcpm_amd.h"

namespace gufo::models::voxcpm {

// The split scratch of the products, grown to the largest product seen
// (the reference's State partials/counters, gemm.cpp:95-98).
struct Bf16Gemm::State {
  vx_scratch* scratch = nullptr;
  std::size_t rows = 0;
  std::size_t out = 0;

  ~State() { vx_scratch_destroy(scratch); }

  vx_scratch* Reserve(std::size_t want_rows, std::size_t want_out) {
    if (want_rows > 128)
      return scratch;  // the expanded path needs no split scratch
    if (scratch != nullptr && want_rows <= rows && want_out <= out)
      return scratch;
    rows = std::max(rows, want_rows);
    out = std::max(out, want_out);
    vx_scratch_destroy(scratch);
    scratch = nullptr;
    CheckVx(vx_scratch_create(&scratch, rows, out), "vx_scratch_create");
    return scratch;
  }
};

Bf16Gemm::Bf16Gemm(hipblasHandle_t /*fallback*/, hipStream_t stream)
    : state_(std::make_unique<State>()), stream_(stream) {}

Bf16Gemm::~Bf16Gemm() = default;

void Bf16Gemm::Linear(const void* x, const Matrix& w, float* y,
                      std::size_t rows, std::size_t in, std::size_t out,
                      bool accumulate) {
  if (w.format != WeightFormat::kQ8Panels)
    throw GpuError("Bf16Gemm::Linear: this build serves Q8_0 panels only");
  vx_scratch* scratch = state_->Reserve(rows, out);
  CheckVx(vx_q8_linear(static_cast<const std::uint16_t*>(x), w.data, y, rows,
                       in, out, accumulate ? 1 : 0, scratch, stream_),
          "Bf16Gemm::Linear");
}

}  // namespace gufo::models::voxcpm
