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
  // bf16 rows packed into panels for products of more than 32 rows (the
  // reference's `unpacked` buffer, gemm.cpp:99).
  void* panels = nullptr;
  std::size_t panel_bytes = 0;

  ~State() {
    vx_scratch_destroy(scratch);
    if (panels != nullptr)
      (void)hipFree(panels);
  }

  void* Panels(std::size_t bytes) {
    if (bytes > panel_bytes) {
      if (panels != nullptr)
        Check(hipFree(panels), "hipFree");
      panels = nullptr;
      panel_bytes = 0;
      Check(hipMalloc(&panels, bytes), "hipMalloc");
      panel_bytes = bytes;
    }
    return panels;
  }

  vx_scratch* Reserve(std::size_t want_rows, std::size_t want_out) {
    if (want_rows > 128) {
      // The expanded path splits k on grids of few tiles into at most
      // VX_PREFILL_SPLIT_FLOATS floats of partial sums: a scratch of
      // 128 x (that / (16 x 128)) holds all of them.
      want_rows = 128;
      want_out = VX_PREFILL_SPLIT_FLOATS / (16 * 128);
    }
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
  const auto* activations = static_cast<const std::uint16_t*>(x);
  switch (w.format) {
    case WeightFormat::kQ8Panels:
      CheckVx(vx_q8_linear(activations, w.data, y, rows, in, out, accumulate ? 1 : 0,
                           state_->Reserve(rows, out), stream_),
              "Bf16Gemm::Linear");
      return;
    case WeightFormat::kBf16Panels:
      CheckVx(vx_bf16_linear(activations, w.data, y, rows, in, out, accumulate ? 1 : 0,
                             state_->Reserve(rows, out), stream_),
              "Bf16Gemm::Linear");
      return;
    case WeightFormat::kBf16: {
      const auto* rows_w = static_cast<const std::uint16_t*>(w.data);
      if (rows <= 32) {
        CheckVx(vx_bf16_linear_rows(activations, rows_w, y, rows, in, out, accumulate ? 1 : 0,
                                    stream_),
                "Bf16Gemm::Linear");
        return;
      }
      void* panels = state_->Panels(vx_bf16_packed_bytes(out, in));
      CheckVx(vx_bf16_pack(rows_w, out, in, panels, stream_), "Bf16Gemm::Linear");
      CheckVx(vx_bf16_linear(activations, panels, y, rows, in, out, accumulate ? 1 : 0,
                             state_->Reserve(rows, out), stream_),
              "Bf16Gemm::Linear");
      return;
    }
    default:
      throw GpuError("Bf16Gemm::Linear: the gfx11 tile formats are not served by this build");
  }
}

}  // namespace gufo::models::voxcpm
