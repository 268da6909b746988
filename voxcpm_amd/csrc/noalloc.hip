// The Q8_0 product for callers that cannot allocate (code under HIP graph
// capture, serving loops, harnesses that forbid hipMalloc): vx_q8_linear
// with its split scratch in a file-scope device array instead of a
// vx_scratch.
//
// The array is `scratch` below. Its name in host code is a host-side
// stand-in, not a device address: each device's address comes from
// hipGetSymbolAddress, taken once per device (with that device current) on
// the first call there, and only that address reaches the kernels. Every
// call on a device shares the device's array; the products write every
// partial sum they later read, so nothing needs clearing between calls,
// and calls that overlap on one device (two streams at once) race.
#include <hip/hip_runtime.h>

#include <array>
#include <cstdint>
#include <mutex>

#include "common.hpp"
#include "products.hpp"
#include "q8.hpp"

/// Floats of the array: the k splits of the prefill products (m > 128)
/// store splits x m x n partial sums here. 12 MiB per device: every default
/// plan keeps its splits' partial sums within it.
constexpr std::size_t kScratchFloats = vx::kMaxSplitFloats;
static_assert(kScratchFloats >= VX_PREFILL_SPLIT_FLOATS, "the array holds every split");

static __device__ __align__(256) float scratch[kScratchFloats];

namespace {

constexpr int kMaxDevices = 64;

struct DeviceScratch {
  std::once_flag once;
  hipError_t status = hipSuccess;
  float* address = nullptr;
};

std::array<DeviceScratch, kMaxDevices> devices;

/// The current device's address of `scratch` (nullptr and a failed status
/// when it cannot be had).
int ScratchAddress(float** address) {
  int device = 0;
  VX_HIP(hipGetDevice(&device), "vx_q8_linear_noalloc: hipGetDevice");
  if (device < 0 || device >= kMaxDevices)
    return vx::Fail(VX_UNSUPPORTED, "vx_q8_linear_noalloc: device index past 63");
  DeviceScratch& entry = devices[static_cast<std::size_t>(device)];
  std::call_once(entry.once, [&entry] {
    void* found = nullptr;
    entry.status = hipGetSymbolAddress(&found, HIP_SYMBOL(scratch));
    entry.address = static_cast<float*>(found);
  });
  if (entry.status != hipSuccess || entry.address == nullptr)
    return vx::FailHip(entry.status != hipSuccess ? entry.status : hipErrorInvalidSymbol,
                       "vx_q8_linear_noalloc: hipGetSymbolAddress");
  *address = entry.address;
  return VX_OK;
}

}  // namespace

extern "C" {

int vx_q8_linear_noalloc(const uint16_t* x, const void* packed, float* y, size_t m,
                         size_t k, size_t n, int accumulate, void* stream) {
  VX_TRY(vx::CheckProduct(x, packed, y, m, k, n, "vx_q8_linear_noalloc"));
  if (m <= vx::kExactRows)  // these plans split nothing over workgroups
    return vx_q8_linear(x, packed, y, m, k, n, accumulate, nullptr, stream);
  // The planners keep every split within kMaxSplitFloats floats whatever
  // room they are given, which the array holds: they pick here the split
  // they pick for a vx_scratch of at least that many floats.
  float* address = nullptr;
  VX_TRY(ScratchAddress(&address));
  if (vx::UseRowBlocks(m, k, n, true))  // no split either
    return vx_q8_linear(x, packed, y, m, k, n, accumulate, nullptr, stream);
  if (vx::UseGemm(m, n))
    return vx::RunGemm(x, packed, y, nullptr, m, k, n, accumulate != 0, false, address,
                       kScratchFloats, vx::Stream(stream));
  return vx::RunTiled(x, packed, y, nullptr, m, k, n, accumulate != 0,
                      vx::TiledMode::kQ8Expanded, address, kScratchFloats, vx::Stream(stream));
}

}  // extern "C"
