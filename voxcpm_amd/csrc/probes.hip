// Launch-cost probes: the per-launch floor and the dependent hand-off that
// every product and DiT kernel of a HIP graph pays, measured with the same
// launch pattern as the kernels themselves (bench.py replays them from a
// graph and times them with events on the launch stream).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.hpp"

namespace {

// Every workgroup reads all `chunks` 16-byte chunks of `in` (as each
// product workgroup reads the whole activation block), and workgroup b
// writes its share of `out` as in + 1 per word, so that a launch reading
// what the previous one wrote waits for it. The XOR of everything read is
// stored only when it equals `never`, so no load is dead.
__global__ __launch_bounds__(1024) void HandoffKernel(const uint4* in, uint4* out,
                                                      std::uint32_t chunks, std::uint32_t never,
                                                      std::uint32_t* sink) {
  const std::uint32_t threads = blockDim.x;
  const std::uint32_t per = (chunks + gridDim.x - 1) / gridDim.x;
  const std::uint32_t lo = blockIdx.x * per;
  const std::uint32_t hi = min(lo + per, chunks);
  std::uint32_t x = 0;
  for (std::uint32_t base = 0; base < chunks; base += 4 * threads) {
    uint4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const std::uint32_t i = base + u * threads + threadIdx.x;
      v[u] = i < chunks ? in[i] : uint4{0U, 0U, 0U, 0U};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const std::uint32_t i = base + u * threads + threadIdx.x;
      x ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
      if (i >= lo && i < hi)
        out[i] = uint4{v[u].x + 1U, v[u].y + 1U, v[u].z + 1U, v[u].w + 1U};
    }
  }
  if (x == never)
    sink[0] = x;
}

}  // namespace

extern "C" {

int vx_handoff(const void* in, void* out, size_t bytes, int workgroups, int threads,
               uint32_t never, uint32_t* sink, void* stream) {
  if (sink == nullptr || bytes % 16 != 0 || bytes > (size_t{1} << 30) || workgroups < 1 ||
      workgroups > 65536 || threads < 64 || threads > 1024 || threads % 64 != 0 ||
      (bytes > 0 && (in == nullptr || out == nullptr)))
    return vx::Fail(VX_BAD_ARG, "vx_handoff: bad arguments");
  HandoffKernel<<<static_cast<unsigned>(workgroups), static_cast<unsigned>(threads), 0,
                  vx::Stream(stream)>>>(static_cast<const uint4*>(in), static_cast<uint4*>(out),
                                        static_cast<std::uint32_t>(bytes / 16), never, sink);
  return vx::LaunchStatus("vx_handoff");
}

}  // extern "C"
