// Products of more than 128 activation rows on Q8_0 panels: a dense
// contraction, bound by the matrix cores. It follows the reference's
// arithmetic for such products (gemm.cpp:305-312): every weight becomes
// bf16_rne(f32(f16 scale) * q) (kernels/wmma_products.hip:94-112) and the
// products sum in float32 over all of k; here the weights stay 8-bit in
// HBM and are expanded in registers, once per workgroup, into LDS.
//
// Tile: 128 rows x 128 weight rows per workgroup (4 waves of 64 x 64),
// 64 columns (one panel pair) per step, double-buffered through LDS with
// the next step's global loads in flight during this step's MFMAs.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.hpp"
#include "products.hpp"
#include "q8.hpp"

namespace vx {
namespace {

using q8::AsBf16x8;
using q8::Bf16x8;
using q8::F32x4;
using q8::kUnitBytes;
using q8::kValueBytes;
using q8::Mfma16x16x32;

constexpr int kTileM = 128;
constexpr int kTileN = 128;
constexpr int kThreads = 256;
// LDS rows of 64 bf16 plus 8 of padding (144 bytes) spread the 16-byte
// fragment reads of consecutive rows over the banks.
constexpr int kLdsRow = 72;

struct PrefillArgs {
  const Bf16* x;
  const std::uint8_t* w;
  float* y;
  Bf16* y_bf16;
  int m, k, n;
  int pairs;
  int accumulate;
};

__device__ inline std::uint32_t PackBf16(float lo, float hi) {
  return static_cast<std::uint32_t>(Bf16Bits(lo)) |
         (static_cast<std::uint32_t>(Bf16Bits(hi)) << 16);
}

// 8 int8 values (two dwords) times `scale`, each rounded to bf16.
__device__ inline uint4 Expand(std::uint32_t w0, std::uint32_t w1,
                               float scale) {
  const auto v = [&](std::uint32_t word, int byte) {
    return scale * static_cast<float>(static_cast<std::int8_t>(word >> (8 * byte)));
  };
  return uint4{PackBf16(v(w0, 0), v(w0, 1)), PackBf16(v(w0, 2), v(w0, 3)),
               PackBf16(v(w1, 0), v(w1, 1)), PackBf16(v(w1, 2), v(w1, 3))};
}

__global__ __launch_bounds__(kThreads) void PrefillKernel(PrefillArgs args) {
  __shared__ uint4 lds_a[2][kTileM * kLdsRow / 8];
  __shared__ uint4 lds_b[2][kTileN * kLdsRow / 8];
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int tile_m = static_cast<int>(blockIdx.x) * kTileM;
  const int tile_n = static_cast<int>(blockIdx.y) * kTileN;
  const int groups = (args.n + 15) / 16;
  const int k_blocks = args.k / 32;
  const int r16 = lane % 16;
  const int octet = lane / 16;

  // Global -> register staging of one pair: the A tile (128 rows x 64
  // columns: 4 pieces of 16 bytes per thread) and 2 panel units per wave.
  struct Staged {
    uint4 a[4];
    uint4 w[2];
    std::uint32_t scales[2];
  };
  const auto fetch = [&](int pair, Staged& s) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int piece = threadIdx.x + kThreads * i;  // 0..1023
      const int row = piece / 8;
      const int column = 64 * pair + 8 * (piece % 8);
      const int global_row = tile_m + row;
      if (global_row < args.m && column / 32 < k_blocks)
        s.a[i] = *reinterpret_cast<const uint4*>(
            args.x + static_cast<std::size_t>(global_row) * args.k + column);
      else
        s.a[i] = uint4{0U, 0U, 0U, 0U};
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int group = min(tile_n / 16 + 2 * wave + u, groups - 1);
      const std::uint8_t* unit =
          args.w + (static_cast<std::size_t>(group) * args.pairs + pair) * kUnitBytes;
      s.w[u] = *reinterpret_cast<const uint4*>(unit + 16 * lane);
      s.scales[u] =
          *reinterpret_cast<const std::uint32_t*>(unit + kValueBytes + 4 * r16);
    }
  };
  const auto store = [&](int buffer, const Staged& s) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int piece = threadIdx.x + kThreads * i;
      lds_a[buffer][((piece / 8) * kLdsRow + 8 * (piece % 8)) / 8] = s.a[i];
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int row = 16 * (2 * wave + u) + r16;
      const float s0 = HalfValue(static_cast<std::uint16_t>(s.scales[u] & 0xFFFFU));
      const float s1 = HalfValue(static_cast<std::uint16_t>(s.scales[u] >> 16));
      lds_b[buffer][(row * kLdsRow + 8 * octet) / 8] = Expand(s.w[u].x, s.w[u].y, s0);
      lds_b[buffer][(row * kLdsRow + 32 + 8 * octet) / 8] =
          Expand(s.w[u].z, s.w[u].w, s1);
    }
  };

  // Wave (wm, wn) computes rows 64 wm .. +64 and weight rows 64 wn .. +64
  // of the tile: 4 x 4 fragments of 16 x 16.
  const int wm = wave / 2;
  const int wn = wave % 2;
  F32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[i][j] = F32x4{0.0F, 0.0F, 0.0F, 0.0F};

  Staged staged;
  fetch(0, staged);
  store(0, staged);
  __syncthreads();
  for (int pair = 0; pair < args.pairs; ++pair) {
    const int buffer = pair % 2;
    if (pair + 1 < args.pairs)
      fetch(pair + 1, staged);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      Bf16x8 a[4];
      Bf16x8 b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        a[i] = AsBf16x8(lds_a[buffer][((64 * wm + 16 * i + r16) * kLdsRow +
                                       32 * h + 8 * octet) / 8]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        b[j] = AsBf16x8(lds_b[buffer][((64 * wn + 16 * j + r16) * kLdsRow +
                                       32 * h + 8 * octet) / 8]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = Mfma16x16x32(a[i], b[j], acc[i][j]);
    }
    if (pair + 1 < args.pairs) {
      store(buffer ^ 1, staged);
      __syncthreads();
    }
  }

#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int column = tile_n + 64 * wn + 16 * j + r16;
      if (column >= args.n)
        continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = tile_m + 64 * wm + 16 * i + 4 * octet + e;
        if (row >= args.m)
          continue;
        const std::size_t at = static_cast<std::size_t>(row) * args.n + column;
        if (args.y_bf16 != nullptr)
          args.y_bf16[at] = Bf16Bits(acc[i][j][e]);
        else
          args.y[at] = args.accumulate ? args.y[at] + acc[i][j][e] : acc[i][j][e];
      }
    }
}

}  // namespace

int RunPrefill(const Bf16* x, const void* w, float* y, Bf16* y_bf16,
               std::size_t m, std::size_t k, std::size_t n, bool accumulate,
               hipStream_t stream) {
  PrefillArgs args;
  args.x = x;
  args.w = static_cast<const std::uint8_t*>(w);
  args.y = y;
  args.y_bf16 = y_bf16;
  args.m = static_cast<int>(m);
  args.k = static_cast<int>(k);
  args.n = static_cast<int>(n);
  args.pairs = static_cast<int>(q8::Pairs(k));
  args.accumulate = accumulate ? 1 : 0;
  const dim3 grid(static_cast<unsigned>((m + kTileM - 1) / kTileM),
                  static_cast<unsigned>((n + kTileN - 1) / kTileN));
  PrefillKernel<<<grid, kThreads, 0, stream>>>(args);
  return LaunchStatus("q8 prefill product");
}

}  // namespace vx
