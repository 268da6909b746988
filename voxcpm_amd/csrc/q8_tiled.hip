// Q8_0 (or bf16) x bfloat16 products of more than 128 activation rows on
// gfx950's matrix cores (the smaller, latency-bound prefill shapes):
// LDS-tiled, BM activation rows x 128 weight rows per workgroup, 64
// columns (one panel pair, two Q8_0 blocks) per step.
//
// The arithmetic is the reference's expansion beyond 128 rows (gemm.cpp:
// 305-312 with kernels/wmma_products.hip:94-112): every weight becomes
// bf16_rne(f32(f16 scale) * q) once per workgroup and step, and the MFMAs
// accumulate over all of k in float32.
// bf16 panels (kernels/wmma_products.hip:210-213, the WmmaBf16 products)
// take the expanded path's MFMA accumulation with the weights copied as
// they are.
//
// Per step the threads load the step after next into registers (two
// register sets, so a load has two steps of MFMAs to arrive), convert the
// next step's weights into the other LDS buffer, and multiply the current
// one: BM / 32 x 2 waves, each 32 activation rows x 64 weight rows of the
// tile. Consecutive tiles (the activation-row tiles of one weight tile
// first) are placed on one compute die, whose L2 then serves their shared
// weights.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "common.hpp"
#include "products.hpp"
#include "q8.hpp"
#include "q8_tile.hpp"

namespace vx {
namespace {

using q8::AsBf16x8;
using q8::Expand;
using q8::Bf16x8;
using q8::F32x4;
using q8::kUnitBytes;
using q8::kValueBytes;
using q8::Mfma16x16x32;
using q8::PackBf16x2;

constexpr int kTileN = 128;
// LDS rows: 64 bf16 plus 8 of padding (144 bytes, 9 chunks of 16 bytes), so
// that the fragment reads of 16 consecutive rows fall on distinct banks.
constexpr int kRowChunks = 9;
constexpr int kDies = 8;

struct TiledArgs {
  const Bf16* x;
  const std::uint8_t* w;
  float* y;
  Bf16* y_bf16;
  int m, k, n;
  int pairs, groups;
  int m_tiles, n_tiles;
  int accumulate;
  // Split over k (splits > 1): workgroup tile t of split s takes pairs
  // [s pairs_per_split, ...) and stores its float32 sums to
  // partials [splits][m][n]; ReduceSplitsKernel adds them in split order.
  int splits, pairs_per_split;
  float* partials;
};

/// Logical tile of workgroup `b` of `blocks`: workgroup b runs on die b % 8;
/// die d takes a contiguous range of logical tiles (the first blocks % 8
/// dies one more). A bijection on 0..blocks-1.
__device__ inline int DieOrdered(int b, int blocks) {
  const int per = blocks / kDies;
  const int extra = blocks % kDies;
  const int die = b % kDies;
  const int index = b / kDies;
  return die < extra ? die * (per + 1) + index
                     : extra * (per + 1) + (die - extra) * per + index;
}

/// A tile shape: BM activation rows, WM waves along them (x 2 along the 128
/// weight rows, each wave BM / WM x 64), D register sets of prefetched
/// steps, and the workgroups per compute unit the registers are sized for.
template<int BM, int WM, int D, int MINB>
struct TileShape {
  static constexpr int kBm = BM;
  static constexpr int kThreads = WM * 2 * kWave;
  static constexpr int kAPieces = BM * 8 / kThreads;  // 16-byte A pieces per thread per step
  static constexpr int kUnits = 8 / (WM * 2);         // panel units per wave per step
  static constexpr int kMi = BM / WM / 16;             // 16-row MFMA tiles per wave
  static constexpr int kD = D;
  static constexpr int kMinBlocks = MINB;
};

/// MODE: TiledMode (products.hpp) as an int: 1 Q8_0 expanded, 2 bf16
/// panels.
template<class T, int MODE>
__global__ __launch_bounds__(T::kThreads, T::kMinBlocks) void TiledKernel(TiledArgs a) {
  static_assert(MODE == 1 || MODE == 2, "expanded Q8_0 or bf16 panels");
  constexpr bool BF16 = MODE == 2;
  constexpr int kUnit = BF16 ? q8::kBf16UnitBytes : kUnitBytes;
  constexpr int BM = T::kBm;
  constexpr int kThreads = T::kThreads;
  constexpr int kAPieces = T::kAPieces;
  constexpr int kUnits = T::kUnits;
  constexpr int kMi = T::kMi;
  constexpr int D = T::kD;
  __shared__ uint4 lds_a[2][BM * kRowChunks];
  __shared__ uint4 lds_b[2][kTileN * kRowChunks];
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  const int r16 = lane % 16;
  const int octet = lane / 16;
  const int tiles = a.m_tiles * a.n_tiles;
  const int logical = DieOrdered(static_cast<int>(blockIdx.x), tiles * a.splits);
  const int split = logical / tiles;
  const int tile = logical % tiles;
  const int row0 = (tile % a.m_tiles) * BM;
  const int group0 = (tile / a.m_tiles) * (kTileN / 16);
  const __amdgpu_buffer_rsrc_t x_buffer = q8::BufferOf(
      a.x, 2U * static_cast<std::uint32_t>(a.m) * static_cast<std::uint32_t>(a.k));
  const int first_pair = split * a.pairs_per_split;
  const int steps = min(a.pairs, first_pair + a.pairs_per_split) - first_pair;
  // The tile's panel groups as one buffer (under 2^31 bytes for k <= 2^22).
  const std::uint32_t group_bytes = static_cast<std::uint32_t>(a.pairs) * kUnit;
  const __amdgpu_buffer_rsrc_t w_buffer =
      q8::BufferOf(a.w + static_cast<std::size_t>(group0) * group_bytes,
                   static_cast<std::uint32_t>(min(kTileN / 16, a.groups - group0)) * group_bytes);

  struct Staging {
    uint4 x[kAPieces];
    uint4 w[kUnits];
    uint4 w2[kUnits];  // bf16: the pair's second block
    std::uint32_t scales[kUnits];
  };
  // Every step issues the same loads, steps past the split's end included:
  // buffer loads at an offset past the buffer read zero without an access,
  // so rows past m, columns past k and dead steps cost no traffic, and with
  // no branch around them the compiler counts the loads in flight and waits
  // for the oldest step only.
  const auto fetch = [&](int step, Staging& s) {
    const int pair = first_pair + step;
    const bool live = step < steps;
#pragma unroll
    for (int i = 0; i < kAPieces; ++i) {
      const int piece = tid + kThreads * i;
      const int row = row0 + piece / 8;
      const int column = 64 * pair + 8 * (piece % 8);
      s.x[i] = q8::BufferLoad16(x_buffer, 2U * static_cast<std::uint32_t>(row * a.k + column),
                                live && row < a.m && column < a.k);
    }
#pragma unroll
    for (int u = 0; u < kUnits; ++u) {
      const int group = min(kUnits * wave + u, a.groups - 1 - group0);
      const std::uint32_t unit =
          static_cast<std::uint32_t>(group) * group_bytes +
          static_cast<std::uint32_t>(live ? pair : 0) * kUnit;
      s.w[u] = q8::BufferLoad16(w_buffer, unit + 16 * lane, live);
      if constexpr (BF16)
        s.w2[u] = q8::BufferLoad16(w_buffer, unit + q8::kBf16HalfBytes + 16 * lane, live);
      else
        s.scales[u] = q8::BufferLoad4(w_buffer, unit + kValueBytes + 4 * r16, live);
    }
  };
  const auto store = [&](int buffer, const Staging& s) {
#pragma unroll
    for (int i = 0; i < kAPieces; ++i) {
      const int piece = tid + kThreads * i;
      lds_a[buffer][(piece / 8) * kRowChunks + piece % 8] = s.x[i];
    }
#pragma unroll
    for (int u = 0; u < kUnits; ++u) {
      const int row = 16 * (kUnits * wave + u) + r16;
      const float s0 = HalfValue(static_cast<std::uint16_t>(s.scales[u] & 0xFFFFU));
      const float s1 = HalfValue(static_cast<std::uint16_t>(s.scales[u] >> 16));
      uint4 first, second;
      if constexpr (BF16) {
        first = s.w[u];
        second = s.w2[u];
      } else {
        first = Expand(s.w[u].x, s.w[u].y, s0);
        second = Expand(s.w[u].z, s.w[u].w, s1);
      }
      lds_b[buffer][row * kRowChunks + octet] = first;
      lds_b[buffer][row * kRowChunks + 4 + octet] = second;
    }
  };

  const int wm = wave / 2;
  const int wn = wave % 2;
  F32x4 acc[kMi][4];
#pragma unroll
  for (int i = 0; i < kMi; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[i][j] = F32x4{0.0F, 0.0F, 0.0F, 0.0F};

  const auto compute = [&](int buffer) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      Bf16x8 af[kMi], bf[4];
#pragma unroll
      for (int i = 0; i < kMi; ++i)
        af[i] = AsBf16x8(
            lds_a[buffer][((BM / (kThreads / kWave / 2)) * wm + 16 * i + r16) * kRowChunks +
                          4 * h + octet]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = 64 * wn + 16 * j + r16;
        bf[j] = AsBf16x8(lds_b[buffer][row * kRowChunks + 4 * h + octet]);
      }
#pragma unroll
      for (int i = 0; i < kMi; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = Mfma16x16x32(af[i], bf[j], acc[i][j]);
    }
  };

  // D register sets: set q % D holds step q from its fetch (D steps ahead)
  // until its store; LDS buffer q % 2 holds step q while it is multiplied.
  // The loop is unrolled over a multiple of D and 2 so that both indices
  // are compile-time.
  constexpr int U = D % 2 == 0 ? D : 2 * D;
  // The stores after the last step write zeros into the LDS buffer that
  // no later step reads.
  Staging staged[D];
#pragma unroll
  for (int d = 0; d < D; ++d)
    fetch(d, staged[d]);
  store(0, staged[0]);
  __syncthreads();
  for (int p = 0; p < steps; p += U) {
#pragma unroll
    for (int d = 0; d < U; ++d) {
      const int q = p + d;
      if (q >= steps)
        break;
      fetch(q + D, staged[d % D]);
      compute(d % 2);
      store((d + 1) % 2, staged[(d + 1) % D]);
      __syncthreads();
    }
  }

  constexpr int kRowsPerWave = BM / (kThreads / kWave / 2);
  // Epilogue: element e of tile (i, j) is row 4 octet + e and column r16 of
  // the tile. One uniform branch picks the output; each element is then one
  // buffer store at the lane's offset plus a constant of e (accumulation:
  // the tile's loads first). Rows past m lie past the buffer, whose range
  // check drops them.
  const std::size_t count = static_cast<std::size_t>(a.m) * a.n;
  const auto emit = [&](auto kind, void* base) {
    constexpr int K = decltype(kind)::value;  // 0 float32, 1 bf16, 2 float32 +=
    constexpr std::uint32_t width = K == 1 ? 2 : 4;
    const __amdgpu_buffer_rsrc_t out =
        q8::BufferOf(base, static_cast<std::uint32_t>(count * width));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int column = 16 * group0 + 64 * wn + 16 * j + r16;
      if (column >= a.n)
        continue;
#pragma unroll
      for (int i = 0; i < kMi; ++i) {
        const std::uint32_t lane_bytes = width * static_cast<std::uint32_t>(
            (row0 + kRowsPerWave * wm + 16 * i + 4 * octet) * a.n + column);
        std::uint32_t offset[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          offset[e] = lane_bytes + width * static_cast<std::uint32_t>(e * a.n);
        // Elements as values first: hipcc's bit cast of a vector element
        // taken in place reads element 0.
        float value[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          value[e] = acc[i][j][e];
        if constexpr (K == 2) {
          float prior[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            prior[e] = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(out, static_cast<int>(offset[e]), 0, 0));
#pragma unroll
          for (int e = 0; e < 4; ++e)
            value[e] += prior[e];
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (K == 1)
            __builtin_amdgcn_raw_buffer_store_b16(q8::Bf16Fast(value[e]), out,
                                                  static_cast<int>(offset[e]), 0, 0);
          else
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(std::uint32_t, value[e]), out,
                                                  static_cast<int>(offset[e]), 0, 0);
        }
      }
    }
  };
  // Offsets stay below 2^31 bytes (rows to the last tile's end included).
  if ((static_cast<std::size_t>(a.m) + BM) * a.n * 4 < (std::size_t{1} << 31)) {
    if (a.splits > 1)
      emit(std::integral_constant<int, 0>{}, a.partials + static_cast<std::size_t>(split) * count);
    else if (a.y_bf16 != nullptr)
      emit(std::integral_constant<int, 1>{}, a.y_bf16);
    else if (a.accumulate)
      emit(std::integral_constant<int, 2>{}, a.y);
    else
      emit(std::integral_constant<int, 0>{}, a.y);
    return;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int column = 16 * group0 + 64 * wn + 16 * j + r16;
    if (column >= a.n)
      continue;
#pragma unroll
    for (int i = 0; i < kMi; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = row0 + kRowsPerWave * wm + 16 * i + 4 * octet + e;
        if (row >= a.m)
          continue;
        const std::size_t at = static_cast<std::size_t>(row) * a.n + column;
        if (a.splits > 1)
          a.partials[static_cast<std::size_t>(split) * a.m * a.n + at] = acc[i][j][e];
        else if (a.y_bf16 != nullptr)
          a.y_bf16[at] = q8::Bf16Fast(acc[i][j][e]);
        else
          a.y[at] = a.accumulate ? a.y[at] + acc[i][j][e] : acc[i][j][e];
      }
  }
}

/// y (+)= the splits' partial sums added in split order, or their bf16
/// rounding; four consecutive elements per thread (n % 4 == 0), else one.
__global__ __launch_bounds__(256) void ReduceSplitsKernel(TiledArgs a) {
  const std::size_t count = static_cast<std::size_t>(a.m) * a.n;
  const std::size_t plane = count;
  const std::size_t first =
      (static_cast<std::size_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (first >= count)
    return;
  const int width = a.n % 4 == 0 ? 4 : 1;
  for (int v = 0; v < 4; v += width) {
    const std::size_t at = first + v;
    if (at >= count)
      break;
    float sum[4] = {0.0F, 0.0F, 0.0F, 0.0F};
    for (int s = 0; s < a.splits; ++s) {
      const float* part = a.partials + s * plane + at;
      if (width == 4) {
        const float4 p = *reinterpret_cast<const float4*>(part);
        sum[0] += p.x;
        sum[1] += p.y;
        sum[2] += p.z;
        sum[3] += p.w;
      } else {
        sum[0] += part[0];
      }
    }
    for (int e = 0; e < width; ++e) {
      if (a.y_bf16 != nullptr)
        a.y_bf16[at + e] = q8::Bf16Fast(sum[e]);
      else
        a.y[at + e] = a.accumulate ? a.y[at + e] + sum[e] : sum[e];
    }
  }
}

template<class T, int MODE>
void Launch(const TiledArgs& args, hipStream_t stream) {
  TiledKernel<T, MODE>
      <<<args.m_tiles * args.n_tiles * args.splits, T::kThreads, 0, stream>>>(args);
  if (args.splits > 1) {
    const std::size_t quads = (static_cast<std::size_t>(args.m) * args.n + 3) / 4;
    ReduceSplitsKernel<<<static_cast<unsigned>((quads + 255) / 256), 256, 0, stream>>>(args);
  }
}

using Small = TileShape<64, 2, 2, 2>;
using Large = TileShape<128, 4, 2, 1>;

}  // namespace

TiledPlan PlanTiled(std::size_t m, std::size_t k, std::size_t n, std::size_t partial_floats) {
  TiledPlan plan;
  const std::size_t n_tiles = (n + kTileN - 1) / kTileN;
  const std::size_t pairs = q8::Pairs(k);
  // 128-row tiles (8 waves of 32 x 64) once they give at least 192
  // workgroups, else 64-row tiles (4 waves, two workgroups per compute
  // unit): the faster of the two at every prefill shape measured on MI355X.
  const std::size_t tiles128 = (m + 127) / 128 * n_tiles;
  plan.bm = m > 64 && tiles128 >= 192 ? 128 : 64;
  plan.m_tiles = static_cast<int>((m + plan.bm - 1) / plan.bm);
  // Grids of at most 144 tiles split k (powers of two, at least four
  // steps each, up to 384 workgroups) when the scratch holds the partial
  // sums: measured faster on MI355X there, slower on larger grids, where
  // the second launch costs more than the parallelism gains.
  plan.splits = 1;
  const std::size_t tiles = static_cast<std::size_t>(plan.m_tiles) * n_tiles;
  const std::size_t room = partial_floats < kMaxSplitFloats ? partial_floats : kMaxSplitFloats;
  while (tiles <= 144 && tiles * 2 * plan.splits <= 384 && pairs >= 8U * plan.splits &&
         2 * plan.splits * m * n <= room)
    plan.splits *= 2;
  return plan;
}

int RunTiled(const Bf16* x, const void* w, float* y, Bf16* y_bf16, std::size_t m,
             std::size_t k, std::size_t n, bool accumulate, TiledMode mode,
             float* partials, std::size_t partial_floats, hipStream_t stream) {
  TiledArgs args;
  args.x = x;
  args.w = static_cast<const std::uint8_t*>(w);
  args.y = y;
  args.y_bf16 = y_bf16;
  args.m = static_cast<int>(m);
  args.k = static_cast<int>(k);
  args.n = static_cast<int>(n);
  args.pairs = static_cast<int>(q8::Pairs(k));
  args.groups = static_cast<int>(q8::Groups(n));
  args.n_tiles = static_cast<int>((n + kTileN - 1) / kTileN);
  args.accumulate = accumulate ? 1 : 0;
  const TiledPlan plan = PlanTiled(m, k, n, partial_floats);
  const int bm = plan.bm;
  args.m_tiles = plan.m_tiles;
  args.splits = plan.splits;
  args.pairs_per_split = (args.pairs + args.splits - 1) / args.splits;
  args.partials = partials;
  switch (mode) {
    case TiledMode::kQ8Expanded:
      bm == 64 ? Launch<Small, 1>(args, stream) : Launch<Large, 1>(args, stream);
      return LaunchStatus("q8 expanded product");
    case TiledMode::kBf16:
      bm == 64 ? Launch<Small, 2>(args, stream) : Launch<Large, 2>(args, stream);
      return LaunchStatus("bf16 tiled product");
  }
  return Fail(VX_BAD_ARG, "tiled product: unknown mode");
}

}  // namespace vx
