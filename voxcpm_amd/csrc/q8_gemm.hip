// Prefill-sized products (more than 128 activation rows) on gfx950's
// 32 x 32 x 16 bf16 matrix cores: the reference's expansion of Q8_0 weights
// to bf16(f16 scale * q) (gemm.cpp:305-312, kernels/wmma_products.hip:94-112)
// with float32 sums over all of k, or bf16 panels as they are
// (kernels/wmma_products.hip:210-213).
//
// A workgroup computes a BM x BN tile of y with WM x WN waves, each wave a
// (BM / WM) x (BN / WN) block of 32 x 32 MFMA tiles whose accumulators stay
// in registers for the whole reduction. k advances 64 columns (one panel
// pair) per step: the threads load one or two steps ahead into registers
// (activation rows as 16-byte pieces, one panel unit per 16 weight rows),
// expand the next step's weights to bf16 once for the whole workgroup and
// store both into the other half of a double-buffered LDS tile, and
// multiply the current half. Every 16-byte LDS chunk of a 128-byte row sits
// at chunk ^ ((row / 2) % 8), so that the 16 rows one 16-lane group reads
// fall on different banks. Tiles of one weight tile are placed on one compute die
// (workgroup b runs on die b % 8), whose L2 then serves their shared
// weights; grids of few tiles split k over workgroups whose partial sums a
// second launch adds in split order.
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
using q8::kUnitBytes;
using q8::kValueBytes;
using q8::PackBf16x2;

constexpr int kDies = 8;

typedef float F32x16 __attribute__((ext_vector_type(16)));

/// C (32 x 32, float32) += A (32 x 16, bf16) B (16 x 32, bf16): lane L holds
/// A row L % 32 and B column L % 32, each at reduction indices
/// 8 (L / 32) .. + 7; C element v of lane L is row 8 (v / 4) + 4 (L / 32) +
/// v % 4, column L % 32.
__device__ inline F32x16 Mfma32(const Bf16x8& a, const Bf16x8& b, const F32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

struct GemmArgs {
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
  // partials [splits][m][n]; a second launch adds them in split order.
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

/// LDS index of 16-byte chunk `chunk` (0..7) of row `row` of a 128-byte-row
/// operand tile: chunk ^ ((row / 2) % 8). Rows alternate between the two
/// 128-byte halves of a 256-byte bank line, so the 16 rows of a 16-lane
/// group land on 16 different 16-byte bank groups (XOR with row % 8 put
/// rows r and r + 8 on one: measured 2-4 % slower on MI355X).
__device__ inline int Swizzled(int row, int chunk) {
  return row * 8 + (chunk ^ ((row >> 1) & 7));
}

/// MODE: 1 Q8_0 panels expanded, 2 bf16 panels (TiledMode). D: register
/// sets of prefetched steps (1 or 2).
template<int BM, int BN, int WM, int WN, int D, int MODE>
__global__ __launch_bounds__(WM * WN * kWave) void GemmKernel(GemmArgs a) {
  constexpr bool BF16 = MODE == 2;
  constexpr int kUnit = BF16 ? q8::kBf16UnitBytes : kUnitBytes;
  constexpr int kThreads = WM * WN * kWave;
  constexpr int kWaves = WM * WN;
  constexpr int TM = BM / WM;
  constexpr int TN = BN / WN;
  constexpr int FM = TM / 32;
  constexpr int FN = TN / 32;
  constexpr int kAPieces = BM * 8 / kThreads;       // 16-byte x pieces per thread per step
  constexpr int kUnits = BN / 16 / kWaves;          // panel units per wave per step
  static_assert(FM >= 1 && FN >= 1 && kAPieces >= 1 && kUnits >= 1, "tile shape");
  static_assert(BM * 8 % kThreads == 0 && (BN / 16) % kWaves == 0, "tile shape");
  extern __shared__ uint4 lds[];
  uint4* const lds_a = lds;               // [2][BM rows][8 chunks]
  uint4* const lds_b = lds + 2 * BM * 8;  // [2][BN rows][8 chunks]

  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  const int r16 = lane % 16;
  const int octet = lane / 16;
  const int tiles = a.m_tiles * a.n_tiles;
  const int logical = DieOrdered(static_cast<int>(blockIdx.x), tiles * a.splits);
  // The divisions run on the vector unit: readfirstlane keeps the tile's
  // coordinates (and the weight buffer made from them) in scalar registers.
  const int split = __builtin_amdgcn_readfirstlane(logical / tiles);
  const int tile = __builtin_amdgcn_readfirstlane(logical % tiles);
  const int row0 = __builtin_amdgcn_readfirstlane((tile % a.m_tiles) * BM);
  const int group0 = __builtin_amdgcn_readfirstlane((tile / a.m_tiles) * (BN / 16));
  const __amdgpu_buffer_rsrc_t x_buffer = q8::BufferOf(
      a.x, 2U * static_cast<std::uint32_t>(a.m) * static_cast<std::uint32_t>(a.k));
  const int first_pair = split * a.pairs_per_split;
  const int steps = min(a.pairs, first_pair + a.pairs_per_split) - first_pair;
  // The tile's panel groups as one buffer (offsets stay 32-bit).
  const std::uint32_t group_bytes = static_cast<std::uint32_t>(a.pairs) * kUnit;
  const int live_groups = min(BN / 16, a.groups - group0);
  const __amdgpu_buffer_rsrc_t w_buffer =
      q8::BufferOf(a.w + static_cast<std::size_t>(group0) * group_bytes,
                   static_cast<std::uint32_t>(live_groups) * group_bytes);

  struct Staging {
    uint4 x[kAPieces];
    uint4 w[kUnits];
    uint4 w2[kUnits];  // bf16: the pair's second block
    std::uint32_t scales[kUnits];
  };
  // Every step issues the same loads, steps past the split's end included:
  // buffer loads at an offset past the buffer read zero without an access,
  // so rows past m, columns past k, groups past n and dead steps cost no
  // traffic, and with no branch around them the compiler counts the loads
  // in flight and waits for the oldest step only.
  // Part `part` of 4 (or all parts, part < 0) of a step's loads: the
  // activation pieces (what & 1) and the panel units (what & 2).
  const auto fetch = [&](int step, Staging& s, int part = -1, int what = 3) {
    const int pair = first_pair + step;
    const bool live = step < steps;
#pragma unroll
    for (int i = 0; i < kAPieces; ++i) {
      if ((what & 1) == 0 || (part >= 0 && i % 4 != part))
        continue;
      const int piece = tid + kThreads * i;
      const int row = row0 + piece / 8;
      const int column = 64 * pair + 8 * (piece % 8);
      s.x[i] = q8::BufferLoad16(x_buffer, 2U * static_cast<std::uint32_t>(row * a.k + column),
                                live && row < a.m && column < a.k);
    }
#pragma unroll
    for (int u = 0; u < kUnits; ++u) {
      if ((what & 2) == 0 || (part >= 0 && (kAPieces + u) % 4 != part))
        continue;
      const int group = kUnits * wave + u;
      const bool ok = live && group < live_groups;
      const std::uint32_t unit = static_cast<std::uint32_t>(group) * group_bytes +
                                 static_cast<std::uint32_t>(pair) * kUnit;
      s.w[u] = q8::BufferLoad16(w_buffer, unit + 16U * lane, ok);
      if constexpr (BF16)
        s.w2[u] = q8::BufferLoad16(w_buffer, unit + q8::kBf16HalfBytes + 16U * lane, ok);
      else
        s.scales[u] = q8::BufferLoad4(w_buffer, unit + kValueBytes + 4U * r16, ok);
    }
  };
  const auto store = [&](int stage, const Staging& sx, const Staging& s) {
    uint4* const a_tile = lds_a + stage * BM * 8;
    uint4* const b_tile = lds_b + stage * BN * 8;
#pragma unroll
    for (int i = 0; i < kAPieces; ++i) {
      const int piece = tid + kThreads * i;
      a_tile[Swizzled(piece / 8, piece % 8)] = sx.x[i];
    }
#pragma unroll
    for (int u = 0; u < kUnits; ++u) {
      const int row = 16 * (kUnits * wave + u) + r16;
      uint4 first, second;
      if constexpr (BF16) {
        first = s.w[u];
        second = s.w2[u];
      } else {
        first = Expand(s.w[u].x, s.w[u].y,
                       HalfValue(static_cast<std::uint16_t>(s.scales[u] & 0xFFFFU)));
        second = Expand(s.w[u].z, s.w[u].w,
                        HalfValue(static_cast<std::uint16_t>(s.scales[u] >> 16)));
      }
      b_tile[Swizzled(row, octet)] = first;
      b_tile[Swizzled(row, 4 + octet)] = second;
    }
  };

  const int wm = wave / WN;
  const int wn = wave % WN;
  const int lr = lane % 32;  // the operand row / column of this lane
  const int lk = lane / 32;  // its half of each 16-column reduction step
  F32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v)
        acc[i][j][v] = 0.0F;

  // The multiply of one LDS stage with the next stage's store spread over
  // its four 16-column reduction steps (measured 2-7 % faster on MI355X than
  // storing after the multiply).
  // With D >= 2 the loads of step `ahead` (into `later`, a free register
  // set) are issued a quarter at a time after each reduction step's
  // products, so that their issue overlaps the matrix cores' work instead
  // of holding every wave before it (ahead < 0: none).
  const auto compute_store = [&](int stage, int next, const Staging& sx, const Staging& s,
                                 int ahead_x, Staging& later_x, int ahead, Staging& later) {
    const uint4* const a_tile = lds_a + stage * BM * 8;
    const uint4* const b_tile = lds_b + stage * BN * 8;
    uint4* const a_next = lds_a + next * BM * 8;
    uint4* const b_next = lds_b + next * BN * 8;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int chunk = 2 * kk + lk;
      Bf16x8 af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = AsBf16x8(a_tile[Swizzled(TM * wm + 32 * i + lr, chunk)]);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bf[j] = AsBf16x8(b_tile[Swizzled(TN * wn + 32 * j + lr, chunk)]);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = Mfma32(af[i], bf[j], acc[i][j]);
      if (ahead >= 0) {
        fetch(ahead_x, later_x, kk, 1);
        fetch(ahead, later, kk, 2);
      }
#pragma unroll
      for (int i = kk; i < kAPieces; i += 4) {
        const int piece = tid + kThreads * i;
        a_next[Swizzled(piece / 8, piece % 8)] = sx.x[i];
      }
#pragma unroll
      for (int h = kk; h < 2 * kUnits; h += 4) {
        const int u = h / 2;
        const int row = 16 * (kUnits * wave + u) + r16;
        uint4 half;
        if constexpr (BF16) {
          half = h % 2 == 0 ? s.w[u] : s.w2[u];
        } else {
          const float scale = HalfValue(static_cast<std::uint16_t>(
              h % 2 == 0 ? s.scales[u] & 0xFFFFU : s.scales[u] >> 16));
          half = h % 2 == 0 ? Expand(s.w[u].x, s.w[u].y, scale)
                            : Expand(s.w[u].z, s.w[u].w, scale);
        }
        b_next[Swizzled(row, 4 * (h % 2) + octet)] = half;
      }
    }
  };

  // D register sets of panel units and DX = min(D, 2) of activation pieces
  // (L2-resident, their latency shorter): set q % D (q % DX) holds step q
  // from its fetch, D (DX) steps ahead, until its store; LDS stage q % 2
  // holds step q while it is multiplied. The stores after the last step
  // write zeros into a stage no later step reads.
  constexpr int DX = D < 2 ? D : 2;
  Staging staged_x[DX];
  Staging staged[D];
#pragma unroll
  for (int d = 0; d < DX; ++d)
    fetch(d, staged_x[d], -1, 1);
#pragma unroll
  for (int d = 0; d < D; ++d)
    fetch(d, staged[d], -1, 2);
  store(0, staged_x[0], staged[0]);
  __syncthreads();
  // U steps per iteration (a multiple of 2 and of D), so that every set and
  // stage index is a constant.
  constexpr int U = D % 2 == 0 ? D : 2 * D;
  for (int p = 0; p < steps; p += U) {
#pragma unroll
    for (int d = 0; d < U; ++d) {
      const int q = p + d;
      if (q >= steps)
        break;
      if constexpr (D >= 2) {
        compute_store(d % 2, 1 - d % 2, staged_x[(d + 1) % DX], staged[(d + 1) % D], q + DX,
                      staged_x[d % DX], q + D, staged[d % D]);
      } else {
        fetch(q + 1, staged_x[0], -1, 1);
        fetch(q + 1, staged[0], -1, 2);
        compute_store(d % 2, 1 - d % 2, staged_x[0], staged[0], -1, staged_x[0], -1, staged[0]);
      }
      __syncthreads();
    }
  }

  // Epilogue: element v of tile (i, j) is row 8 (v / 4) + 4 lk + v % 4 and
  // column lr of the tile. One uniform branch picks the output; each
  // element is then one buffer store at the lane's offset plus a constant
  // of v (accumulation: one load, issued for the whole 32 x 32 tile before
  // its stores). Rows past m lie past the buffer, whose range check drops
  // them.
  const std::size_t count = static_cast<std::size_t>(a.m) * a.n;
  const auto emit = [&](auto kind, void* base) {
    constexpr int K = decltype(kind)::value;  // 0 float32, 1 bf16, 2 float32 +=
    constexpr std::uint32_t width = K == 1 ? 2 : 4;
    const __amdgpu_buffer_rsrc_t out =
        q8::BufferOf(base, static_cast<std::uint32_t>(count * width));
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int column = 16 * group0 + TN * wn + 32 * j + lr;
      if (column >= a.n)
        continue;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const std::uint32_t lane_bytes =
            width * static_cast<std::uint32_t>((row0 + TM * wm + 32 * i + 4 * lk) * a.n + column);
        std::uint32_t offset[16];
#pragma unroll
        for (int v = 0; v < 16; ++v)
          offset[v] = lane_bytes + width * static_cast<std::uint32_t>((8 * (v / 4) + v % 4) * a.n);
        if constexpr (K == 2) {
          float prior[16];
#pragma unroll
          for (int v = 0; v < 16; ++v)
            prior[v] = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(out, static_cast<int>(offset[v]), 0, 0));
#pragma unroll
          for (int v = 0; v < 16; ++v)
            __builtin_amdgcn_raw_buffer_store_b32(
                __builtin_bit_cast(std::uint32_t, prior[v] + acc[i][j][v]), out,
                static_cast<int>(offset[v]), 0, 0);
        } else {
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            // The element as a value first: hipcc's bit cast of a vector
            // element taken in place reads element 0.
            const float value = acc[i][j][v];
            if constexpr (K == 1)
              __builtin_amdgcn_raw_buffer_store_b16(q8::Bf16Fast(value), out,
                                                    static_cast<int>(offset[v]), 0, 0);
            else
              __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(std::uint32_t, value), out,
                                                    static_cast<int>(offset[v]), 0, 0);
          }
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
  for (int j = 0; j < FN; ++j) {
    const int column = 16 * group0 + TN * wn + 32 * j + lr;
    if (column >= a.n)
      continue;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = row0 + TM * wm + 32 * i + 8 * (v / 4) + 4 * lk + v % 4;
        if (row >= a.m)
          continue;
        const std::size_t at = static_cast<std::size_t>(row) * a.n + column;
        if (a.splits > 1)
          a.partials[static_cast<std::size_t>(split) * count + at] = acc[i][j][v];
        else if (a.y_bf16 != nullptr)
          a.y_bf16[at] = q8::Bf16Fast(acc[i][j][v]);
        else
          a.y[at] = a.accumulate ? a.y[at] + acc[i][j][v] : acc[i][j][v];
      }
  }
}

/// y (+)= the splits' partial sums added in split order, or their bf16
/// rounding; four consecutive elements per thread (n % 4 == 0), else one.
__global__ __launch_bounds__(256) void AddSplitsKernel(GemmArgs a) {
  const std::size_t count = static_cast<std::size_t>(a.m) * a.n;
  const std::size_t first = (static_cast<std::size_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (first >= count)
    return;
  const int width = a.n % 4 == 0 ? 4 : 1;
  for (int v = 0; v < 4; v += width) {
    const std::size_t at = first + v;
    if (at >= count)
      break;
    float sum[4] = {0.0F, 0.0F, 0.0F, 0.0F};
    for (int s = 0; s < a.splits; ++s) {
      const float* part = a.partials + s * count + at;
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

template<int BM, int BN, int WM, int WN, int D>
struct Shape {
  static constexpr int kBm = BM;
  static constexpr int kBn = BN;
  static constexpr int kThreads = WM * WN * kWave;
  static constexpr std::size_t kLds = 2 * (BM + BN) * 8 * sizeof(uint4);
  template<int MODE>
  static void Launch(const GemmArgs& args, hipStream_t stream) {
    GemmKernel<BM, BN, WM, WN, D, MODE>
        <<<args.m_tiles * args.n_tiles * args.splits, kThreads, kLds, stream>>>(args);
  }
  static bool Allow() {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(GemmKernel<BM, BN, WM, WN, D, 1>),
                               hipFuncAttributeMaxDynamicSharedMemorySize,
                               static_cast<int>(kLds)) == hipSuccess &&
           hipFuncSetAttribute(reinterpret_cast<const void*>(GemmKernel<BM, BN, WM, WN, D, 2>),
                               hipFuncAttributeMaxDynamicSharedMemorySize,
                               static_cast<int>(kLds)) == hipSuccess;
  }
};

// The 256 x 256 tile's 128 accumulators per lane leave registers for one
// prefetched step only.
using Big = Shape<256, 256, 2, 4, 1>;    // 8 waves of 128 x 64
using Wide = Shape<128, 256, 2, 4, 2>;   // 8 waves of 64 x 64
using Small = Shape<128, 128, 2, 2, 2>;  // 4 waves of 64 x 64
using Tall = Shape<256, 128, 4, 2, 3>;   // 8 waves of 64 x 64, three steps prefetched
using BigDeep = Shape<256, 256, 2, 4, 2>;
using Narrow = Shape<128, 64, 2, 1, 2>;  // 2 waves of 64 x 64

/// Whether the kernels' LDS sizes are allowed (set once per process).
bool Prepare() {
  static const bool ready = Big::Allow() && Wide::Allow() && Small::Allow() &&
                            Tall::Allow() && BigDeep::Allow() && Narrow::Allow();
  return ready;
}

}  // namespace

namespace {

constexpr int kShapeTiles[6][2] = {{256, 256}, {128, 256}, {128, 128},
                                   {256, 128}, {256, 256}, {128, 64}};

}  // namespace

GemmPlan PlanGemm(std::size_t m, std::size_t k, std::size_t n, std::size_t partial_floats,
                  int shape, int splits) {
  GemmPlan plan;
  const auto tiles = [&](int bm, int bn) {
    return static_cast<int>(((m + bm - 1) / bm) * ((n + bn - 1) / bn));
  };
  if (shape >= 0) {
    plan.shape = shape;
    plan.bm = kShapeTiles[shape][0];
    plan.bn = kShapeTiles[shape][1];
    plan.tiles = tiles(plan.bm, plan.bn);
    plan.splits = splits;
    return plan;
  }
  // Measured on MI355X over m 129..1024, k 2048, n 2048..16384: 256 x 256
  // tiles (two steps prefetched) once they fill three quarters of the
  // compute units (768 x 2048 x 16384: 70.5 -> 58.8 us against 256 x 128
  // tiles), else 256 x 128 tiles, k split while the grid has fewer than
  // 192 workgroups and the partial sums fit the scratch.
  if (tiles(256, 256) >= 192) {
    plan.shape = 4;
  } else {
    plan.shape = 3;
  }
  plan.bm = kShapeTiles[plan.shape][0];
  plan.bn = kShapeTiles[plan.shape][1];
  plan.tiles = tiles(plan.bm, plan.bn);
  plan.splits = 1;
  const std::size_t pairs = q8::Pairs(k);
  const std::size_t room = partial_floats < kMaxSplitFloats ? partial_floats : kMaxSplitFloats;
  while (plan.tiles * plan.splits < 192 && pairs >= 16U * plan.splits &&
         2 * plan.splits * m * n <= room)
    plan.splits *= 2;
  return plan;
}

// From 512 rows over 6144 or more columns, and from 384 rows over 16384 or
// more (384 x 2048 x 16384: 44.5 -> 39.1 us against the tiled kernel).
bool UseGemm(std::size_t m, std::size_t n) {
  return (m >= 512 && n >= 6144) || (m >= 384 && n >= 16384);
}

int RunGemm(const Bf16* x, const void* w, float* y, Bf16* y_bf16, std::size_t m, std::size_t k,
            std::size_t n, bool accumulate, bool bf16_weights, float* partials,
            std::size_t partial_floats, hipStream_t stream, int shape, int splits) {
  if (!Prepare())
    return Fail(VX_HIP_ERROR, "prefill product: LDS size not allowed");
  if (shape >= 6 || (shape >= 0 && (splits < 1 || splits > 64)))
    return Fail(VX_UNSUPPORTED, "prefill product: no such plan");
  if (shape >= 0 && splits > 1 &&
      (partials == nullptr || static_cast<std::size_t>(splits) * m * n > partial_floats))
    return Fail(VX_BAD_ARG, "prefill product: the split needs more scratch");
  const GemmPlan plan = PlanGemm(m, k, n, partials != nullptr ? partial_floats : 0, shape, splits);
  GemmArgs args{};
  args.x = x;
  args.w = static_cast<const std::uint8_t*>(w);
  args.y = y;
  args.y_bf16 = y_bf16;
  args.m = static_cast<int>(m);
  args.k = static_cast<int>(k);
  args.n = static_cast<int>(n);
  args.pairs = static_cast<int>(q8::Pairs(k));
  args.groups = static_cast<int>(q8::Groups(n));
  args.m_tiles = static_cast<int>((m + plan.bm - 1) / plan.bm);
  args.n_tiles = static_cast<int>((n + plan.bn - 1) / plan.bn);
  args.accumulate = accumulate ? 1 : 0;
  args.splits = plan.splits;
  args.pairs_per_split = (args.pairs + plan.splits - 1) / plan.splits;
  args.partials = partials;
  const auto launch = [&](auto shape) {
    if (bf16_weights)
      decltype(shape)::template Launch<2>(args, stream);
    else
      decltype(shape)::template Launch<1>(args, stream);
  };
  switch (plan.shape) {
    case 0: launch(Big{}); break;
    case 1: launch(Wide{}); break;
    case 3: launch(Tall{}); break;
    case 4: launch(BigDeep{}); break;
    case 5: launch(Narrow{}); break;
    default: launch(Small{}); break;
  }
  if (plan.splits > 1) {
    const std::size_t quads = (m * n + 3) / 4;
    AddSplitsKernel<<<static_cast<unsigned>((quads + 255) / 256), 256, 0, stream>>>(args);
  }
  return LaunchStatus(bf16_weights ? "bf16 prefill product" : "q8 prefill product");
}

}  // namespace vx
