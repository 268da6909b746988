// Q8_0 x bfloat16 products on gfx950's matrix cores.
//
// Up to 128 activation rows ("skinny", the memory-bound case: the DiT's 22
// rows, decoding's 1) the Q8_0 arithmetic stays exact: each weight pair of
// blocks is converted int8 -> bf16 exactly in registers, each 32-column
// block is one v_mfma_f32_16x16x32_bf16 from zero (a float32 block sum), and
// acc = fmaf(f16 scale, block sum, acc) applies the block's scale; the
// arithmetic of kernels/wmma_products.hip:192-215 on wave64 MFMA.
//
// Work split: a workgroup owns `rg` row groups (16 weight rows each) and a
// range of column pairs; its waves split that range and every wave
// streams all `rg` row groups, so an activation fragment, loaded once from
// L2, feeds rg x 2 MFMAs. The waves' partial sums meet in LDS and are added
// in wave order; a product split over several workgroups along k stores
// per-split partials and the last workgroup of a tile (an atomic counter)
// adds them in split order and resets the counter. No float atomics: the
// result is the same on every run.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "common.hpp"
#include "products.hpp"
#include "q8.hpp"
#include "q8_tile.hpp"

namespace vx {
namespace {

using q8::AsBf16x8;
using q8::Bf16x8;
using q8::F32x4;
using q8::Int8x8ToBf16;
using q8::kUnitBytes;
using q8::kValueBytes;
using q8::Mfma16x16x32;

// Workgroups of up to 16 waves (1024 threads) split a tile's pairs for the
// smaller register footprints; the others take up to 8 waves.
constexpr int kMaxThreads = 1024;

constexpr int ThreadsFor(int mt, int rg) { return mt * rg <= 2 ? 1024 : 512; }

struct SkinnyArgs {
  const Bf16* x;
  const std::uint8_t* w;
  float* y;
  Bf16* y_bf16;  // non-null: bf16 output (no accumulation)
  float* partials;
  unsigned* counters;
  int m, k, n;
  int pairs;
  int pairs_per_split;
  int pairs_per_wave;
  int splits;
  int accumulate;
};

template<int MT, int RG>
struct Stage {
  uint4 w[RG];
  std::uint32_t scales[RG];
  uint4 a[MT][2];
};

template<int MT, int RG, int kThreads>
__global__ __launch_bounds__(kThreads) void SkinnyKernel(SkinnyArgs args) {
  extern __shared__ float reduce[];  // [waves][RG * MT][4][64]
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int waves = blockDim.x / kWave;
  const int groups = (args.n + 15) / 16;
  const int first_group = static_cast<int>(blockIdx.x) * RG;
  const int split = static_cast<int>(blockIdx.y);
  const int split_begin = split * args.pairs_per_split;
  const int split_end = min(split_begin + args.pairs_per_split, args.pairs);
  const int begin = split_begin + wave * args.pairs_per_wave;
  const int end = min(begin + args.pairs_per_wave, split_end);
  const int r16 = lane % 16;
  const int octet = lane / 16;
  const int k_blocks = args.k / 32;

  // The lane's bytes in the units of its row groups (groups past the
  // matrix re-read the last one; their results are dropped).
  const std::uint8_t* unit[RG];
#pragma unroll
  for (int r = 0; r < RG; ++r)
    unit[r] = args.w +
              static_cast<std::size_t>(min(first_group + r, groups - 1)) *
                  args.pairs * kUnitBytes;
  const Bf16* x_row[MT];
  bool row_ok[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int row = 16 * t + r16;
    row_ok[t] = row < args.m;
    x_row[t] = args.x + static_cast<std::size_t>(row_ok[t] ? row : 0) * args.k +
               8 * octet;
  }

  F32x4 acc[RG][MT];
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int t = 0; t < MT; ++t)
      acc[r][t] = F32x4{0.0F, 0.0F, 0.0F, 0.0F};

  const auto load = [&](int pair, Stage<MT, RG>& s) {
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      const std::uint8_t* u = unit[r] + static_cast<std::size_t>(pair) * kUnitBytes;
      s.w[r] = *reinterpret_cast<const uint4*>(u + 16 * lane);
      s.scales[r] =
          *reinterpret_cast<const std::uint32_t*>(u + kValueBytes + 4 * r16);
    }
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if (row_ok[t] && 2 * pair + h < k_blocks)
          s.a[t][h] = *reinterpret_cast<const uint4*>(x_row[t] + 64 * pair + 32 * h);
        else
          s.a[t][h] = uint4{0U, 0U, 0U, 0U};
      }
  };
  const auto compute = [&](const Stage<MT, RG>& s) {
    const F32x4 zero{0.0F, 0.0F, 0.0F, 0.0F};
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      const Bf16x8 b0 = Int8x8ToBf16(s.w[r].x, s.w[r].y);
      const Bf16x8 b1 = Int8x8ToBf16(s.w[r].z, s.w[r].w);
      const float s0 = HalfValue(static_cast<std::uint16_t>(s.scales[r] & 0xFFFFU));
      const float s1 = HalfValue(static_cast<std::uint16_t>(s.scales[r] >> 16));
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const F32x4 sum0 = Mfma16x16x32(AsBf16x8(s.a[t][0]), b0, zero);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[r][t][i] = fmaf(s0, sum0[i], acc[r][t][i]);
        const F32x4 sum1 = Mfma16x16x32(AsBf16x8(s.a[t][1]), b1, zero);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[r][t][i] = fmaf(s1, sum1[i], acc[r][t][i]);
      }
    }
  };

  // Two pairs in flight: the next pair's loads are issued before this
  // pair's products.
  Stage<MT, RG> even, odd;
  if (begin < end)
    load(begin, even);
  for (int pair = begin; pair < end; pair += 2) {
    if (pair + 1 < end)
      load(pair + 1, odd);
    compute(even);
    if (pair + 1 >= end)
      break;
    if (pair + 2 < end)
      load(pair + 2, even);
    compute(odd);
  }

  // Writes one finished 16 x 16 fragment (rows 16 t + 4 (lane / 16) + i,
  // column 16 g + lane % 16).
  const auto emit = [&](int r, int t, const float* v) {
    const int column = 16 * (first_group + r) + r16;
    if (first_group + r >= groups || column >= args.n)
      return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * t + 4 * octet + i;
      if (row >= args.m)
        continue;
      const std::size_t at = static_cast<std::size_t>(row) * args.n + column;
      if (args.splits > 1)
        args.partials[static_cast<std::size_t>(split) * args.m * args.n + at] =
            v[i];
      else if (args.y_bf16 != nullptr)
        args.y_bf16[at] = Bf16Bits(v[i]);
      else
        args.y[at] = args.accumulate ? args.y[at] + v[i] : v[i];
    }
  };

  if (waves == 1) {
#pragma unroll
    for (int r = 0; r < RG; ++r)
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        float v[4] = {acc[r][t][0], acc[r][t][1], acc[r][t][2], acc[r][t][3]};
        emit(r, t, v);
      }
  } else {
    constexpr int kFragments = RG * MT;
    float* mine = reduce + static_cast<std::size_t>(wave) * kFragments * 4 * kWave;
#pragma unroll
    for (int r = 0; r < RG; ++r)
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          mine[((r * MT + t) * 4 + i) * kWave + lane] = acc[r][t][i];
    __syncthreads();
    for (int f = wave; f < kFragments; f += waves) {
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float total = reduce[(f * 4 + i) * kWave + lane];
        for (int w = 1; w < waves; ++w)
          total += reduce[((static_cast<std::size_t>(w) * kFragments + f) * 4 + i) *
                              kWave + lane];
        v[i] = total;
      }
      emit(f / MT, f % MT, v);
    }
  }
  if (args.splits == 1)
    return;

  // Split along k: the last workgroup of this tile adds the partials. The
  // barrier orders every wave's partial stores before thread 0's release
  // (one L2 write-back per workgroup); only the last workgroup acquires
  // (one L2 invalidation per tile), and its barrier orders the acquire
  // before every wave's loads.
  __shared__ unsigned last;
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned previous = __hip_atomic_fetch_add(
        args.counters + blockIdx.x, 1U, __ATOMIC_RELEASE,
        __HIP_MEMORY_SCOPE_AGENT);
    last = previous + 1 == static_cast<unsigned>(args.splits) ? 1U : 0U;
    if (last != 0)
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
  if (last == 0)
    return;
  const int columns = 16 * RG;
  const int elements = columns * 16 * MT;
  for (int e = threadIdx.x; e < elements; e += blockDim.x) {
    const int column = 16 * first_group + e % columns;
    const int row = e / columns;
    if (column >= args.n || row >= args.m)
      continue;
    const std::size_t at = static_cast<std::size_t>(row) * args.n + column;
    const std::size_t stride = static_cast<std::size_t>(args.m) * args.n;
    float total = args.partials[at];
    for (int s = 1; s < args.splits; ++s)
      total += args.partials[s * stride + at];
    if (args.y_bf16 != nullptr)
      args.y_bf16[at] = Bf16Bits(total);
    else
      args.y[at] = args.accumulate ? args.y[at] + total : total;
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(args.counters + blockIdx.x, 0U, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

template<int MT, int RG>
void LaunchSkinny(const SkinnyArgs& args, const ProductPlan& plan,
                  hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(plan.tiles),
                  static_cast<unsigned>(plan.splits));
  const std::size_t shared =
      plan.waves > 1 ? static_cast<std::size_t>(plan.waves) * RG * MT * 4 *
                           kWave * sizeof(float)
                     : 0;
  SkinnyKernel<MT, RG, ThreadsFor(MT, RG)>
      <<<grid, plan.waves * kWave, shared, stream>>>(args);
}

using Launcher = void (*)(const SkinnyArgs&, const ProductPlan&, hipStream_t);

template<int MT>
Launcher PickRg(int rg) {
  if constexpr (MT * 4 <= 8) {
    if (rg == 4)
      return LaunchSkinny<MT, 4>;
  }
  if constexpr (MT * 2 <= 8) {
    if (rg == 2)
      return LaunchSkinny<MT, 2>;
  }
  if (rg == 1)
    return LaunchSkinny<MT, 1>;
  return nullptr;
}

Launcher PickLauncher(int mt, int rg) {
  switch (mt) {
    case 1: return PickRg<1>(rg);
    case 2: return PickRg<2>(rg);
    case 3: return PickRg<3>(rg);
    case 4: return PickRg<4>(rg);
    case 5: return PickRg<5>(rg);
    case 6: return PickRg<6>(rg);
    case 7: return PickRg<7>(rg);
    case 8: return PickRg<8>(rg);
    default: return nullptr;
  }
}

// ---- the one-pass engine on row-major activations ---------------------------

template<int MT, int RG, int PW, int JR, q8::Weights WK, int NW = 0>
void LaunchEngine(const q8::TileArgs& args, int tiles, int waves,
                  hipStream_t stream) {
  const std::size_t shared = q8::EngineShared(MT, RG, waves, q8::ASource::kRowMajor);
  q8::EngineKernel<MT, RG, q8::ASource::kRowMajor, q8::Output::kStore, PW, JR, WK, NW>
      <<<tiles, waves * kWave, shared, stream>>>(args);
}

using EngineLauncher = void (*)(const q8::TileArgs&, int, int, hipStream_t);

/// Up to 64 rows (a workgroup's block; `m` here is the block's rows) the
/// engine stages the rows through LDS in JR load groups of 8 rows, JR the
/// fewest that cover them.
template<int MT, int RG, int PW, q8::Weights WK, int NW = 0>
EngineLauncher EngineJr(int m) {
  if constexpr (q8::StagesRows(q8::ASource::kRowMajor, MT)) {
    if (m <= 16 * MT - 8)
      return LaunchEngine<MT, RG, PW, 2 * MT - 1, WK, NW>;
  }
  return LaunchEngine<MT, RG, PW, 2 * MT, WK, NW>;
}

/// Pairs in flight per wave (`pw`, kMaxPairsInFlight): one 16-row tile
/// (m <= 16) takes up to four, so that the decode shapes' long reductions
/// (k = 6144: 96 pairs over 16 waves) need few memory round trips; 32 rows
/// take one at most (measured fastest on MI355X at the M = 22 sweep shapes,
/// where more pairs in flight cost registers).
template<int MT, int RG, q8::Weights WK>
EngineLauncher EnginePw(int pw, int m) {
  if constexpr (MT == 1) {
    switch (pw) {
      case 2: return EngineJr<MT, RG, 2, WK>(m);
      case 3: return EngineJr<MT, RG, 3, WK>(m);
      case 4: return EngineJr<MT, RG, 4, WK>(m);
      default: break;
    }
  }
  if constexpr (MT == 2 && RG == 1) {
    if (pw == 2)
      return EngineJr<MT, RG, 2, WK>(m);
  }
  if constexpr (MT == 3 && WK == q8::Weights::kQ8) {
    if (pw == 2)
      return EngineJr<MT, RG, 2, WK>(m);
  }
  return pw == 1 ? EngineJr<MT, RG, 1, WK>(m) : nullptr;
}

template<int MT, q8::Weights WK>
EngineLauncher EngineRg(int rg, int pw, int m) {
  if constexpr (MT * 4 <= 16) {
    if (rg == 4)
      return EnginePw<MT, 4, WK>(pw, m);
  }
  if constexpr (MT * 2 <= 8) {
    if (rg == 2)
      return EnginePw<MT, 2, WK>(pw, m);
  }
  if (rg == 1)
    return EnginePw<MT, 1, WK>(pw, m);
  return nullptr;
}

/// Eight-wave workgroups of one or two row groups for wide products of
/// 17-32 rows (PlanEngine's 512-workgroup plans).
template<q8::Weights WK>
EngineLauncher EngineEight(int rg, int pw, int m) {
  if (pw == 1 && rg == 1)
    return EngineJr<2, 1, 1, WK, 8>(m);
  if (pw == 1 && rg == 2)
    return EngineJr<2, 2, 1, WK, 8>(m);
  if (pw == 2 && rg == 2)
    return EngineJr<2, 2, 2, WK, 8>(m);
  return nullptr;
}

template<q8::Weights WK>
EngineLauncher PickEngineFor(int mt, int rg, int pw, int m, int waves) {
  if (mt == 2 && waves * kWave != q8::EngineThreads(mt, rg))
    return waves == 8 ? EngineEight<WK>(rg, pw, m) : nullptr;
  switch (mt) {
    case 1: return EngineRg<1, WK>(rg, pw, m);
    case 2: return EngineRg<2, WK>(rg, pw, m);
    case 3: return EngineRg<3, WK>(rg, pw, m);
    case 4: return EngineRg<4, WK>(rg, pw, m);
    case 5: return EngineRg<5, WK>(rg, pw, m);
    case 6: return EngineRg<6, WK>(rg, pw, m);
    case 7: return EngineRg<7, WK>(rg, pw, m);
    case 8: return EngineRg<8, WK>(rg, pw, m);
    default: return nullptr;
  }
}

// ---- forced engine plans (tuning) ----------------------------------------------

template<int RG, int PW, int NW, int JR>
void LaunchTuned(const q8::TileArgs& args, int tiles, hipStream_t stream) {
  const std::size_t shared = q8::EngineShared(2, RG, NW, q8::ASource::kRowMajor);
  q8::EngineKernel<2, RG, q8::ASource::kRowMajor, q8::Output::kStore, PW, JR, q8::Weights::kQ8,
                   NW><<<tiles * args.row_blocks, NW * kWave, shared, stream>>>(args);
}

using TunedLauncher = void (*)(const q8::TileArgs&, int, hipStream_t);

template<int RG, int PW, int NW>
TunedLauncher TunedJr(int m) {
  return m <= 24 ? LaunchTuned<RG, PW, NW, 3> : LaunchTuned<RG, PW, NW, 4>;
}

template<int RG, int PW>
TunedLauncher TunedNw(int waves, int m) {
  switch (waves) {
    case 4: return TunedJr<RG, PW, 4>(m);
    case 8: return TunedJr<RG, PW, 8>(m);
    case 16:
      if constexpr (RG <= 2)
        return TunedJr<RG, PW, 16>(m);
      return nullptr;
    default: return nullptr;
  }
}

template<int RG>
TunedLauncher TunedPw(int pw, int waves, int m) {
  switch (pw) {
    case 1: return TunedNw<RG, 1>(waves, m);
    case 2: return TunedNw<RG, 2>(waves, m);
    default: return nullptr;
  }
}

TunedLauncher PickTuned(int rg, int pw, int waves, int m) {
  switch (rg) {
    case 1: return TunedPw<1>(pw, waves, m);
    case 2: return TunedPw<2>(pw, waves, m);
    case 4: return TunedPw<4>(pw, waves, m);
    default: return nullptr;
  }
}

/// bf16 rows [n][k] are read by the staged engine only (m <= 32); the
/// expanded Q8_0 arithmetic runs in blocks of 64 rows only (mt = 4).
EngineLauncher PickEngine(int mt, int rg, int pw, int m, int waves, q8::Weights kind) {
  switch (kind) {
    case q8::Weights::kQ8Expanded:
      if (mt != 4 || pw != 1 || waves * kWave != q8::EngineThreads(4, rg))
        return nullptr;
      return rg == 1   ? EngineJr<4, 1, 1, q8::Weights::kQ8Expanded>(m)
             : rg == 2 ? EngineJr<4, 2, 1, q8::Weights::kQ8Expanded>(m)
                       : nullptr;
    case q8::Weights::kQ8: return PickEngineFor<q8::Weights::kQ8>(mt, rg, pw, m, waves);
    case q8::Weights::kBf16: return PickEngineFor<q8::Weights::kBf16>(mt, rg, pw, m, waves);
    case q8::Weights::kBf16Rows:
      if (mt == 2 && waves * kWave != q8::EngineThreads(mt, rg))
        return waves == 8 ? EngineEight<q8::Weights::kBf16Rows>(rg, pw, m) : nullptr;
      if (mt == 1)
        return EngineRg<1, q8::Weights::kBf16Rows>(rg, pw, m);
      if (mt == 2)
        return EngineRg<2, q8::Weights::kBf16Rows>(rg, pw, m);
      return nullptr;
  }
  return nullptr;
}

constexpr int kMaxPairsInFlight = 4;

/// Engine plan in blocks of at most 64 rows (four 16-row tiles), one or two
/// row groups per workgroup of 8 waves.
ProductPlan PlanRowBlocks(std::size_t m, std::size_t k, std::size_t n) {
  ProductPlan plan;
  plan.engine = true;
  plan.mt = 4;
  plan.row_blocks = static_cast<int>((m + 63) / 64);
  const int groups = static_cast<int>(q8::Groups(n));
  const int pairs = static_cast<int>(q8::Pairs(k));
  plan.rg = groups <= 256 ? 1 : 2;
  plan.tiles = (groups + plan.rg - 1) / plan.rg;
  plan.waves = q8::EngineThreads(plan.mt, plan.rg) / kWave;
  plan.splits = 1;
  plan.pairs_per_split = pairs;
  plan.pairs_per_wave = (pairs + plan.waves - 1) / plan.waves;
  return plan;
}

/// Engine plan: up to 256 row groups take one per workgroup; wider products
/// share each activation fragment over 2 or 4 row groups (fewer workgroups
/// read the activations). Waves split the pairs, up to 16 (8 for the larger
/// register footprints).
ProductPlan PlanEngine(std::size_t m, std::size_t k, std::size_t n, q8::Weights kind) {
  ProductPlan plan;
  plan.mt = static_cast<int>((m + 15) / 16);
  if ((plan.mt == 3 || plan.mt == 4) && kind == q8::Weights::kQ8 && q8::Groups(n) <= 256) {
    // 33-64 rows over at most 256 row groups: two blocks of at most 32
    // rows, each the plan of its rows (the blocks of a tile `tiles`
    // workgroups apart, on one compute die where tiles is a multiple of 8,
    // so that its L2 serves the weights to both). Measured on MI355X:
    // (1024, 3072) 5.12 -> 4.84 us at 44 rows, 5.54 -> 5.21 us at 64; wider
    // products measured slower so ((2048, 16384) 16.5 -> 18.2 us at 44).
    ProductPlan half = PlanEngine((m + 1) / 2, k, n, kind);
    half.row_blocks *= 2;
    return half;
  }
  if (plan.mt > 4 && kind != q8::Weights::kBf16Rows) {
    // More than 64 rows: blocks of at most 64 rows, four 16-row tiles each,
    // staged per wave from whole-line loads; the blocks of a tile lie
    // `tiles` workgroups apart, a multiple of 8 for the sweep's widths, on
    // one compute die, whose L2 serves each weight row group to both.
    // Measured on MI355X at 100 and 128 rows: (1024, 3072) 11.1 -> 7.4 us,
    // (1024, 8192) 21.1 -> 10.6 us, (2048, 2048) 14.0 -> 7.6 us against the
    // engine on all 128 rows; (2048, 16384) 29.2 -> 28.8 us against the
    // LDS-tiled kernel.
    ProductPlan blocks = PlanRowBlocks(m, k, n);
    if (kind == q8::Weights::kQ8 && q8::Groups(n) > 256) {
      // Exact arithmetic over more than 256 row groups: four per workgroup
      // (measured on MI355X at 128 rows: (1024, 8192) 10.95 -> 10.65 us,
      // (2048, 16384) 29.9 -> 29.0 us against two).
      blocks.rg = 4;
      blocks.tiles = static_cast<int>((q8::Groups(n) + 3) / 4);
      blocks.waves = q8::EngineThreads(blocks.mt, blocks.rg) / kWave;
      blocks.pairs_per_wave = (blocks.pairs_per_split + blocks.waves - 1) / blocks.waves;
    }
    return blocks;
  }
  plan.engine = true;
  const int groups = static_cast<int>(q8::Groups(n));
  const int pairs = static_cast<int>(q8::Pairs(k));
  // Up to 8 rows (one staged load group) the activations cost little to
  // re-read: one row group per workgroup spreads wide products over more
  // compute units (measured on MI355X at 1 and 5 rows, n 12288 and 16384).
  // 33-64 rows over more than 512 row groups keep four (150-178 VGPRs in
  // 8-wave workgroups, no spill): (2048, 16384) 15.4 -> 14.4 us at 44
  // rows, 17.9 -> 16.6 us at 64, measured on MI355X against two.
  int rg = (m <= 8 || groups <= 256) ? 1 : groups <= 512 ? 2 : 4;
  while (rg > 1 && rg * plan.mt > 16)
    rg /= 2;
  plan.rg = rg;
  plan.tiles = (groups + rg - 1) / rg;
  plan.waves = q8::EngineThreads(plan.mt, rg) / kWave;  // idle waves add zeros
  // Few tiles: row blocks (each workgroup loads its rows' activations only)
  // fill the compute units; tiles a multiple of 8 keep a tile's blocks on
  // one compute die. Measured on MI355X for the (2048, 2048) M=22 shape.
  plan.row_blocks = 1;
  while (plan.tiles % 8 == 0 && plan.row_blocks < 4 && plan.tiles * 2 * plan.row_blocks <= 256 &&
         static_cast<int>(m) >= 10 * plan.row_blocks)
    plan.row_blocks *= 2;
  // Each workgroup stages and multiplies its block's rows only: the tiles
  // (and RunSkinny's load groups) follow the block's rows, not m's.
  // Measured on MI355X at (2048, 2048): 22 rows 4.80 -> 4.36 us, 44 rows
  // 6.67 -> 5.16 us, 64 rows 7.31 -> 5.49 us.
  const int block_tiles =
      static_cast<int>((m + plan.row_blocks - 1) / plan.row_blocks + 15) / 16;
  if (block_tiles < plan.mt) {
    plan.mt = block_tiles;
    plan.waves = q8::EngineThreads(plan.mt, plan.rg) / kWave;
  }
  if (plan.mt == 2 && groups >= 512 && kind == q8::Weights::kQ8) {
    // Wide Q8_0 products of 17-32 rows: about 512 workgroups of 8 waves
    // (two per compute unit), the fewest row groups that keep them at most
    // 512 (measured on MI355X at M=22: (1024, 8192) 5.49 -> 5.19 us with
    // one row group instead of two in 16-wave workgroups; (2048, 16384)
    // the same 11.0-11.1 us with two row groups as with four). bf16
    // weights keep the 16-wave plans: (1024, 8192) measured 6.3 -> 6.7 us
    // on panels and 7.5 -> 7.6 us on rows with these.
    plan.rg = groups <= 512 ? 1 : groups <= 1024 ? 2 : 4;
    plan.tiles = (groups + plan.rg - 1) / plan.rg;
    plan.waves = 8;
    plan.row_blocks = 1;
    // Two row groups over four or more pairs per wave: two pairs in
    // flight ((2048, 16384): 11.04 -> 10.92 us).
    if (plan.rg == 2 && pairs >= 4 * plan.waves)
      plan.pw = 2;
  } else if (plan.mt == 2 && plan.rg == 1 && pairs >= 2 * plan.waves && kind == q8::Weights::kQ8) {
    // One row group, two or more pairs per 16-wave workgroup's wave: two in
    // flight ((2048, 2048) with two row blocks: 4.79 -> 4.69 us).
    plan.pw = 2;
  }
  if (plan.mt == 3 && kind == q8::Weights::kQ8 && pairs >= 2 * plan.waves) {
    // 33-48 rows over more than 256 row groups (one block of three tiles):
    // two pairs in flight per wave (measured on MI355X at 44 rows:
    // (1024, 8192) 6.81 -> 6.44 us, (2048, 16384) 14.36 -> 14.02 us; the
    // same at 64 rows in blocks of four tiles measured slower).
    plan.pw = 2;
  }
  plan.splits = 1;
  plan.pairs_per_split = pairs;
  plan.pairs_per_wave = (pairs + plan.waves - 1) / plan.waves;
  if (plan.mt == 1) {
    // Passes of equal length, at most four pairs (two with four row groups)
    // in flight per wave.
    const int most = std::min(kMaxPairsInFlight, 8 / rg);
    const int passes = (plan.pairs_per_wave + most - 1) / most;
    plan.pw = (plan.pairs_per_wave + passes - 1) / passes;
  }
  return plan;
}

}  // namespace

int MaxWaves(int mt, int rg) { return ThreadsFor(mt, rg) / kWave; }

int MaxRowGroups(int mt) {
  if (mt * 4 <= 8)
    return 4;
  if (mt * 2 <= 8)
    return 2;
  return 1;
}

ProductPlan PlanSkinny(std::size_t m, std::size_t k, std::size_t n,
                       std::size_t scratch_floats,
                       std::size_t scratch_counters, int rg, int waves,
                       int splits, q8::Weights kind) {
  if (rg <= 0 && waves <= 0 && splits <= 0)
    return PlanEngine(m, k, n, kind);
  ProductPlan plan;
  plan.mt = static_cast<int>((m + 15) / 16);
  const int groups = static_cast<int>(q8::Groups(n));
  const int pairs = static_cast<int>(q8::Pairs(k));
  if (rg <= 0) {
    // Wide products reuse each activation fragment for two row groups.
    rg = groups >= 1024 ? 2 : 1;
  }
  rg = std::min(rg, MaxRowGroups(plan.mt));
  const int tiles = (groups + rg - 1) / rg;
  const int max_waves = MaxWaves(plan.mt, rg);
  if (waves <= 0) {
    // About 2048 waves over the chip with at least two pairs each; a tile's
    // waves split its pairs and meet in LDS.
    waves = 4;
    while (waves < max_waves && tiles * waves < 2048 && pairs >= 4 * waves)
      waves *= 2;
    while (waves > 1 && pairs < 2 * waves)
      waves /= 2;
  }
  waves = std::max(1, std::min(waves, max_waves));
  plan.rg = rg;
  plan.waves = waves;
  plan.tiles = tiles;
  if (splits <= 0) {
    // Still fewer tiles than compute units: split k over workgroups too.
    splits = 1;
    while (plan.tiles * splits < 128 && pairs >= 4 * waves * splits)
      splits *= 2;
  }
  splits = std::max(1, std::min(splits, pairs));
  plan.pairs_per_split = (pairs + splits - 1) / splits;
  plan.splits = (pairs + plan.pairs_per_split - 1) / plan.pairs_per_split;
  if (plan.splits > 1 &&
      (scratch_floats < static_cast<std::size_t>(plan.splits) * m * n ||
       scratch_counters < static_cast<std::size_t>(plan.tiles))) {
    plan.splits = 1;
    plan.pairs_per_split = pairs;
  }
  plan.pairs_per_wave = (plan.pairs_per_split + waves - 1) / waves;
  return plan;
}

int RunSkinny(const Bf16* x, const void* w, float* y, Bf16* y_bf16,
              std::size_t m, std::size_t k, std::size_t n, bool accumulate,
              const ProductPlan& plan, float* partials, unsigned* counters,
              hipStream_t stream, q8::Weights kind) {
  if (plan.engine) {
    // The rows one workgroup loads (its block's), which set the load groups.
    const int block_rows = static_cast<int>((m + plan.row_blocks - 1) / plan.row_blocks);
    const EngineLauncher launch =
        PickEngine(plan.mt, plan.rg, plan.pw, block_rows, plan.waves, kind);
    if (launch == nullptr)
      return Fail(VX_UNSUPPORTED, "no product engine for this plan");
    q8::TileArgs args{};
    args.w = static_cast<const std::uint8_t*>(w);
    args.m = static_cast<int>(m);
    args.k = static_cast<int>(k);
    args.n = static_cast<int>(n);
    args.pairs = static_cast<int>(q8::Pairs(k));
    args.groups = static_cast<int>(q8::Groups(n));
    args.group_stride = 1;
    args.row_blocks = plan.row_blocks;
    args.rows_per_block = block_rows;
    args.x = x;
    args.y = y_bf16 != nullptr ? nullptr : y;
    args.y_bf16 = y_bf16;
    args.accumulate = accumulate ? 1 : 0;
    launch(args, plan.tiles * plan.row_blocks, plan.waves, stream);
    return LaunchStatus(q8::IsQ8(kind) ? "q8 product" : "bf16 product");
  }
  if (kind != q8::Weights::kQ8)
    return Fail(VX_UNSUPPORTED, "split plans take Q8_0 panels only");
  const Launcher launch = PickLauncher(plan.mt, plan.rg);
  if (launch == nullptr)
    return Fail(VX_UNSUPPORTED, "no product kernel for this plan");
  SkinnyArgs args;
  args.x = x;
  args.w = static_cast<const std::uint8_t*>(w);
  args.y = y;
  args.y_bf16 = y_bf16;
  args.partials = partials;
  args.counters = counters;
  args.m = static_cast<int>(m);
  args.k = static_cast<int>(k);
  args.n = static_cast<int>(n);
  args.pairs = static_cast<int>(q8::Pairs(k));
  args.pairs_per_split = plan.pairs_per_split;
  args.pairs_per_wave = plan.pairs_per_wave;
  args.splits = plan.splits;
  args.accumulate = accumulate ? 1 : 0;
  launch(args, plan, stream);
  return LaunchStatus("q8 product");
}

bool UseRowBlocks(std::size_t m, std::size_t k, std::size_t n, bool q8) {
  // Measured on MI355X against the tiled kernel (with its k split) and the
  // 32 x 32 MFMA kernel, Q8_0 and bf16 panels alike: faster up to about
  // 1.2 G multiply-adds (129 x 2048 x 2048 15.6 -> 9.2 us, 256 x 1024 x 4096
  // 14.3 -> 10.9 us), and on 2048 x 2048 weights up to 512 rows (512 rows
  // 21.0 -> 17.3 us); slower beyond (1024 x 2048 x 2048 24.7 -> 32.9 us),
  // where each 64-row block re-reads the weights. Q8_0 panels of up to
  // 2048 x 6144 values also up to 256 rows (129 x 2048 x 6144 24.2 -> 16.1
  // us, 256 x 6144 x 2048 25.8 -> 23.6 us; 256 x 2048 x 4096 and
  // 256 x 1024 x 8192 on a par), and up to 512 rows while k is at most
  // 4096 (384 / 512 x 2048 x 6144 32.3 / 33.3 -> 25.4 / 30.6 us, 320 x
  // 4096 x 2048 25.4 -> 20.7 us; 512 x 6144 x 2048 36.8 -> 40.0 us, so not
  // there); bf16 panels lost there.
  if (m <= kExactRows)
    return false;
  const double work = static_cast<double>(m) * static_cast<double>(k) * static_cast<double>(n);
  return work <= 1.2e9 || (m <= 512 && k >= 2048 && k * n <= 2048 * 2048) ||
         (q8 && k * n <= 2048 * 6144 && (m <= 256 || (m <= 512 && k <= 4096)));
}

int RunRowBlocks(const Bf16* x, const void* w, float* y, Bf16* y_bf16, std::size_t m,
                 std::size_t k, std::size_t n, bool accumulate, bool bf16, hipStream_t stream) {
  if (m <= kExactRows)
    return Fail(VX_UNSUPPORTED, "row-block product: more than 128 rows");
  return RunSkinny(x, w, y, y_bf16, m, k, n, accumulate, PlanRowBlocks(m, k, n), nullptr,
                   nullptr, stream, bf16 ? q8::Weights::kBf16 : q8::Weights::kQ8Expanded);
}

int RunEngineTuned(const Bf16* x, const void* w, float* y, std::size_t m, std::size_t k,
                   std::size_t n, int rg, int waves, int pw, int row_blocks,
                   hipStream_t stream) {
  if (m <= 16 || m > 32)
    return Fail(VX_UNSUPPORTED, "tuned engine plans take 17..32 rows");
  const TunedLauncher launch = PickTuned(rg, pw, waves, static_cast<int>(m));
  if (launch == nullptr || row_blocks < 1 || row_blocks > 4)
    return Fail(VX_UNSUPPORTED, "no tuned engine for this plan");
  q8::TileArgs args{};
  args.w = static_cast<const std::uint8_t*>(w);
  args.m = static_cast<int>(m);
  args.k = static_cast<int>(k);
  args.n = static_cast<int>(n);
  args.pairs = static_cast<int>(q8::Pairs(k));
  args.groups = static_cast<int>(q8::Groups(n));
  args.group_stride = 1;
  args.row_blocks = row_blocks;
  args.rows_per_block = static_cast<int>((m + row_blocks - 1) / row_blocks);
  args.x = x;
  args.y = y;
  launch(args, (args.groups + rg - 1) / rg, stream);
  return LaunchStatus("tuned q8 product");
}

}  // namespace vx
