// The skinny Q8_0 product engine, shared by the standalone products (up to
// 128 rows with the exact arithmetic, more in blocks of 64 rows with the
// expanded one) and the DiT's fused layer kernels.
//
// A workgroup owns RG row groups (16 weight rows each) of the output and the
// whole reduction length; its waves split the column pairs (two Q8_0
// blocks, one panel unit per row group), PW pairs per wave per pass, the
// next pass's weights and activations in flight while the current pass is
// multiplied. Each 32-column block is one v_mfma_f32_16x16x32_bf16 from
// zero (the float32 block sum) followed by acc = fmaf(f16 scale, sum, acc),
// the arithmetic of kernels/wmma_products.hip:192-215. The waves' partial
// sums meet in LDS and are added in wave order, so every run gives the same
// bits.
//
// Activations come from one of three sources:
//  - kRowMajor: bf16 [m][k] row-major (the drop-in product's x); up to
//    64 rows (a block of them) are staged per wave through LDS from
//    whole-line loads;
//  - kFragBf16: bf16 in fragment order (below), written by the DiT kernels
//    so that each wave's operand load is 1 KB of contiguous bytes;
//  - kNormF32: the float32 residual stream in fragment order, RMS-normalised
//    on the fly (kernels/generator_kernels.hip:91-108): each wave loads its
//    pairs' values, the per-row sums of squares meet in LDS, and the operand
//    is bf16((x * rsqrt(mean + eps)) * gamma), exactly the reference's
//    normalised bf16 activations;
//  - kNormRows: the same from a row-major float32 residual stream of up to
//    16 rows (one tile: the stacks' decode steps and encoder patches);
//  - kScaledBf16: bf16 in fragment order holding bf16(x * gamma) of the
//    residual stream, written by the epilogue that produced x together with
//    each row's sums of squares over its 16-column groups; the outputs are
//    scaled by the row's rsqrt(sum / k + eps): RMSNorm's per-row factor
//    applied after the product instead of before the rounding to bf16.
//
// and leave through one of three epilogues:
//  - kStore: float32 [m][n] row-major (optionally accumulated) or bf16;
//  - kResidual: added into the float32 fragment-order residual stream
//    (optionally also the next norm's kScaledBf16 operand and sums);
//  - kSwiGlu: RG = 2 with the up rows `group_stride` row groups after the
//    gate rows; bf16(silu(gate) * up) in bf16 fragment order
//    (kernels/generator_kernels.hip:243-254);
//  - kSwiGluRows: the same into bf16 [m][n / 2] row-major (y_bf16);
//  - kQkvCache: RG = 1, workgroup 2 p + h taking rows 8 h .. 8 h + 7 of
//    group pair p's two row groups (each rotary dimension's partner,
//    head_dim / 2 columns on, is `group_stride` row groups after it); the
//    rotary embedding at each row's position, then q [m][heads][head_dim]
//    and the row's key and value cache rows
//    (kernels/generator_kernels.hip:110-158).
#ifndef VOXCPM_AMD_Q8_TILE_HPP_
#define VOXCPM_AMD_Q8_TILE_HPP_

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "common.hpp"
#include "q8.hpp"

namespace vx::q8 {

// ---- fragment-order activation layouts (up to 32 rows) ----------------------
//
// The A operand of v_mfma_f32_16x16x32_bf16 for rows 16 t .. 16 t + 15 and
// columns 64 p + 32 h .. + 31 is lane L = 16 octet + r16 holding row
// 16 t + r16, columns 64 p + 32 h + 8 octet + 0..7. Fragment order stores
// those eight values of each lane contiguously, lanes in order, then
// (p, t, h) with h fastest:
//   bf16: 16 bytes per lane, 1 KB per (p, t, h);
//   f32:  32 bytes per lane as two 16-byte quarters (values 0..3, 4..7),
//         quarter-major, so one 16-byte load per lane still reads 1 KB of
//         contiguous bytes.
// Rows run to 32 (two 16-row tiles); columns to a multiple of 64.

constexpr int kFragRows = 32;
// Floats per wave of the norm prologue's row sums of squares (32 rows,
// padded so that the two halves of the waves read disjoint banks).
constexpr int kSquaresStride = 36;

__host__ __device__ inline std::size_t BfFragIndex(int row, int column) {
  const int pair = column >> 6;
  const int half = (column >> 5) & 1;
  const int octet = (column >> 3) & 3;
  const int t = row >> 4;
  const int lane = 16 * octet + (row & 15);
  return ((((static_cast<std::size_t>(pair) * 2 + t) * 2 + half) * 64 + lane) * 8) +
         (column & 7);
}

__host__ __device__ inline std::size_t F32FragIndex(int row, int column) {
  const int pair = column >> 6;
  const int half = (column >> 5) & 1;
  const int octet = (column >> 3) & 3;
  const int quarter = (column >> 2) & 1;
  const int t = row >> 4;
  const int lane = 16 * octet + (row & 15);
  return ((((static_cast<std::size_t>(pair) * 2 + t) * 2 + half) * 2 + quarter) * 64 +
          lane) * 4 +
         (column & 3);
}

/// Elements of a fragment-order matrix of `columns` columns (32 rows).
inline std::size_t FragElements(std::size_t columns) {
  return static_cast<std::size_t>(kFragRows) * ((columns + 63) / 64) * 64;
}

enum class ASource : int {
  kRowMajor = 0,
  kFragBf16 = 1,
  kNormF32 = 2,
  kNormRows = 3,
  kScaledBf16 = 4
};
enum class Output : int { kStore = 0, kResidual = 1, kSwiGlu = 2, kSwiGluRows = 3, kQkvCache = 4 };

struct TileArgs {
  const std::uint8_t* w;  // panels [groups][pairs] units
  int m;                  // activation rows
  int k;                  // reduction length (columns of x)
  int n;                  // output columns (weight rows)
  int pairs;              // Pairs(k)
  int groups;             // Groups(n)
  int group_stride;       // row group r of tile b: RgGroup(b, r, stride)
  // Row blocks (>= 1): the grid is row_blocks x the tiles; workgroup
  // b = tile + tiles * block takes activation rows
  // [block rows_per_block, + rows_per_block) of the tile, so that a launch
  // of few tiles fills the compute units and each loads only its rows.
  // The blocks of a tile lie a multiple of 8 workgroups apart (tiles a
  // multiple of 8), on one compute die, whose L2 serves their weights.
  int row_blocks;
  int rows_per_block;
  // Fragment-order sources with MT = 1 take tile-aligned row blocks
  // instead: block b is part b % tile_blocks of the 16-row tile
  // b / tile_blocks (row_blocks = tiles of m x tile_blocks), so that each
  // workgroup loads and multiplies one 16-row tile.
  int tile_blocks;
  // activations
  const Bf16* x;          // kRowMajor [m][k] / kFragBf16
  const float* h;         // kNormF32: float32 fragment order [32][k];
                          // kNormRows: float32 [m][k] row-major
  const Bf16* gamma;      // kNormF32, kNormRows: [k]
  float eps;              // kNormF32, kNormRows
  // outputs
  float* y;               // kStore float32 [m][n]
  Bf16* y_bf16;           // kStore bf16 [m][n] (used when y is null);
                          // kSwiGluRows bf16 [m][n / 2]
  int accumulate;         // kStore float32: y += product
  float* residual;        // kResidual: float32 fragment order [32][n]
  const float* residual_in;  // kResidual: the stream added to (null: residual)
  Bf16* frag_out;         // kSwiGlu: bf16 fragment order [32][n / 2]
  // kQkvCache: n = (heads + 2 kv_heads) head_dim columns q | k | v.
  float* q_out;                    // [m][heads][head_dim], rotated
  float* k_cache;                  // [kv_heads][capacity][head_dim]
  float* v_cache;
  const float* rope;               // [positions][head_dim] cos | sin, or null
  const std::int32_t* positions;   // [m] rotary position of each row
  const std::int32_t* cache_rows;  // [m] cache row of each row
  int heads;
  int kv_heads;
  int head_dim;
  int capacity;
  // kResidual with norm_out non-null: the next RMSNorm's operand
  // bf16(x * norm_gamma) in bf16 fragment order [32][n] and each row's sum
  // of x^2 over the workgroup's 16 columns, norm_squares[row][column / 16].
  Bf16* norm_out;
  const Bf16* norm_gamma;
  float* norm_squares;
  // kScaledBf16: those sums, [32][squares_groups] (eps above).
  const float* row_squares;
  int squares_groups;
};

/// Row group r of workgroup tile b: consecutive groups (stride 1) or a
/// group and its partner `stride` groups later (SwiGLU's gate and up).
__host__ __device__ inline int RgGroup(int tile, int r, int stride, int rg) {
  return (tile / stride) * stride * rg + tile % stride + r * stride;
}

/// Maximum threads of a workgroup of the engine for (MT, RG): the larger
/// register footprints take 8 waves.
constexpr int EngineThreads(int mt, int rg) {
  return (mt <= 2 && rg <= 2) ? 1024 : 512;
}

/// Row-major activations of up to 64 rows (a workgroup's row block) are
/// staged per wave through LDS (below); more rows are loaded straight into
/// the MFMA operands.
__host__ __device__ constexpr bool StagesRows(ASource source, int mt) {
  return source == ASource::kRowMajor && mt <= 4;
}

/// Floats of a wave's row-staging region: one pair's 16 MT rows x 64
/// columns of bf16 (the pairs of a pass are staged one after another).
__host__ __device__ constexpr int StageFloats(int mt) {
  return mt * 16 * 32;
}

/// Floats of the normalised bf16 rows [m][k + 8] of the kNormRows source
/// (a multiple of 4: the sums behind them stay 16-byte aligned).
__host__ __device__ constexpr std::size_t NormRowsFloats(int m, int k) {
  return ((static_cast<std::size_t>(m) * (k + 8) + 7) / 8) * 4;
}

/// LDS bytes of the kNormRows source for m rows of k (k a multiple of 64,
/// at most 8 times the threads): the normalised rows and the row sums,
/// later the waves' partial sums over the same bytes.
__host__ __device__ constexpr std::size_t NormRowsShared(int mt, int rg, int m, int k) {
  const int threads = EngineThreads(mt, rg);
  const std::size_t rows = NormRowsFloats(m, k) + threads + 16;
  const std::size_t reduce = static_cast<std::size_t>(threads / 64) * rg * mt * 256;
  return (rows > reduce ? rows : reduce) * sizeof(float);
}

/// LDS bytes the engine needs for `waves` waves. The row-staging regions
/// and the waves' partial sums share the same bytes (a barrier separates
/// them).
__host__ __device__ constexpr std::size_t EngineShared(int mt, int rg, int waves,
                                                      ASource source) {
  std::size_t per_wave = static_cast<std::size_t>(rg) * mt * 256;
  if (StagesRows(source, mt) && static_cast<std::size_t>(StageFloats(mt)) > per_wave)
    per_wave = static_cast<std::size_t>(StageFloats(mt));
  std::size_t floats = static_cast<std::size_t>(waves) * per_wave;
  if (source == ASource::kNormF32)
    floats += static_cast<std::size_t>(waves) * kSquaresStride;
  return floats * sizeof(float);
}

__device__ inline float Silu(float value) {
  return value / (1.0F + expf(-value));
}

/// Two float32 -> two bf16 (nearest even) packed low / high, one
/// v_cvt_pk_bf16_f32 on gfx950; the same bits as Bf16Bits, including the
/// quiet-NaN rule (checked against it on the GPU).
__device__ inline std::uint32_t PackBf16x2(float lo, float hi) {
  typedef float F32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 Bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(std::uint32_t,
                            __builtin_convertvector(F32x2{lo, hi}, Bf16x2));
}

/// Eight float32 -> eight bf16 (nearest even), packed for an MFMA operand.
__device__ inline uint4 PackBf16x8(const float (&v)[8]) {
  return uint4{PackBf16x2(v[0], v[1]), PackBf16x2(v[2], v[3]),
               PackBf16x2(v[4], v[5]), PackBf16x2(v[6], v[7])};
}

/// Eight int8 values (two little-endian dwords) times `scale`, each rounded
/// to bf16 (nearest even, quiet NaNs) by v_cvt_pk_bf16_f32: the
/// reference's expansion of a Q8_0 block beyond 128 rows
/// (kernels/wmma_products.hip:94-112, gemm.cpp:305-312).
__device__ inline uint4 Expand(std::uint32_t w0, std::uint32_t w1, float scale) {
  const auto v = [&](std::uint32_t word, int byte) {
    return scale * static_cast<float>(static_cast<std::int8_t>(word >> (8 * byte)));
  };
  return uint4{PackBf16x2(v(w0, 0), v(w0, 1)), PackBf16x2(v(w0, 2), v(w0, 3)),
               PackBf16x2(v(w1, 0), v(w1, 1)), PackBf16x2(v(w1, 2), v(w1, 3))};
}

/// One float32 -> bf16 bits through the same instruction.
__device__ inline Bf16 Bf16Fast(float value) {
  return static_cast<Bf16>(PackBf16x2(value, 0.0F) & 0xFFFFU);
}

__device__ inline float Bf16Lo(std::uint32_t word) {
  return __uint_as_float(word << 16);
}
__device__ inline float Bf16Hi(std::uint32_t word) {
  return __uint_as_float(word & 0xFFFF0000U);
}

// Activation loads go through buffer resources: a lane whose value is
// masked (a row outside the block, a pair past k) loads at an offset past
// the buffer's range, which returns zero without a memory access. A load
// guarded by a per-lane condition would instead be a divergent branch
// whose zero-filling side writes the same registers, which makes the
// compiler wait for each load before the next: a wave's loads would
// arrive one round trip after another instead of together.
__device__ inline __amdgpu_buffer_rsrc_t BufferOf(const void* base, std::uint32_t bytes) {
  // Raw buffer, 32-bit data format (the gfx9 family's word 3).
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0,
                                           static_cast<int>(bytes), 0x00020000);
}
constexpr std::uint32_t kPastBuffer = 0x7FFFFFF0U;
/// 16 bytes at `offset` of the buffer, or zero (no access) unless `keep`.
__device__ inline uint4 BufferLoad16(__amdgpu_buffer_rsrc_t buffer, std::uint32_t offset,
                                     bool keep) {
  return __builtin_bit_cast(
      uint4, __builtin_amdgcn_raw_buffer_load_b128(
                 buffer, static_cast<int>(keep ? offset : kPastBuffer), 0, 0));
}
/// 4 bytes at `offset` of the buffer, or zero (no access) unless `keep`.
__device__ inline std::uint32_t BufferLoad4(__amdgpu_buffer_rsrc_t buffer, std::uint32_t offset,
                                            bool keep) {
  return static_cast<std::uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(
      buffer, static_cast<int>(keep ? offset : kPastBuffer), 0, 0));
}

/// One pair's operands in flight: RG weight fragments (Q8_0: both blocks'
/// values and the scale pairs; bf16: `w` and `w2`, one block each), and
/// the MT x 2 activation fragments.
template<int MT, int RG>
struct PairStage {
  uint4 w[RG];
  uint4 w2[RG];
  std::uint32_t scales[RG];
  uint4 a[MT][2];
};

/// Stores of the engine's epilogues: ordinary, or (kCoherent) device-scope
/// relaxed atomic stores, which write through the compute die's L2 so that
/// workgroups on other dies read them after a grid barrier.
template<bool kCoherent, typename T>
__device__ inline void Put(T* p, T v) {
  if constexpr (kCoherent)
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    *p = v;
}

/// LDS bytes EnginePrefetch stages: one panel unit per wave, pass slot and
/// row group.
__host__ __device__ constexpr int PrefetchBytes(int rg, int pw, int waves) {
  return waves * pw * rg * kUnitBytes;
}

/// The Q8_0 weights of the first pass of pairs (pair p waves + wave of
/// slot p) of workgroup `block_id` of a `grid`-workgroup launch, copied
/// into the LDS at `stage` (PrefetchBytes bytes, 16-byte aligned) by the
/// vector memory unit's LDS loads (no registers hold them), unit (wave, p,
/// r) at ((wave PW + p) RG + r) units: a persistent kernel issues them
/// before the grid barriers that precede the product, and EngineBody's kPre
/// reads them from there. Each wave waits for its own copies
/// (s_waitcnt) before reading them.
template<int MT, int RG, Output OUT, int PW, int NW = 0>
__device__ __forceinline__ void EnginePrefetch(const TileArgs& a, int block_id, int grid,
                                               int thread, std::uint8_t* stage) {
  static_assert(OUT != Output::kQkvCache, "half pairs are not prefetched");
  constexpr int waves = NW > 0 ? NW : EngineThreads(MT, RG) / kWave;
  typedef __attribute__((address_space(3))) void LdsVoid;
  const int lane = thread % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(thread / kWave);
  const int tiles = grid / a.row_blocks;
  const int tile = block_id % tiles;
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    const int g = min(RgGroup(tile, r, a.group_stride, RG), a.groups - 1);
    const std::uint8_t* unit = a.w + static_cast<std::size_t>(g) * a.pairs * kUnitBytes;
#pragma unroll
    for (int p = 0; p < PW; ++p) {
      const int pair = p * waves + wave;
      const std::uint8_t* u = unit + static_cast<std::size_t>(pair < a.pairs ? pair : 0) * kUnitBytes;
      std::uint8_t* dst = stage + ((wave * PW + p) * RG + r) * kUnitBytes;
      // 1024 bytes of values, lane L's 16 at 16 L; then the 64 bytes of
      // scales from lanes 0..3.
      __builtin_amdgcn_global_load_lds(u + 16 * lane, (LdsVoid*)(dst), 16, 0, 0);
      if (lane < 4)
        __builtin_amdgcn_global_load_lds(u + kValueBytes + 16 * lane,
                                         (LdsVoid*)(dst + kValueBytes), 16, 0, 0);
    }
  }
}

/// The engine. Grid: one workgroup per tile (RG row groups); blockDim.x =
/// EngineThreads(MT, RG) (waves without pairs add zeros). PW pairs per wave
/// per pass; kNormF32 needs every pair in one pass (pairs <= waves * PW).
/// Staged row-major sources load JR groups of 8 rows (8 JR >= m). WK: the
/// weights' format; bf16 weights (panels or rows [n][k]) accumulate each
/// block's MFMA straight into the sums, as the reference's bf16 products do
/// (kernels/wmma_products.hip:210-213). The workgroup is `block_id` of a
/// `grid`-workgroup launch (a kernel's blockIdx.x and gridDim.x, or a phase
/// of a persistent kernel), `thread` its thread (threadIdx.x, or a value
/// the compiler cannot follow, so that a persistent kernel does not keep
/// the engine's per-lane index arithmetic in registers across its phases). kCoherent: the epilogue's stores are
/// device-scope (Put). kPre: fragment-order sources over Q8_0 panels whose
/// first pass's weights EnginePrefetch staged in the LDS at `pre`.
/// kOnePass: fragment-order sources whose pairs one pass covers
/// (pairs <= waves PW, the launcher's promise): no registers are set aside
/// for a next pass in flight.
template<int MT, int RG, ASource SRC, Output OUT, int PW = 1, int JR = 2 * MT,
         Weights WK = Weights::kQ8, int NW = 0, bool kCoherent = false, bool kPre = false,
         bool kOnePass = false>
__device__ __forceinline__ void EngineBody(const TileArgs& a, int block_id, int grid, int thread,
                                           const std::uint8_t* pre = nullptr) {
  // One 16-row tile of a fragment-order source per workgroup.
  constexpr bool kScaled = SRC == ASource::kScaledBf16;
  constexpr bool kOneTile = MT == 1 && (SRC == ASource::kFragBf16 || kScaled);
  static_assert(!kScaled || (MT == 2 && !kOneTile), "scaled rows are the 32 fragment rows");
  constexpr bool kNorm = SRC == ASource::kNormF32 || SRC == ASource::kNormRows;
  constexpr bool kSwish = OUT == Output::kSwiGlu || OUT == Output::kSwiGluRows;
  constexpr bool kRope = OUT == Output::kQkvCache;
  static_assert(SRC != ASource::kNormF32 || MT == 2, "norm source is 32 rows");
  static_assert(SRC != ASource::kNormRows || MT == 1, "row-major norm source is one tile");
  static_assert(OUT == Output::kStore || OUT == Output::kSwiGluRows ||
                    OUT == Output::kQkvCache || MT == 2 || kOneTile,
                "fragment outputs are 32 rows or one tile of them");
  // kQkvCache: each workgroup takes the same 8 rows of a rotary
  // dimension's two row groups (lanes r16 < 8 the first group's, r16 >= 8
  // the second's), so that twice as many workgroups as pairs share the
  // weights; each output's partner is 8 lanes away.
  constexpr bool kHalfPairs = kRope;
  static_assert(!kSwish || RG == 2, "SwiGLU pairs two groups");
  static_assert(!kRope || RG == 1, "the rotary embedding takes half pairs");
  static_assert(!kHalfPairs || WK != Weights::kBf16Rows, "half pairs read panels");
  extern __shared__ float lds[];
  const int lane = thread % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(thread / kWave);
  // NW > 0: a workgroup of NW waves instead of EngineThreads(MT, RG).
  constexpr int waves = NW > 0 ? NW : EngineThreads(MT, RG) / kWave;
  const int r16 = lane % 16;
  const int octet = lane / 16;
  static_assert(!kPre || ((SRC == ASource::kFragBf16 || SRC == ASource::kScaledBf16) &&
                          WK == Weights::kQ8 && OUT != Output::kQkvCache),
                "prefetched weights are Q8_0 panels of the fragment-order passes");
  const int tiles = grid / a.row_blocks;
  const int tile = block_id % tiles;
  const int block = block_id / tiles;
  int row_lo, row_hi;
  int tile_base = 0;  // the workgroup's first 16-row tile
  if constexpr (kOneTile) {
    tile_base = block / a.tile_blocks;
    const int first = 16 * tile_base;
    const int count = min(16, a.m - first);
    const int per = (count + a.tile_blocks - 1) / a.tile_blocks;
    row_lo = first + (block % a.tile_blocks) * per;
    row_hi = min(first + count, row_lo + per);
  } else {
    row_lo = block * a.rows_per_block;
    row_hi = min(a.m, row_lo + a.rows_per_block);
  }
  const auto in_rows = [&](int row) { return row >= row_lo && row < row_hi; };
  // kPre: the first pass's weights were staged in the LDS by this wave's
  // own copies; they are complete once nothing of the wave is in flight,
  // which costs nothing more here, before its first loads.
  if constexpr (kPre)
    __builtin_amdgcn_s_waitcnt(0);
  // The workgroup's first activation row: its 16-row tile of a fragment
  // source, or the first row of its block for row-major activations (the
  // block's rows then lie in the MT tiles from there).
  constexpr bool kBlockTile = SRC == ASource::kRowMajor;
  const int row_base = kBlockTile ? row_lo : 16 * tile_base;
  const int k_blocks = a.k / 32;

  constexpr int kUnit = IsQ8(WK) ? kUnitBytes : kBf16UnitBytes;
  // kHalfPairs: workgroup tile is half tile % 2 (rows 8 half .. + 7) of
  // the group pair tile / 2; the lane reads its row of its group's panel
  // (panel lane 16 octet + row holds the row's k chunk octet).
  const int half_of_pair = kHalfPairs ? tile % 2 : 0;
  const int pair_tile = kHalfPairs ? tile / 2 : tile;
  const int panel_row = kHalfPairs ? 8 * half_of_pair + r16 % 8 : r16;
  const int panel_lane = 16 * octet + panel_row;
  const auto group_of = [&](int r, int column_lane) {
    return kHalfPairs ? RgGroup(pair_tile, column_lane >= 8 ? 1 : 0, a.group_stride, 2)
                      : RgGroup(tile, r, a.group_stride, RG);
  };
  const std::uint8_t* unit[RG];
  int first_row[RG];  // bf16 rows: the group's first weight row
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    const int g = min(group_of(r, r16), a.groups - 1);
    unit[r] = a.w + static_cast<std::size_t>(g) * a.pairs * kUnit;
    first_row[r] = 16 * g;
  }
  bool row_ok[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t)
    row_ok[t] = in_rows(row_base + 16 * t + r16);
  // The activations as buffers: row-major [m][k] bf16, fragment-order bf16
  // (32 rows x pairs x 64 columns), fragment-order float32 or row-major
  // float32 [m][k].
  const __amdgpu_buffer_rsrc_t x_buffer = BufferOf(
      a.x, SRC == ASource::kRowMajor
               ? 2U * static_cast<std::uint32_t>(a.m) * static_cast<std::uint32_t>(a.k)
               : 4096U * static_cast<std::uint32_t>(a.pairs));
  const __amdgpu_buffer_rsrc_t h_buffer = BufferOf(
      a.h, SRC == ASource::kNormRows
               ? 4U * static_cast<std::uint32_t>(a.m) * static_cast<std::uint32_t>(a.k)
               : 8192U * static_cast<std::uint32_t>(a.pairs));

  // Output element e of the tile (thread e, e + threads, ...): fragment
  // f = r MT + t, accumulator i, lane l -> (row, column); false past m / n.
  constexpr int kThreads = waves * kWave;
  constexpr int kOutputsPerThread = (RG * MT * 256 + kThreads - 1) / kThreads;
  const auto output_of = [&](int e, int& row, int& column) {
    const int f = e / 256;
    const int i = (e / 64) % 4;
    const int l = e % 64;
    const int r = f / MT;
    const int t = f % MT;
    row = row_base + 16 * t + 4 * (l / 16) + i;
    const int group = group_of(r, l % 16);
    column = kHalfPairs ? 16 * group + 8 * half_of_pair + l % 8 : 16 * group + l % 16;
    return in_rows(row) && group < a.groups && column < a.n;
  };
  // The values the epilogue adds to (the residual stream, an accumulated
  // y) are loaded now, beside the first weights, instead of after the sums.
  float before[kOutputsPerThread];
  // kResidual with norm_out: the next norm's gamma of each output's column,
  // loaded now for the same reason.
  float next_gamma[kOutputsPerThread];
  // kQkvCache: each output's row position and cache row, loaded now by
  // masked buffer loads (no branch, so nothing waits for them here); the
  // rotary table entries they select are loaded with the activations.
  std::uint32_t position[kOutputsPerThread];
  std::uint32_t cache_row[kOutputsPerThread];
  if constexpr (kRope) {
    const __amdgpu_buffer_rsrc_t positions = BufferOf(a.positions, 4U * a.m);
    const __amdgpu_buffer_rsrc_t cache_rows = BufferOf(a.cache_rows, 4U * a.m);
#pragma unroll
    for (int u = 0; u < kOutputsPerThread; ++u) {
      const int e = thread + u * kThreads;
      int row, column;
      const bool live = e < RG * MT * 256 && output_of(e, row, column);
      const std::uint32_t at = 4U * static_cast<std::uint32_t>(live ? row : 0);
      position[u] = BufferLoad4(positions, at, live);
      cache_row[u] = BufferLoad4(cache_rows, at, live);
    }
  }
#pragma unroll
  for (int u = 0; u < kOutputsPerThread; ++u) {
    before[u] = 0.0F;
    next_gamma[u] = 0.0F;
    const int e = thread + u * kThreads;
    int row, column;
    if (e >= RG * MT * 256 || !output_of(e, row, column))
      continue;
    if constexpr (OUT == Output::kResidual) {
      before[u] = (a.residual_in != nullptr ? a.residual_in : a.residual)[F32FragIndex(row, column)];
      if (a.norm_out != nullptr)
        next_gamma[u] = Bf16Value(a.norm_gamma[column]);
    } else if constexpr (OUT == Output::kStore) {
      if (a.y != nullptr && a.accumulate)
        before[u] = a.y[static_cast<std::size_t>(row) * a.n + column];
    }
  }

  // Pairs past k load pair 0's unit, branch-free: their stages are never
  // multiplied.
  // bf16 rows [n][k]: a buffer over the matrix, rows past n and columns
  // past k masked.
  const __amdgpu_buffer_rsrc_t row_buffer =
      BufferOf(a.w, WK == Weights::kBf16Rows
                        ? 2U * static_cast<std::uint32_t>(a.n) * static_cast<std::uint32_t>(a.k)
                        : 0U);
  const auto load_weights = [&](int pair, PairStage<MT, RG>& s) {
    const bool ok = pair < a.pairs;
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      if constexpr (WK == Weights::kBf16Rows) {
        const int row = first_row[r] + r16;
        const int column = 64 * pair + 8 * octet;
        const std::uint32_t at = 2U * static_cast<std::uint32_t>(row * a.k + column);
        s.w[r] = BufferLoad16(row_buffer, at, ok && row < a.n && column < a.k);
        s.w2[r] = BufferLoad16(row_buffer, at + 64U, ok && row < a.n && column + 32 < a.k);
      } else {
        const std::uint8_t* u = unit[r] + static_cast<std::size_t>(ok ? pair : 0) * kUnit;
        s.w[r] = *reinterpret_cast<const uint4*>(u + 16 * panel_lane);
        if constexpr (IsQ8(WK))
          s.scales[r] = *reinterpret_cast<const std::uint32_t*>(u + kValueBytes + 4 * panel_row);
        else
          s.w2[r] = *reinterpret_cast<const uint4*>(u + kBf16HalfBytes + 16 * panel_lane);
      }
    }
  };
  const auto load_activations = [&](int pair, PairStage<MT, RG>& s) {
    const bool ok = pair < a.pairs;
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        uint4 v{0U, 0U, 0U, 0U};
        if constexpr (SRC == ASource::kRowMajor) {
          v = BufferLoad16(x_buffer,
                           2U * static_cast<std::uint32_t>((row_base + 16 * t + r16) * a.k +
                                                           64 * pair + 32 * hf + 8 * octet),
                           ok && row_ok[t] && 2 * pair + hf < k_blocks);
        } else if constexpr (SRC == ASource::kFragBf16 || kScaled) {
          v = BufferLoad16(
              x_buffer,
              16U * static_cast<std::uint32_t>(((pair * 2 + tile_base + t) * 2 + hf) * 64 + lane),
              ok && row_ok[t]);
        }
        s.a[t][hf] = v;
      }
  };

  // Row staging (row-major x, a block of up to 64 rows): a pair's rows come in as
  // whole 128-byte row segments, eight rows per load instruction (lane L:
  // row 8 j + L / 8, bytes 16 (L % 8) .. + 15 of the segment), go to the
  // wave's private LDS region with each 16-byte chunk index XORed with
  // row % 8 (conflict-free writes and reads), and come back as the MFMA A
  // fragments. A wave-load then touches 8 full cache lines instead of 16
  // half-used ones.
  static_assert(JR >= 1 && JR <= 2 * MT, "JR load groups of 8 rows cover the m rows");
  struct RawRows {
    uint4 v[JR];
  };
  const auto load_rows = [&](int pair, RawRows& raw) {
    const int column = 64 * pair + 8 * (lane % 8);
    // Lanes past k or outside the rows load an in-range address and keep
    // zero.
    const bool column_ok = column < a.k && pair < a.pairs;
#pragma unroll
    for (int j = 0; j < JR; ++j) {
      const int row = row_base + 8 * j + lane / 8;
      raw.v[j] = BufferLoad16(x_buffer, 2U * static_cast<std::uint32_t>(row * a.k + column),
                              column_ok && in_rows(row));
    }
  };
  // The pairs of a pass go through the one region in turn: a wave's LDS
  // accesses complete in order, so a pair's writes follow the previous
  // pair's reads without a wait.
  uint4* const region = reinterpret_cast<uint4*>(lds + wave * StageFloats(MT));
  const auto stage_rows = [&](const RawRows& raw, PairStage<MT, RG>& s) {
#pragma unroll
    for (int j = 0; j < JR; ++j) {
      // Rows outside the block were loaded as zero; writing them keeps the
      // code branch-free (they are never read as operands).
      const int row = 8 * j + lane / 8;
      region[row * 8 + ((lane % 8) ^ (row % 8))] = raw.v[j];
    }
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int row = 16 * t + r16;
        const int chunk = 4 * hf + octet;
        s.a[t][hf] = row_ok[t] ? region[row * 8 + (chunk ^ (row % 8))] : uint4{0U, 0U, 0U, 0U};
      }
  };

  F32x4 acc[RG][MT];
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int t = 0; t < MT; ++t)
      acc[r][t] = F32x4{0.0F, 0.0F, 0.0F, 0.0F};

  // kScaledBf16: the rows' sums of squares, loaded with the first operands
  // (thread t: row t / 32 of each pass of kThreads / 32 rows, groups
  // t % 32, + 32, + 64, + 96) and added after the products.
  constexpr int kSquareRows = kThreads / 32;
  constexpr int kSquarePasses = kScaled ? (32 + kSquareRows - 1) / kSquareRows : 1;
  float squares[kSquarePasses][4];
  const auto load_squares = [&]() {
    const __amdgpu_buffer_rsrc_t buffer = BufferOf(
        a.row_squares, 4U * 32U * static_cast<std::uint32_t>(a.squares_groups));
#pragma unroll
    for (int pass = 0; pass < kSquarePasses; ++pass) {
      const int row = pass * kSquareRows + thread / 32;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int g = thread % 32 + 32 * j;
        squares[pass][j] = __builtin_bit_cast(
            float, BufferLoad4(buffer, 4U * static_cast<std::uint32_t>(row * a.squares_groups + g),
                               row < 32 && g < a.squares_groups));
      }
    }
  };

  const auto multiply = [&](const PairStage<MT, RG>& s) {
    const F32x4 zero{0.0F, 0.0F, 0.0F, 0.0F};
    if constexpr (WK == Weights::kQ8Expanded) {
      // Each block's weights as bf16(scale * q), one float32 sum over k.
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        const float s0 = HalfValue(static_cast<std::uint16_t>(s.scales[r] & 0xFFFFU));
        const float s1 = HalfValue(static_cast<std::uint16_t>(s.scales[r] >> 16));
        const Bf16x8 b0 = AsBf16x8(Expand(s.w[r].x, s.w[r].y, s0));
        const Bf16x8 b1 = AsBf16x8(Expand(s.w[r].z, s.w[r].w, s1));
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          acc[r][t] = Mfma16x16x32(AsBf16x8(s.a[t][0]), b0, acc[r][t]);
          acc[r][t] = Mfma16x16x32(AsBf16x8(s.a[t][1]), b1, acc[r][t]);
        }
      }
      return;
    }
    if constexpr (WK != Weights::kQ8) {
#pragma unroll
      for (int r = 0; r < RG; ++r)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          acc[r][t] = Mfma16x16x32(AsBf16x8(s.a[t][0]), AsBf16x8(s.w[r]), acc[r][t]);
          acc[r][t] = Mfma16x16x32(AsBf16x8(s.a[t][1]), AsBf16x8(s.w2[r]), acc[r][t]);
        }
      return;
    }
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

  // kQkvCache: the cos / sin of each output's rotary dimension. Their
  // loads depend on the positions loaded at the start, so they are issued
  // after the first activation loads, whose wait they share.
  constexpr int kPairedOutputs = MT * 256;
  float rope_cos[kOutputsPerThread];
  float rope_sin[kOutputsPerThread];
  const auto load_rope = [&] {
#pragma unroll
    for (int u = 0; u < kOutputsPerThread; ++u) {
      rope_cos[u] = 1.0F;
      rope_sin[u] = 0.0F;
      const int e = thread + u * kThreads;
      int row, column;
      if (e < kPairedOutputs && output_of(e, row, column) && a.rope != nullptr &&
          column < (a.heads + a.kv_heads) * a.head_dim) {
        // The position is used here, not hoisted ahead of the first loads.
        std::uint32_t at = position[u];
        asm volatile("" : "+v"(at));
        // The rotary dimension: the column's index within its half-head.
        const float* table = a.rope + static_cast<std::size_t>(at) * a.head_dim +
                             (column % a.head_dim) % (a.head_dim / 2);
        rope_cos[u] = table[0];
        rope_sin[u] = table[a.head_dim / 2];
      }
    }
  };
  static_assert(!kRope || SRC == ASource::kNormRows, "the rotary epilogue takes norm rows");

  float* reduce = lds;
  if constexpr (SRC == ASource::kNormRows) {
    // The workgroup's m rows, RMS-normalised once into LDS as bf16 (rows
    // k + 8 values apart, which spreads their banks), are every wave's
    // operands: only the weights are held in registers, so two workgroups
    // fit a compute unit. Threads take 8 consecutive values of a row, the
    // rows of a pass side by side; each row's sum of squares is added by
    // one wave in a fixed order.
    const int stride = a.k + 8;
    Bf16* xs = reinterpret_cast<Bf16*>(lds);
    float* sums = lds + NormRowsFloats(a.m, a.k);  // [threads] partials, [16] inverses
    PairStage<MT, RG> stage[PW];
#pragma unroll
    for (int p = 0; p < PW; ++p)
      load_weights(wave + p * waves, stage[p]);
    __builtin_amdgcn_sched_barrier(0);
    const int t = thread;
    const int per_row = a.k / 8;
    // A wave adds each row's sums: at most one row per wave per pass.
    const int rows_per_pass = min(kThreads / per_row, waves);
    const int c = t % per_row;
    const uint4 g = *reinterpret_cast<const uint4*>(a.gamma + 8 * c);
    for (int first = 0; first < a.m; first += rows_per_pass) {
      const int r = first + t / per_row;
      const bool live = t < rows_per_pass * per_row && r < a.m;
      const std::uint32_t at = 4U * static_cast<std::uint32_t>(r * a.k + 8 * c);
      const float4 lo = __builtin_bit_cast(float4, BufferLoad16(h_buffer, at, live));
      const float4 hi = __builtin_bit_cast(float4, BufferLoad16(h_buffer, at + 16U, live));
      if constexpr (kRope) {
        if (first == 0)
          load_rope();
      }
      const float x[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      float square = 0.0F;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        square += x[i] * x[i];
      sums[t] = square;
      __syncthreads();
      if (wave < rows_per_pass && first + wave < a.m) {
        float total = 0.0F;
        for (int j = lane; j < per_row; j += kWave)
          total += sums[wave * per_row + j];
        total = AddXor32(AddXor16(RowSum16(total)));
        if (lane == 0)
          sums[kThreads + wave] = rsqrtf(total / static_cast<float>(a.k) + a.eps);
      }
      __syncthreads();
      if (live) {
        // The norm weights are unpacked here, after this pass's loads were
        // issued: unpacked before the loop, their wait (in order behind the
        // weights' loads) held back the residual rows' loads by a round
        // trip.
        uint4 gw = g;
        asm volatile("" : "+v"(gw.x), "+v"(gw.y), "+v"(gw.z), "+v"(gw.w));
        const float gamma[8] = {Bf16Lo(gw.x), Bf16Hi(gw.x), Bf16Lo(gw.y), Bf16Hi(gw.y),
                                Bf16Lo(gw.z), Bf16Hi(gw.z), Bf16Lo(gw.w), Bf16Hi(gw.w)};
        const float inverse = sums[kThreads + t / per_row];
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          v[i] = x[i] * inverse * gamma[i];
        *reinterpret_cast<uint4*>(xs + r * stride + 8 * c) = PackBf16x8(v);
      }
      __syncthreads();
    }
#pragma unroll
    for (int p = 0; p < PW; ++p) {
      const int pair = wave + p * waves;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
        stage[p].a[0][hf] =
            row_ok[0] ? *reinterpret_cast<const uint4*>(xs + r16 * stride +
                                                         64 * (pair < a.pairs ? pair : 0) +
                                                         32 * hf + 8 * octet)
                      : uint4{0U, 0U, 0U, 0U};
      if (pair < a.pairs)
        multiply(stage[p]);
    }
    // The partial sums below reuse the rows' bytes.
    __syncthreads();
  } else if constexpr (kNorm) {
    // Every pair in this pass: wave w owns pairs w, w + waves, ...
    float* squares = lds + static_cast<std::size_t>(waves) * RG * MT * 256;
    PairStage<MT, RG> stage[PW];
    float4 hv[PW][MT][2][2];  // [pair][t][half][quarter]
    uint4 gamma_bits[PW][2];  // [pair][half]: 8 bf16 norm weights
#pragma unroll
    for (int p = 0; p < PW; ++p)
      load_weights(wave + p * waves, stage[p]);
#pragma unroll
    for (int p = 0; p < PW; ++p) {
      const int pair = wave + p * waves;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
        gamma_bits[p][hf] = *reinterpret_cast<const uint4*>(
            a.gamma + 64 * (pair < a.pairs ? pair : 0) + 32 * hf + 8 * octet);
    }
    // The weights and norm weights are in flight before the residual
    // stream's loads are issued.
    __builtin_amdgcn_sched_barrier(0);
    float partial[2] = {0.0F, 0.0F};
#pragma unroll
    for (int p = 0; p < PW; ++p) {
      const int pair = wave + p * waves;
      const bool ok = pair < a.pairs;
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            hv[p][t][hf][q] = __builtin_bit_cast(
                float4, BufferLoad16(h_buffer,
                                     16U * static_cast<std::uint32_t>(
                                               (((pair * 2 + t) * 2 + hf) * 2 + q) * 64 + lane),
                                     ok && row_ok[t]));
          }
    }
#pragma unroll
    for (int p = 0; p < PW; ++p) {
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const float4 v = hv[p][t][hf][q];
            partial[t] += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
          }
    }
    // The four octets of a row meet across lanes (permlane swaps, no LDS
    // round trip); waves meet in LDS.
#pragma unroll
    for (int t = 0; t < MT; ++t)
      partial[t] = AddXor32(AddXor16(partial[t]));
    if (octet == 0) {
      squares[wave * kSquaresStride + r16] = partial[0];
      squares[wave * kSquaresStride + 16 + r16] = partial[1];
    }
    __syncthreads();
    // Lane l adds row l % 32 over one half of the waves (the halves' reads
    // fall on different banks), the halves meet by one shuffle, and every
    // lane takes its two rows' inverses from the lanes that hold them.
    constexpr int kHalf = waves / 2;
    const int first = (lane / 32) * kHalf;
    float total = 0.0F;
#pragma unroll
    for (int w = 0; w < kHalf; ++w)
      total += squares[(first + w) * kSquaresStride + lane % 32];
    total = AddXor32(total);
    const float row_inverse = rsqrtf(total / static_cast<float>(a.k) + a.eps);
    float inverse[2];
    BroadcastRows01(row_inverse, inverse[0], inverse[1]);
#pragma unroll
    for (int p = 0; p < PW; ++p) {
      const int pair = wave + p * waves;
      const bool ok = pair < a.pairs;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const uint4 g = gamma_bits[p][hf];
        const float gamma[8] = {Bf16Lo(g.x), Bf16Hi(g.x), Bf16Lo(g.y), Bf16Hi(g.y),
                                Bf16Lo(g.z), Bf16Hi(g.z), Bf16Lo(g.w), Bf16Hi(g.w)};
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const float4 lo = hv[p][t][hf][0];
          const float4 hi = hv[p][t][hf][1];
          const float x[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
          float v[8];
#pragma unroll
          for (int i = 0; i < 8; ++i)
            v[i] = x[i] * inverse[t] * gamma[i];
          stage[p].a[t][hf] = (ok && row_ok[t]) ? PackBf16x8(v) : uint4{0U, 0U, 0U, 0U};
        }
      }
    }
#pragma unroll
    for (int p = 0; p < PW; ++p)
      if (wave + p * waves < a.pairs)
        multiply(stage[p]);
  } else if constexpr (StagesRows(SRC, MT)) {
    // Passes of PW pairs per wave (pair base + p waves + wave), every load
    // of a pass issued before its first product, so that PW pairs per wave
    // are in flight; plans pick PW so that few passes cover k. (Loading the
    // next pass before multiplying this one measured slower on MI355X:
    // 11.3 against 10.9 us at (2048, 16384), and masked loads past k cost
    // address cycles at one-pass shapes.)
    for (int base = 0; base < a.pairs; base += waves * PW) {
      PairStage<MT, RG> stage[PW];
      RawRows raw[PW];
#pragma unroll
      for (int p = 0; p < PW; ++p) {
        load_weights(base + p * waves + wave, stage[p]);
        load_rows(base + p * waves + wave, raw[p]);
      }
#pragma unroll
      for (int p = 0; p < PW; ++p) {
        stage_rows(raw[p], stage[p]);
        if (base + p * waves + wave < a.pairs)
          multiply(stage[p]);
      }
    }
    // The partial sums below reuse the staging regions.
    __syncthreads();
  } else {
    // Passes of PW pairs per wave (slot p of the pass at base: pair
    // base + p waves + wave); the next pass is loaded before this one is
    // multiplied, so 2 PW pairs per wave are in flight.
    PairStage<MT, RG> current[PW];
    PairStage<MT, RG> next[kOnePass ? 1 : PW];
    const int step = waves * PW;
#pragma unroll
    for (int p = 0; p < PW; ++p) {
      load_activations(p * waves + wave, current[p]);
      if constexpr (!kPre)
        load_weights(p * waves + wave, current[p]);
    }
    if constexpr (kPre) {
      // The staged weights, read from the LDS once the activations' loads
      // are in flight.
#pragma unroll
      for (int p = 0; p < PW; ++p)
#pragma unroll
        for (int r = 0; r < RG; ++r) {
          const std::uint8_t* unit = pre + ((wave * PW + p) * RG + r) * kUnitBytes;
          current[p].w[r] = *reinterpret_cast<const uint4*>(unit + 16 * lane);
          current[p].scales[r] = *reinterpret_cast<const std::uint32_t*>(unit + kValueBytes + 4 * r16);
        }
    }
    if constexpr (kScaled)
      load_squares();
    for (int base = 0; base < a.pairs; base += step) {
      const bool more = !kOnePass && base + step < a.pairs;
      if constexpr (!kOnePass) {
        if (more) {
#pragma unroll
          for (int p = 0; p < PW; ++p) {
            load_activations(base + step + p * waves + wave, next[p]);
            load_weights(base + step + p * waves + wave, next[p]);
          }
        }
      }
#pragma unroll
      for (int p = 0; p < PW; ++p)
        if (base + p * waves + wave < a.pairs)
          multiply(current[p]);
      if (!more)
        break;
      if constexpr (!kOnePass) {
#pragma unroll
        for (int p = 0; p < PW; ++p)
          current[p] = next[p];
      }
    }
  }

  // kScaledBf16: each row's RMSNorm factor rsqrt(sum / k + eps), the
  // groups' sums added per lane and then over the row's 32 lanes in a
  // fixed order (made visible by the barrier below).
  __shared__ float row_scale[kScaled ? 32 : 1];
  if constexpr (kScaled) {
#pragma unroll
    for (int pass = 0; pass < kSquarePasses; ++pass) {
      float total = ((squares[pass][0] + squares[pass][1]) + squares[pass][2]) + squares[pass][3];
      total = AddXor16(RowSum16(total));
      const int row = pass * kSquareRows + thread / 32;
      if (thread % 32 == 0 && row < 32)
        row_scale[row] = rsqrtf(total / static_cast<float>(a.k) + a.eps);
    }
  }

  // Partial sums of the waves meet in LDS: [wave][fragment r MT + t][i][lane].
  constexpr int kFragmentFloats = RG * MT * 256;
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        reduce[wave * kFragmentFloats + ((r * MT + t) * 4 + i) * 64 + lane] = acc[r][t][i];
  __syncthreads();

  // All waves' partials are read at once, then added in wave order.
  constexpr int kWaves = waves;
  const auto total_of = [&](int e) {
    float parts[kWaves];
#pragma unroll
    for (int w = 0; w < kWaves; ++w)
      parts[w] = reduce[w * kFragmentFloats + e];
    float total = parts[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w)
      total += parts[w];
    return total;
  };
  const int outputs = kSwish || kRope ? MT * 256 : kFragmentFloats;
  // kResidual with norm_out: each output's new residual value (0 past the
  // outputs), for the next norm's operand and sums below.
  float fresh[kOutputsPerThread];
#pragma unroll
  for (int u = 0; u < kOutputsPerThread; ++u) {
    fresh[u] = 0.0F;
    const int e = thread + u * kThreads;
    // kHalfPairs: every lane of a wave with outputs takes part in the
    // exchange with its partner 8 lanes away (outputs are whole waves).
    float mine = 0.0F;
    float partner_value = 0.0F;
    if constexpr (kHalfPairs) {
      mine = e < outputs ? total_of(e) : 0.0F;
      partner_value = RowDpp<kDppRotate8>(mine);
    }
    int row, column;
    if (e >= outputs || !output_of(e, row, column))
      continue;
    const float v = kHalfPairs ? mine : kScaled ? total_of(e) * row_scale[row] : total_of(e);
    if constexpr (OUT == Output::kStore) {
      const std::size_t at = static_cast<std::size_t>(row) * a.n + column;
      if (a.y != nullptr)
        Put<kCoherent>(a.y + at, a.accumulate ? before[u] + v : v);
      else
        Put<kCoherent>(a.y_bf16 + at, Bf16Fast(v));
    } else if constexpr (OUT == Output::kResidual) {
      fresh[u] = before[u] + v;
      Put<kCoherent>(a.residual + F32FragIndex(row, column), fresh[u]);
    } else if constexpr (OUT == Output::kSwiGlu) {
      const float up = kScaled ? total_of(e + MT * 256) * row_scale[row] : total_of(e + MT * 256);
      Put<kCoherent>(a.frag_out + BfFragIndex(row, column), Bf16Fast(Silu(v) * up));
    } else if constexpr (kRope) {
      // (x_i, x_{i + half}) -> (x_i c - x_{i + half} s, x_{i + half} c + x_i s)
      // on q and k; v is stored as it is. Lanes r16 < 8 hold x_i and
      // lanes r16 >= 8 x_{i + half}; each received its partner's value.
      const int head = column / a.head_dim;
      const bool second_half = e % 16 >= 8;
      float out = v;
      if (a.rope != nullptr && head < a.heads + a.kv_heads) {
        const float c = rope_cos[u];
        const float sn = rope_sin[u];
        out = second_half ? v * c + partner_value * sn : v * c - partner_value * sn;
      }
      float* target;
      if (head < a.heads)
        target = a.q_out + (static_cast<std::size_t>(row) * a.heads + head) * a.head_dim;
      else if (head < a.heads + a.kv_heads)
        target = a.k_cache + (static_cast<std::size_t>(head - a.heads) * a.capacity +
                              static_cast<std::size_t>(cache_row[u])) *
                                 a.head_dim;
      else
        target = a.v_cache + (static_cast<std::size_t>(head - a.heads - a.kv_heads) * a.capacity +
                              static_cast<std::size_t>(cache_row[u])) *
                                 a.head_dim;
      target[column % a.head_dim] = out;
    } else {
      const float up = total_of(e + MT * 256);
      a.y_bf16[static_cast<std::size_t>(row) * (a.n / 2) + column] = Bf16Fast(Silu(v) * up);
    }
  }
  if constexpr (OUT == Output::kResidual) {
    if (a.norm_out != nullptr) {
      // The next norm's operand, and each row's sum of squares over the 16
      // columns of its group: the 16 lanes of a DPP row hold one row's 16
      // columns, so one row reduction per output slot (uniform control
      // flow; outputs past the block add zeros and are not written).
#pragma unroll
      for (int u = 0; u < kOutputsPerThread; ++u) {
        const int e = thread + u * kThreads;
        int row = 0, column = 0;
        const bool live = e < outputs && output_of(e, row, column);
        const float square = RowSum16(fresh[u] * fresh[u]);
        if (live) {
          Put<kCoherent>(a.norm_out + BfFragIndex(row, column), Bf16Fast(fresh[u] * next_gamma[u]));
          if (column % 16 == 0)
            Put<kCoherent>(a.norm_squares + row * (a.n / 16) + column / 16, square);
        }
      }
    }
  }
}

template<int MT, int RG, ASource SRC, Output OUT, int PW = 1, int JR = 2 * MT,
         Weights WK = Weights::kQ8, int NW = 0, bool kOnePass = false>
__global__ __launch_bounds__(NW > 0 ? NW * kWave : EngineThreads(MT, RG)) void EngineKernel(
    TileArgs a) {
  EngineBody<MT, RG, SRC, OUT, PW, JR, WK, NW, false, false, kOnePass>(a, static_cast<int>(blockIdx.x),
                                              static_cast<int>(gridDim.x),
                                              static_cast<int>(threadIdx.x));
}


}  // namespace vx::q8

#endif  // VOXCPM_AMD_Q8_TILE_HPP_
