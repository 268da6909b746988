// One DiT evaluation as one persistent launch (dit_persistent.hpp).
//
// Phases of a launch, each ended by a grid barrier:
//   in      in_proj of x and the assembly of the 2 (3 + 2 P) rows
//           (generator.cpp:297-316; kernels/generator_kernels.hip:320-340);
//   per layer (transformer.cpp:74-96):
//   qkv     rmsnorm(h) Wqkv^T, one 16-row group per workgroup
//           (generator_kernels.hip:91-108 inside the product's prologue);
//           the last workgroup to finish a head's q, k and v groups (a
//           device-scope counter per head) then runs that head's rotary
//           embedding and attention for both branches
//           (generator_kernels.hip:110-241);
//   o       h += attn Wo^T, one group per workgroup;
//   gate_up swiglu(rmsnorm(h) Wgate_up^T), a gate group and its up group
//           per workgroup (generator_kernels.hip:243-254);
//   down    h += s Wdown^T;
//   then the final norm, out_proj, its bias and the guided Euler step in
//   workgroup 0 (generator.cpp:318-324; generator_kernels.hip:342-360).
//
// The Q8_0 arithmetic is the products' (q8_tile.hpp): each 32-column block
// one v_mfma_f32_16x16x32_bf16 from zero, then acc = fmaf(f16 scale, sum,
// acc) (kernels/wmma_products.hip:192-215); the 16 waves of a workgroup
// split the pairs and their sums meet in LDS in wave order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>

#include "common.hpp"
#include "dit_fused.hpp"
#include "dit_persistent.hpp"
#include "q8.hpp"
#include "q8_tile.hpp"

namespace vx::persistent {
namespace {

using q8::AsBf16x8;
using q8::Bf16x8;
using q8::BfFragIndex;
using q8::F32FragIndex;
using q8::F32x4;
using q8::Int8x8ToBf16;
using q8::kUnitBytes;
using q8::kValueBytes;
using q8::Mfma16x16x32;

/// Elements of a 32-row fragment-order matrix of `columns` columns.
__host__ __device__ inline std::size_t Frag(int columns) {
  return static_cast<std::size_t>(32) * ((columns + 63) / 64) * 64;
}

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kWave;
constexpr int kMaxGrid = 256;
// Barrier arrivals spread over 16 counters 256 bytes apart (workgroup w
// counts in slot w % 16), so no counter takes more than 16 atomics.
constexpr int kSlots = 16;
constexpr int kSlotStride = 64;
constexpr int kGenerationWord = kSlots * kSlotStride;
constexpr int kErrorWord = kGenerationWord + 64;
// Then one arrival counter per (layer, hidden group) of the down product,
// then one per (layer, head) of the qkv product.
constexpr int kArrivalsWord = kErrorWord + 64;
// The down product splits its k over this many workgroups per group.
constexpr int kDownSplits = 4;
// About a second of polling before a wait gives up (one poll is well under
// a microsecond).
constexpr int kSpinLimit = 1 << 21;
constexpr int kMaxLength = 16;  // rows of one branch
constexpr int kOutGroups = 4;   // feat <= 64

// LDS (floats): wave partial sums [waves][2 row groups][2 tiles][4][64],
// the norm's squares [waves][32], a phase's output block [32][16], the
// output phase's rows, and at the end the flags. The attention phase uses
// everything before the flags. 96 KB are requested so that a compute unit
// holds one workgroup.
constexpr int kRedFloats = kWaves * 2 * 2 * 256;
constexpr int kSquaresAt = kRedFloats;
constexpr int kStageAt = kSquaresAt + kWaves * 32;
constexpr int kVelocityAt = kStageAt + 32 * 16;
constexpr int kBlockAt = kVelocityAt + 2 * 8 * 64;
constexpr std::size_t kLdsBytes = 96 * 1024;
constexpr int kFlagsAt = static_cast<int>(kLdsBytes / sizeof(float)) - 16;
static_assert(kBlockAt + kWaves <= kFlagsAt, "LDS plan");
// A phase's output block is one element per thread.
static_assert(kThreads == 32 * 16, "output blocks map one element per thread");

struct Args {
  // shape
  int rows, length, patch, hidden, heads, kv_heads, head_dim, ffn, feat;
  int layers, q_width, qkv_width;
  float eps, attention_scale;
  Weights w;
  // inputs
  const float* mu;     // [2][hidden]
  const float* time;   // [hidden]
  const float* cond;   // [patch][hidden]
  const float* x;      // [patch][feat]
  // outputs
  float* velocity;     // [2][patch][feat]
  float* x_update;     // [patch][feat] or null
  float cfg, dt;
  int zero_star;
  Workspace ws;
  // Optional timestamps (s_memrealtime, 100 MHz) per workgroup and barrier:
  // [workgroup][barrier + 1][arrive, leave, operands, products]: arrival at
  // and exit from the barrier, and inside the phase before it the times
  // its activations and its products were done; slot 0 holds the kernel's
  // start and end. Null: not recorded.
  unsigned long long* trace;
};

// ---- thread indices -------------------------------------------------------------
//
// Opaque to the optimizer: index arithmetic derived from them is recomputed
// in each phase instead of being hoisted out of the layer loop, where it
// would hold registers for the whole launch.

__device__ inline int Tid() {
  int v = static_cast<int>(threadIdx.x);
  asm volatile("" : "+v"(v));
  return v;
}
__device__ inline int Lane() { return Tid() % kWave; }
__device__ inline int Wave() {
  return __builtin_amdgcn_readfirstlane(Tid() / kWave);
}

// ---- device-scope stores and loads -------------------------------------------

__device__ inline void StoreU32(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline unsigned LoadU32(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/// Every memory operation of this wave so far has completed (its
/// device-scope stores are visible to every compute die). Called after a
/// phase's stores and before the next phase's weight loads, so that the
/// grid barrier does not wait for those loads.
__device__ inline void WaitStores() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

/// Grid barrier number `index` (1-based within the launch). Every wave has
/// waited for its stores (WaitStores); wave 0 counts the workgroup in and
/// polls the slot counters while the other waves' weight loads for the
/// next phase are in flight. Returns false when the launch must stop: the
/// wait timed out (the error word is set) or another workgroup stopped.
__device__ bool GridBarrier(unsigned* sync, unsigned base, int index,
                            int* quit, unsigned long long* trace = nullptr) {
  __syncthreads();
  if (trace != nullptr && threadIdx.x == 0)
    trace[4 * index] = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x < kWave) {
    const int lane = static_cast<int>(threadIdx.x);
    const int grid = static_cast<int>(gridDim.x);
    const int slot = static_cast<int>(blockIdx.x) % kSlots;
    if (lane == 0)
      __hip_atomic_fetch_add(sync + slot * kSlotStride, 1U, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    bool stop = false;
    bool timed_out = false;
    for (int spin = 0;; ++spin) {
      bool ok = true;
      if (lane < kSlots) {
        const unsigned members =
            static_cast<unsigned>((grid - lane + kSlots - 1) / kSlots);
        const unsigned target = (base + static_cast<unsigned>(index)) * members;
        ok = static_cast<int>(LoadU32(sync + lane * kSlotStride) - target) >= 0;
      }
      if (__all(ok))
        break;
      // Wave-uniform: every lane takes the same exit.
      if (__any(LoadU32(sync + kErrorWord) != 0U)) {
        stop = true;
        break;
      }
      if (spin >= kSpinLimit) {
        stop = true;
        timed_out = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) {
      if (timed_out)
        StoreU32(sync + kErrorWord, 1U);
      *quit = stop ? 1 : 0;
      if (trace != nullptr)
        trace[4 * index + 1] = __builtin_amdgcn_s_memrealtime();
    }
  }
  __syncthreads();
  return *quit == 0;
}

/// Records the time into trace word `at` (thread 0; no-op without a trace).
__device__ inline void Mark(unsigned long long* trace, int at) {
  if (trace != nullptr && threadIdx.x == 0)
    trace[at] = __builtin_amdgcn_s_memrealtime();
}

// ---- the product pieces ---------------------------------------------------------

/// A tile's weights for one wave: RG row groups of PW pairs (pair
/// wave + 16 p), with their scale pairs.
template<int RG, int PW>
struct Stage {
  uint4 w[PW][RG];
  std::uint32_t s[PW][RG];
};

/// Pairs [first, first + count) of a panel of `pairs` pairs per row group;
/// wave w takes pairs first + w + 16 p.
template<int RG, int PW>
__device__ inline void LoadStage(const std::uint8_t* panels, int pairs,
                                 int groups, int stride, int tile,
                                 Stage<RG, PW>& st, int first = 0, int count = -1) {
  const int lane = Lane();
  const int wave = Wave();
  const int r16 = lane % 16;
  if (count < 0)
    count = pairs;
#pragma unroll
  for (int p = 0; p < PW; ++p) {
    const int local = wave + p * kWaves;
    const bool ok = local < count;
    const int pair = first + (ok ? local : 0);
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      const int g = min(q8::RgGroup(tile, r, stride, RG), groups - 1);
      const std::uint8_t* u =
          panels + (static_cast<std::size_t>(g) * pairs + pair) * kUnitBytes;
      st.w[p][r] = ok ? *reinterpret_cast<const uint4*>(u + 16 * lane)
                      : uint4{0U, 0U, 0U, 0U};
      st.s[p][r] =
          ok ? *reinterpret_cast<const std::uint32_t*>(u + kValueBytes + 4 * r16) : 0U;
    }
  }
}

/// A operands of PW pairs from bf16 fragment order [32][k]: pairs
/// [first, first + count), wave w taking first + w + 16 p.
template<int PW>
__device__ inline void FragOperands(const Bf16* x, int first, int count, int rows,
                                    uint4 (&a)[PW][2][2]) {
  const int lane = Lane();
  const int wave = Wave();
  const int r16 = lane % 16;
#pragma unroll
  for (int p = 0; p < PW; ++p) {
    const bool ok = wave + p * kWaves < count;
    const int pair = first + wave + p * kWaves;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
        a[p][t][hf] = (ok && 16 * t + r16 < rows)
                          ? reinterpret_cast<const uint4*>(x)[((pair * 2 + t) * 2 + hf) * 64 + lane]
                          : uint4{0U, 0U, 0U, 0U};
  }
}

/// A operands of PW pairs from the float32 residual stream in fragment
/// order, RMS-normalised over all k columns (every pair in this pass):
/// bf16((x * rsqrt(mean(x^2) + eps)) * gamma). Contains a barrier.
template<int PW>
__device__ inline void NormOperands(const float* h, const Bf16* gamma, int k,
                                    int rows, float eps, float* squares,
                                    uint4 (&a)[PW][2][2]) {
  const int lane = Lane();
  const int wave = Wave();
  const int r16 = lane % 16;
  const int octet = lane / 16;
  const int pairs = k / 64;
  bool row_ok[2];
  row_ok[0] = r16 < rows;
  row_ok[1] = 16 + r16 < rows;
  float4 hv[PW][2][2][2];
  uint4 gamma_bits[PW][2];
#pragma unroll
  for (int p = 0; p < PW; ++p) {
    const int pair = wave + p * kWaves;
    const bool ok = pair < pairs;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
      gamma_bits[p][hf] =
          ok ? *reinterpret_cast<const uint4*>(gamma + 64 * pair + 32 * hf + 8 * octet)
             : uint4{0U, 0U, 0U, 0U};
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int q = 0; q < 2; ++q)
          hv[p][t][hf][q] =
              (ok && row_ok[t])
                  ? reinterpret_cast<const float4*>(h)[(((pair * 2 + t) * 2 + hf) * 2 + q) * 64 + lane]
                  : float4{0.0F, 0.0F, 0.0F, 0.0F};
  }
  float partial[2] = {0.0F, 0.0F};
#pragma unroll
  for (int p = 0; p < PW; ++p)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const float4 v = hv[p][t][hf][q];
          partial[t] += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    partial[t] += __shfl_xor(partial[t], 16, kWave);
    partial[t] += __shfl_xor(partial[t], 32, kWave);
  }
  if (octet == 0) {
    squares[wave * 32 + r16] = partial[0];
    squares[wave * 32 + 16 + r16] = partial[1];
  }
  __syncthreads();
  float inverse[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    float total = 0.0F;
    for (int w = 0; w < kWaves; ++w)
      total += squares[w * 32 + 16 * t + r16];
    inverse[t] = rsqrtf(total / static_cast<float>(k) + eps);
  }
#pragma unroll
  for (int p = 0; p < PW; ++p) {
    const bool ok = wave + p * kWaves < pairs;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const uint4 g = gamma_bits[p][hf];
      const float gm[8] = {q8::Bf16Lo(g.x), q8::Bf16Hi(g.x), q8::Bf16Lo(g.y),
                           q8::Bf16Hi(g.y), q8::Bf16Lo(g.z), q8::Bf16Hi(g.z),
                           q8::Bf16Lo(g.w), q8::Bf16Hi(g.w)};
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const float4 lo = hv[p][t][hf][0];
        const float4 hi = hv[p][t][hf][1];
        const float xv[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          v[i] = xv[i] * inverse[t] * gm[i];
        a[p][t][hf] = (ok && row_ok[t]) ? q8::PackBf16x8(v) : uint4{0U, 0U, 0U, 0U};
      }
    }
  }
}

template<int RG, int PW>
__device__ inline void Multiply(const Stage<RG, PW>& st, const uint4 (&a)[PW][2][2],
                                int pairs, F32x4 (&acc)[RG][2]) {
  const int wave = Wave();
  const F32x4 zero{0.0F, 0.0F, 0.0F, 0.0F};
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int t = 0; t < 2; ++t)
      acc[r][t] = zero;
#pragma unroll
  for (int p = 0; p < PW; ++p) {
    if (wave + p * kWaves >= pairs)
      continue;
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      const Bf16x8 b0 = Int8x8ToBf16(st.w[p][r].x, st.w[p][r].y);
      const Bf16x8 b1 = Int8x8ToBf16(st.w[p][r].z, st.w[p][r].w);
      const float s0 = HalfValue(static_cast<std::uint16_t>(st.s[p][r] & 0xFFFFU));
      const float s1 = HalfValue(static_cast<std::uint16_t>(st.s[p][r] >> 16));
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const F32x4 sum0 = Mfma16x16x32(AsBf16x8(a[p][t][0]), b0, zero);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[r][t][i] = fmaf(s0, sum0[i], acc[r][t][i]);
        const F32x4 sum1 = Mfma16x16x32(AsBf16x8(a[p][t][1]), b1, zero);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[r][t][i] = fmaf(s1, sum1[i], acc[r][t][i]);
      }
    }
  }
}

/// The waves' sums to LDS ([wave][(r 2 + t) 4 + i][lane]), then a barrier.
template<int RG>
__device__ inline void WaveSums(float* red, const F32x4 (&acc)[RG][2]) {
  const int lane = Lane();
  const int wave = Wave();
  constexpr int kFrag = RG * 2 * 256;
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        red[wave * kFrag + ((r * 2 + t) * 4 + i) * 64 + lane] = acc[r][t][i];
  __syncthreads();
}

/// Sum in wave order of LDS element `e` of a fragment set of kFrag floats.
template<int RG>
__device__ inline float Total(const float* red, int e) {
  constexpr int kFrag = RG * 2 * 256;
  float parts[kWaves];
#pragma unroll
  for (int w = 0; w < kWaves; ++w)
    parts[w] = red[w * kFrag + e];
  float total = parts[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w)
    total += parts[w];
  return total;
}

/// LDS element of output (row group r, row, column c16 of the group).
__device__ inline int Slot(int r, int row, int c16) {
  return ((r * 2 + row / 16) * 4 + row % 4) * 64 + 16 * ((row % 16) / 4) + c16;
}

// ---- whole-line stores of a workgroup's 32 x 16 output block ------------------
//
// Phases gather their output block in LDS (one element per thread), then 16
// consecutive threads write 256 contiguous bytes with 16-byte device-scope
// stores, so that every 128-byte line is written whole by one request and
// rows past the CFG pair are written as zeros.

/// 16 bytes with one device-scope store: global_store_dwordx4 with sc1, the
/// cache policy the compiler gives a relaxed agent-scope atomic store.
__device__ inline void Store16(void* p, const uint4& v) {
  typedef unsigned U32x4 __attribute__((ext_vector_type(4)));
  const U32x4 d{v.x, v.y, v.z, v.w};
  asm volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(p), "v"(d) : "memory");
}

/// staging float32 [32][16] (rows >= rows as 0), plus `add` when non-null,
/// to columns 16 group .. + 15 of a float32 fragment-order matrix.
__device__ inline void BlockToF32Frag(const float* staging, int rows, int group,
                                      const float* add, float* dst) {
  const int tid = Tid();
  if (tid >= 128)
    return;
  const int r16 = tid % 16;
  const int quarter = (tid / 16) % 2;
  const int o2 = (tid / 32) % 2;
  const int row = 16 * (tid / 64) + r16;
  const int c16 = 8 * o2 + 4 * quarter;
  const std::size_t at = F32FragIndex(row, 16 * group + c16);
  float4 v{0.0F, 0.0F, 0.0F, 0.0F};
  if (row < rows) {
    v = *reinterpret_cast<const float4*>(staging + row * 16 + c16);
    if (add != nullptr) {
      const float4 b = *reinterpret_cast<const float4*>(add + at);
      v = float4{b.x + v.x, b.y + v.y, b.z + v.z, b.w + v.w};
    }
  }
  Store16(dst + at, __builtin_bit_cast(uint4, v));
}

/// staging bf16 [32][16] to columns 16 group .. + 15 of a bf16
/// fragment-order matrix.
__device__ inline void BlockToBf16Frag(const Bf16* staging, int rows, int group,
                                       Bf16* dst) {
  const int tid = Tid();
  if (tid >= 64)
    return;
  const int r16 = tid % 16;
  const int o2 = (tid / 16) % 2;
  const int row = 16 * (tid / 32) + r16;
  const uint4 v = row < rows
                      ? *reinterpret_cast<const uint4*>(staging + row * 16 + 8 * o2)
                      : uint4{0U, 0U, 0U, 0U};
  Store16(dst + BfFragIndex(row, 16 * group + 8 * o2), v);
}

/// staging float32 [32][16] to group `group` of a tile-major matrix
/// [groups][32][16] (2 KB per group).
__device__ inline void BlockToTile(const float* staging, int rows, int group,
                                   float* dst) {
  const int tid = Tid();
  if (tid >= 128)
    return;
  const int row = tid / 4;
  const int quad = tid % 4;
  const float4 v = row < rows ? *reinterpret_cast<const float4*>(staging + row * 16 + 4 * quad)
                              : float4{0.0F, 0.0F, 0.0F, 0.0F};
  Store16(dst + (static_cast<std::size_t>(group) * 32 + row) * 16 + 4 * quad,
          __builtin_bit_cast(uint4, v));
}

/// Four floats at (row, column) of a tile-major matrix (column % 4 == 0).
__device__ inline float4 TileQuad(const float* m, int row, int column) {
  return *reinterpret_cast<const float4*>(
      m + (static_cast<std::size_t>(column / 16) * 32 + row) * 16 + column % 16);
}

/// This thread's element of a 32 x 16 output block: row tid / 16, column
/// tid % 16.
__device__ inline int BlockRow() { return Tid() / 16; }
__device__ inline int BlockColumn() { return Tid() % 16; }

// ---- phases -------------------------------------------------------------------------

/// in_proj of the patch rows (x rounded to bf16, the exact product, the
/// bias) for 16 hidden columns (wave 0), and the mu / time / condition rows
/// of those columns, gathered as the group's block of h.
__device__ void PhaseIn(const Args& a, int group, float* h, float* lds) {
  float* staging = lds + kStageAt;
  const int tid = Tid();
  if (tid < kWave) {
    const int lane = tid;
    const int r16 = lane % 16;
    const int octet = lane / 16;
    const int pairs = (a.feat + 63) / 64;
    const std::uint8_t* unit =
        a.w.in_w + static_cast<std::size_t>(group) * pairs * kUnitBytes;
    F32x4 acc{0.0F, 0.0F, 0.0F, 0.0F};
    const F32x4 zero{0.0F, 0.0F, 0.0F, 0.0F};
    for (int pair = 0; pair < pairs; ++pair) {
      const std::uint8_t* u = unit + static_cast<std::size_t>(pair) * kUnitBytes;
      const uint4 wv = *reinterpret_cast<const uint4*>(u + 16 * lane);
      const std::uint32_t scales =
          *reinterpret_cast<const std::uint32_t*>(u + kValueBytes + 4 * r16);
      uint4 xa[2];
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int column = 64 * pair + 32 * hf + 8 * octet;
        float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (r16 < a.patch && column < a.feat) {
          const float4* source = reinterpret_cast<const float4*>(
              a.x + static_cast<std::size_t>(r16) * a.feat + column);
          const float4 lo = source[0];
          const float4 hi = source[1];
          v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
          v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
        }
        xa[hf] = q8::PackBf16x8(v);
      }
      const F32x4 sum0 = Mfma16x16x32(AsBf16x8(xa[0]), Int8x8ToBf16(wv.x, wv.y), zero);
      const F32x4 sum1 = Mfma16x16x32(AsBf16x8(xa[1]), Int8x8ToBf16(wv.z, wv.w), zero);
      const float s0 = HalfValue(static_cast<std::uint16_t>(scales & 0xFFFFU));
      const float s1 = HalfValue(static_cast<std::uint16_t>(scales >> 16));
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[i] = fmaf(s0, sum0[i], acc[i]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[i] = fmaf(s1, sum1[i], acc[i]);
    }
    const int column = 16 * group + r16;
    const float bias = a.w.in_b != nullptr ? Bf16Value(a.w.in_b[column]) : 0.0F;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * octet + i;
      if (row >= a.patch)
        continue;
      const float value = acc[i] + bias;
      staging[(3 + a.patch + row) * 16 + r16] = value;
      staging[(a.length + 3 + a.patch + row) * 16 + r16] = value;
    }
  } else {
    const int fixed = 3 + a.patch;  // mu, mu, time, condition rows
    for (int e = tid - kWave; e < 2 * fixed * 16; e += kThreads - kWave) {
      const int branch = e / (fixed * 16);
      const int row = (e / 16) % fixed;
      const int c = 16 * group + e % 16;
      float value;
      if (row < 2)
        value = branch == 0 ? a.mu[static_cast<std::size_t>(row) * a.hidden + c] : 0.0F;
      else if (row == 2)
        value = a.time[c];
      else
        value = a.cond[static_cast<std::size_t>(row - 3) * a.hidden + c];
      staging[(branch * a.length + row) * 16 + e % 16] = value;
    }
  }
  __syncthreads();
  BlockToF32Frag(staging, a.rows, group, nullptr, h);
}

/// qkv group `tile` = rmsnorm(h) Wqkv^T, stored tile-major [groups][32][16].
__device__ void PhaseAttention(const Args& a, const float* qkv, Bf16* out, int head,
                               float* lds);

/// qkv group `tile` = rmsnorm(h) Wqkv^T, stored tile-major [groups][32][16];
/// then, by the last tile of each head, that head's attention.
template<int PA>
__device__ void PhaseQkv(const Args& a, const Stage<1, PA>& st, const float* h,
                         const Bf16* norm, float* qkv, int tile, float* lds,
                         unsigned long long* mark, unsigned* head_arrivals,
                         Bf16* attention) {
  uint4 operands[PA][2][2];
  NormOperands<PA>(h, norm, a.hidden, a.rows, a.eps, lds + kSquaresAt, operands);
  Mark(mark, 2);
  F32x4 acc[1][2];
  Multiply<1, PA>(st, operands, a.hidden / 64, acc);
  WaveSums<1>(lds, acc);
  Mark(mark, 3);
  float* staging = lds + kStageAt;
  staging[Tid()] = Total<1>(lds, Slot(0, BlockRow(), BlockColumn()));
  __syncthreads();
  BlockToTile(staging, a.rows, tile, qkv);
  // Count this tile in for every head it feeds (a q tile one head, a k or
  // v tile the heads sharing its kv head); the last tile of a head to
  // arrive runs that head's attention.
  WaitStores();
  __syncthreads();
  int* flags = reinterpret_cast<int*>(lds + kFlagsAt);
  const int group_heads = a.heads / a.kv_heads;
  const int column = 16 * tile;
  int first_head, count;
  if (column < a.q_width) {
    first_head = column / a.head_dim;
    count = 1;
  } else {
    const int kv = ((column - a.q_width) % (a.kv_heads * a.head_dim)) / a.head_dim;
    first_head = kv * group_heads;
    count = group_heads;
  }
  const unsigned tiles_per_head = 3U * static_cast<unsigned>(a.head_dim / 16);
  if (Tid() < count) {
    const unsigned before = __hip_atomic_fetch_add(head_arrivals + first_head + Tid(), 1U,
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    flags[4 + Tid()] = (before + 1U) % tiles_per_head == 0U ? 1 : 0;
  }
  __syncthreads();
  for (int h = 0; h < count; ++h) {
    if (flags[4 + h] == 0)
      continue;
    // Every tile of the head was written whole and finished before its
    // workgroup arrived; none was read on this die before, so plain loads
    // see them.
    PhaseAttention(a, qkv, attention, first_head + h, lds);
    __syncthreads();
  }
}

/// Rotary embedding and attention of head `head` for both branches (each
/// over its own keys, bidirectional), output bf16 fragment order
/// [32][q width]. The rotated, scaled queries, rotated keys and values of
/// the rows go to LDS (rows padded to a multiple of 4 floats); each (query,
/// key) score is two threads' halves of the dot product with 16-byte LDS
/// reads in flight together; the softmax runs over the 16 key lanes of a
/// query; each output octet of dimensions is two threads' halves of the
/// keys; the head's output block is then written in whole lines.
__device__ void PhaseAttention(const Args& a, const float* qkv, Bf16* out, int head,
                               float* lds) {
  const int tid = Tid();
  const int dims = a.head_dim;
  const int half = dims / 2;
  const int kv_head = head / (a.heads / a.kv_heads);
  const int stride = dims + 4;
  float* qs = lds;                                  // [32][stride]
  float* ks = qs + 32 * stride;                     // [32][stride]
  float* vs = ks + 32 * stride;                     // [32][stride]
  float* weights = vs + 32 * stride;                // [2][16][16]
  float* inverse = weights + 2 * kMaxLength * kMaxLength;  // [32]
  Bf16* result = reinterpret_cast<Bf16*>(inverse + 32);    // [32][dims]
  const int quads = half / 4;
  const int items = a.rows * quads;
  for (int e = tid; e < items; e += kThreads) {
    const int r = e / quads;  // row of the pair
    const int position = r % a.length;
    const int d = 4 * (e % quads);
    const float4 q0 = TileQuad(qkv, r, head * dims + d);
    const float4 q1 = TileQuad(qkv, r, head * dims + half + d);
    const float4 k0 = TileQuad(qkv, r, (a.heads + kv_head) * dims + d);
    const float4 k1 = TileQuad(qkv, r, (a.heads + kv_head) * dims + half + d);
    const float4 v0 = TileQuad(qkv, r, (a.heads + a.kv_heads + kv_head) * dims + d);
    const float4 v1 = TileQuad(qkv, r, (a.heads + a.kv_heads + kv_head) * dims + half + d);
    float4 c{1.0F, 1.0F, 1.0F, 1.0F};
    float4 sn{0.0F, 0.0F, 0.0F, 0.0F};
    if (a.w.rope != nullptr) {
      const float* table = a.w.rope + static_cast<std::size_t>(position) * dims;
      c = *reinterpret_cast<const float4*>(table + d);
      sn = *reinterpret_cast<const float4*>(table + half + d);
    }
    const float qa[4] = {q0.x, q0.y, q0.z, q0.w};
    const float qb[4] = {q1.x, q1.y, q1.z, q1.w};
    const float ka[4] = {k0.x, k0.y, k0.z, k0.w};
    const float kb[4] = {k1.x, k1.y, k1.z, k1.w};
    const float cs[4] = {c.x, c.y, c.z, c.w};
    const float ss[4] = {sn.x, sn.y, sn.z, sn.w};
    float q_first[4], q_second[4], k_first[4], k_second[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      q_first[j] = qa[j];
      q_second[j] = qb[j];
      k_first[j] = ka[j];
      k_second[j] = kb[j];
      if (a.w.rope != nullptr) {
        // (a, b) at (i, i + half) -> (a c - b s, b c + a s)
        q_first[j] = qa[j] * cs[j] - qb[j] * ss[j];
        q_second[j] = qb[j] * cs[j] + qa[j] * ss[j];
        k_first[j] = ka[j] * cs[j] - kb[j] * ss[j];
        k_second[j] = kb[j] * cs[j] + ka[j] * ss[j];
      }
    }
    const float scale = a.attention_scale;
    *reinterpret_cast<float4*>(qs + r * stride + d) =
        float4{q_first[0] * scale, q_first[1] * scale, q_first[2] * scale, q_first[3] * scale};
    *reinterpret_cast<float4*>(qs + r * stride + half + d) =
        float4{q_second[0] * scale, q_second[1] * scale, q_second[2] * scale,
               q_second[3] * scale};
    *reinterpret_cast<float4*>(ks + r * stride + d) =
        float4{k_first[0], k_first[1], k_first[2], k_first[3]};
    *reinterpret_cast<float4*>(ks + r * stride + half + d) =
        float4{k_second[0], k_second[1], k_second[2], k_second[3]};
    *reinterpret_cast<float4*>(vs + r * stride + d) = v0;
    *reinterpret_cast<float4*>(vs + r * stride + half + d) = v1;
  }
  __syncthreads();
  {
    // Scores: thread t -> branch t / 256, query i = (t / 16) % 16, key
    // j = t % 16; the whole dot product, four independent partial sums.
    const int branch = tid / 256;
    const int i = (tid / 16) % kMaxLength;
    const int j = tid % kMaxLength;
    const bool valid = i < a.length && j < a.length;
    float partial[4] = {0.0F, 0.0F, 0.0F, 0.0F};
    if (valid) {
      const int base = branch * a.length;
      const float4* qp = reinterpret_cast<const float4*>(qs + (base + i) * stride);
      const float4* kp = reinterpret_cast<const float4*>(ks + (base + j) * stride);
      for (int c = 0; c < 2 * quads; c += 4) {
        float4 qv[4], kv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          qv[u] = qp[c + u];
          kv[u] = kp[c + u];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
          partial[u] += qv[u].x * kv[u].x + qv[u].y * kv[u].y + qv[u].z * kv[u].z +
                        qv[u].w * kv[u].w;
      }
    }
    const float score = valid ? (partial[0] + partial[1]) + (partial[2] + partial[3]) : -INFINITY;
    float maximum = score;
#pragma unroll
    for (int offset = 1; offset < kMaxLength; offset *= 2)
      maximum = fmaxf(maximum, __shfl_xor(maximum, offset, kWave));
    const float weight = valid ? expf(score - maximum) : 0.0F;
    float sum = weight;
#pragma unroll
    for (int offset = 1; offset < kMaxLength; offset *= 2)
      sum += __shfl_xor(sum, offset, kWave);
    weights[(branch * kMaxLength + i) * kMaxLength + j] = weight;
    if (j == 0 && i < a.length)
      inverse[branch * a.length + i] = 1.0F / sum;
  }
  __syncthreads();
  // Weighted values: thread -> (row, octet of dimensions, half of the
  // keys); the halves meet through one lane shuffle.
  const int octets = dims / 8;
  const int units = a.rows * octets * 2;
  for (int e = tid; e < ((units + kWave - 1) / kWave) * kWave; e += kThreads) {
    const bool active = e < units;
    const int part = e % 2;
    const int r = active ? e / 2 / octets : 0;
    const int branch = r / a.length;
    const int i = r % a.length;
    const int d = active ? 8 * ((e / 2) % octets) : 0;
    float o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < kMaxLength / 2; ++u) {
      const int j = part * (kMaxLength / 2) + u;
      if (active && j < a.length) {
        const float w = weights[(branch * kMaxLength + i) * kMaxLength + j];
        const float* vrow = vs + (branch * a.length + j) * stride + d;
        const float4 lo = *reinterpret_cast<const float4*>(vrow);
        const float4 hi = *reinterpret_cast<const float4*>(vrow + 4);
        o[0] += w * lo.x; o[1] += w * lo.y; o[2] += w * lo.z; o[3] += w * lo.w;
        o[4] += w * hi.x; o[5] += w * hi.y; o[6] += w * hi.z; o[7] += w * hi.w;
      }
    }
#pragma unroll
    for (int x = 0; x < 8; ++x)
      o[x] += __shfl_xor(o[x], 1, kWave);
    if (active && part == 0) {
#pragma unroll
      for (int x = 0; x < 8; ++x)
        o[x] *= inverse[r];
      *reinterpret_cast<uint4*>(result + r * dims + d) = q8::PackBf16x8(o);
    }
  }
  __syncthreads();
  // The head's block [32][dims] in whole lines: thread -> (tile t, octet,
  // row r16), rows past the pair as zeros.
  for (int e = tid; e < 2 * octets * 16; e += kThreads) {
    const int r16 = e % 16;
    const int octet = (e / 16) % octets;
    const int row = 16 * (e / (16 * octets)) + r16;
    const uint4 v = row < a.rows
                        ? *reinterpret_cast<const uint4*>(result + row * dims + 8 * octet)
                        : uint4{0U, 0U, 0U, 0U};
    Store16(out + BfFragIndex(row, head * dims + 8 * octet), v);
  }
}

/// h_out = h_in + act W^T for the 16 columns of group `tile` (act bf16
/// fragment order [32][k]).
template<int P>
__device__ void PhaseResidual(const Args& a, const Stage<1, P>& st,
                              const Bf16* act, int k, const float* h_in,
                              float* h_out, int tile, float* lds,
                              unsigned long long* mark) {
  uint4 operands[P][2][2];
  FragOperands<P>(act, 0, k / 64, a.rows, operands);
  F32x4 acc[1][2];
  Multiply<1, P>(st, operands, k / 64, acc);
  WaveSums<1>(lds, acc);
  Mark(mark, 3);
  float* staging = lds + kStageAt;
  staging[Tid()] = Total<1>(lds, Slot(0, BlockRow(), BlockColumn()));
  __syncthreads();
  BlockToF32Frag(staging, a.rows, tile, h_in, h_out);
}

/// Split `split` of the down product of group `group`: its k range's
/// partial sums go to partials[split] (tile-major [groups][32][16]); the
/// last of the group's kDownSplits workgroups to arrive (a device-scope
/// counter) adds the partials in split order and writes h_out = h_in + sum.
template<int PE>
__device__ void PhaseDown(const Args& a, const Stage<1, PE>& st, const Bf16* act,
                          const float* h_in, float* h_out, float* partials,
                          unsigned* arrival, int group, int split, float* lds,
                          unsigned long long* mark) {
  const int per_split = a.ffn / 64 / kDownSplits;
  uint4 operands[PE][2][2];
  FragOperands<PE>(act, split * per_split, per_split, a.rows, operands);
  F32x4 acc[1][2];
  Multiply<1, PE>(st, operands, per_split, acc);
  WaveSums<1>(lds, acc);
  Mark(mark, 2);
  float* staging = lds + kStageAt;
  staging[Tid()] = Total<1>(lds, Slot(0, BlockRow(), BlockColumn()));
  __syncthreads();
  const std::size_t split_size = static_cast<std::size_t>(a.hidden) * 32;
  BlockToTile(staging, a.rows, group, partials + split * split_size);
  int* last = reinterpret_cast<int*>(lds + kFlagsAt + 1);
  WaitStores();
  __syncthreads();
  if (Tid() == 0) {
    const unsigned before = __hip_atomic_fetch_add(arrival, 1U, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
    *last = (before + 1U) % kDownSplits == 0U ? 1 : 0;
  }
  __syncthreads();
  Mark(mark, 3);
  if (*last == 0)
    return;
  // Every split's block was written whole by its workgroup before it
  // arrived; none was read here before, so plain loads see it.
  const int row = BlockRow();
  const std::size_t at = (static_cast<std::size_t>(group) * 32 + row) * 16 + BlockColumn();
  float sum = partials[at];
  for (int sp = 1; sp < kDownSplits; ++sp)
    sum += partials[sp * split_size + at];
  staging[Tid()] = sum;
  __syncthreads();
  BlockToF32Frag(staging, a.rows, group, h_in, h_out);
}

/// swiglu of gate group `tile` and its up group (ffn / 16 groups later),
/// bf16 fragment order [32][ffn].
template<int PA>
__device__ void PhaseGateUp(const Args& a, const Stage<2, PA>& st, const float* h,
                            const Bf16* norm, Bf16* out, int tile, float* lds,
                            unsigned long long* mark) {
  uint4 operands[PA][2][2];
  NormOperands<PA>(h, norm, a.hidden, a.rows, a.eps, lds + kSquaresAt, operands);
  Mark(mark, 2);
  F32x4 acc[2][2];
  Multiply<2, PA>(st, operands, a.hidden / 64, acc);
  WaveSums<2>(lds, acc);
  Mark(mark, 3);
  Bf16* staging = reinterpret_cast<Bf16*>(lds + kStageAt);
  const float gate = Total<2>(lds, Slot(0, BlockRow(), BlockColumn()));
  const float up = Total<2>(lds, Slot(1, BlockRow(), BlockColumn()));
  staging[Tid()] = q8::Bf16Fast(q8::Silu(gate) * up);
  __syncthreads();
  BlockToBf16Frag(staging, a.rows, tile, out);
}

/// Final norm of the 2 P output rows, out_proj with its bias, and with
/// x_update the guided Euler step over the whole velocity; one workgroup
/// (kPw pairs per wave: hidden <= 1024 kPw).
template<int kPw>
__device__ void PhaseOut(const Args& a, const float* h, float* lds) {
  float* squares = lds + kSquaresAt;      // [waves][16]
  float* reduce = lds;                    // [waves][kOutGroups][4][64]
  float* velocity = lds + kVelocityAt;    // [2 patch feat]
  float* block = lds + kBlockAt;          // [waves]
  const int lane = Lane();
  const int wave = Wave();
  const int r16 = lane % 16;
  const int octet = lane / 16;
  const int pairs = a.hidden / 64;
  const int groups = (a.feat + 15) / 16;
  const int out_rows = 2 * a.patch;
  // A row r16 (< 2 patch) is branch r16 / patch, output row r16 % patch.
  const bool row_ok = r16 < out_rows;
  const int h_row = row_ok ? (r16 / a.patch) * a.length + 3 + a.patch + r16 % a.patch : 0;
  uint4 wv[kPw][kOutGroups];
  std::uint32_t sc[kPw][kOutGroups];
  float4 hv[kPw][2][2];
#pragma unroll
  for (int p = 0; p < kPw; ++p) {
    const int pair = wave + p * kWaves;
    const bool ok = pair < pairs;
#pragma unroll
    for (int g = 0; g < kOutGroups; ++g) {
      const bool use = ok && g < groups;
      const std::uint8_t* u = a.w.out_w +
          (static_cast<std::size_t>(use ? g : 0) * pairs + (use ? pair : 0)) * kUnitBytes;
      wv[p][g] = use ? *reinterpret_cast<const uint4*>(u + 16 * lane) : uint4{0U, 0U, 0U, 0U};
      sc[p][g] = use ? *reinterpret_cast<const std::uint32_t*>(u + kValueBytes + 4 * r16) : 0U;
    }
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int q = 0; q < 2; ++q)
        hv[p][hf][q] = (ok && row_ok)
                           ? *reinterpret_cast<const float4*>(
                                 h + F32FragIndex(h_row, 64 * pair + 32 * hf + 8 * octet + 4 * q))
                           : float4{0.0F, 0.0F, 0.0F, 0.0F};
  }
  float partial = 0.0F;
#pragma unroll
  for (int p = 0; p < kPw; ++p)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const float4 v = hv[p][hf][q];
        partial += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
      }
  partial += __shfl_xor(partial, 16, kWave);
  partial += __shfl_xor(partial, 32, kWave);
  if (octet == 0)
    squares[wave * 16 + r16] = partial;
  __syncthreads();
  float total = 0.0F;
  for (int w = 0; w < kWaves; ++w)
    total += squares[w * 16 + r16];
  const float inverse = rsqrtf(total / static_cast<float>(a.hidden) + a.eps);
  F32x4 acc[kOutGroups];
#pragma unroll
  for (int g = 0; g < kOutGroups; ++g)
    acc[g] = F32x4{0.0F, 0.0F, 0.0F, 0.0F};
  const F32x4 zero{0.0F, 0.0F, 0.0F, 0.0F};
#pragma unroll
  for (int p = 0; p < kPw; ++p) {
    const int pair = wave + p * kWaves;
    if (pair >= pairs)
      continue;
    uint4 xa[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const uint4 gw =
          *reinterpret_cast<const uint4*>(a.w.final_norm + 64 * pair + 32 * hf + 8 * octet);
      const float gamma[8] = {q8::Bf16Lo(gw.x), q8::Bf16Hi(gw.x), q8::Bf16Lo(gw.y),
                              q8::Bf16Hi(gw.y), q8::Bf16Lo(gw.z), q8::Bf16Hi(gw.z),
                              q8::Bf16Lo(gw.w), q8::Bf16Hi(gw.w)};
      const float4 lo = hv[p][hf][0];
      const float4 hi = hv[p][hf][1];
      const float x8[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        v[i] = x8[i] * inverse * gamma[i];
      xa[hf] = row_ok ? q8::PackBf16x8(v) : uint4{0U, 0U, 0U, 0U};
    }
#pragma unroll
    for (int g = 0; g < kOutGroups; ++g) {
      if (g >= groups)
        continue;
      const float s0 = HalfValue(static_cast<std::uint16_t>(sc[p][g] & 0xFFFFU));
      const float s1 = HalfValue(static_cast<std::uint16_t>(sc[p][g] >> 16));
      const F32x4 sum0 =
          Mfma16x16x32(AsBf16x8(xa[0]), Int8x8ToBf16(wv[p][g].x, wv[p][g].y), zero);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[g][i] = fmaf(s0, sum0[i], acc[g][i]);
      const F32x4 sum1 =
          Mfma16x16x32(AsBf16x8(xa[1]), Int8x8ToBf16(wv[p][g].z, wv[p][g].w), zero);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[g][i] = fmaf(s1, sum1[i], acc[g][i]);
    }
  }
#pragma unroll
  for (int g = 0; g < kOutGroups; ++g)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      reduce[((wave * kOutGroups + g) * 4 + i) * kWave + lane] = acc[g][i];
  __syncthreads();
  const int values = a.patch * a.feat;  // per branch
  for (int e = Tid(); e < kOutGroups * 256; e += kThreads) {
    const int g = e / 256;
    const int i = (e / 64) % 4;
    const int l = e % 64;
    const int row = 4 * (l / 16) + i;
    const int column = 16 * g + l % 16;
    if (row >= out_rows || column >= a.feat)
      continue;
    float v = reduce[((0 * kOutGroups + g) * 4 + i) * kWave + l];
    for (int w = 1; w < kWaves; ++w)
      v += reduce[((w * kOutGroups + g) * 4 + i) * kWave + l];
    if (a.w.out_b != nullptr)
      v += Bf16Value(a.w.out_b[column]);
    const int at = row * a.feat + column;  // [branch][patch][feat]
    a.velocity[at] = v;
    velocity[at] = v;
  }
  if (a.x_update == nullptr)
    return;
  __syncthreads();
  const float* c = velocity;
  const float* u = velocity + values;
  float s = 1.0F;
  if (a.zero_star) {
    float dot = 0.0F;
    float norm = 0.0F;
    for (int i = Tid(); i < values; i += kThreads) {
      dot += c[i] * u[i];
      norm += u[i] * u[i];
    }
    dot = BlockSum(dot, block);
    norm = BlockSum(norm, block);
    s = dot / (norm + 1e-8F);
  }
  for (int i = Tid(); i < values; i += kThreads) {
    const float guided = u[i] * s + a.cfg * (c[i] - u[i] * s);
    a.x_update[i] -= a.dt * guided;
  }
}

// ---- the kernel -------------------------------------------------------------------------

template<int PA, int PC, int PE>
__global__ __launch_bounds__(kThreads) void EvaluateKernel(Args a) {
  extern __shared__ float lds[];
  int* quit = reinterpret_cast<int*>(lds + kFlagsAt);
  unsigned* sync = a.ws.sync;
  if (LoadU32(sync + kErrorWord) != 0U)
    return;  // a previous launch timed out: the host resets the area
  const unsigned generation = LoadU32(sync + kGenerationWord);
  const unsigned barriers = 1U + 4U * static_cast<unsigned>(a.layers);
  unsigned long long* trace =
      a.trace != nullptr ? a.trace + static_cast<std::size_t>(blockIdx.x) * 4 * (barriers + 1)
                         : nullptr;
  if (trace != nullptr && threadIdx.x == 0)
    trace[0] = __builtin_amdgcn_s_memrealtime();
  const unsigned base = generation * barriers;
  int index = 0;
  const int wg = static_cast<int>(blockIdx.x);
  const int hidden_groups = a.hidden / 16;
  const int qkv_groups = a.qkv_width / 16;
  const int ffn_groups = a.ffn / 16;
  const int down_tiles = kDownSplits * hidden_groups;
  const std::size_t h_size = Frag(a.hidden);
  const std::size_t qkv_size = static_cast<std::size_t>(32) * a.qkv_width;
  const std::size_t attention_size = Frag(a.q_width);
  const std::size_t swiglu_size = Frag(a.ffn);

  if (wg < hidden_groups)
    PhaseIn(a, wg, a.ws.h, lds);
  WaitStores();
  Stage<1, PA> stage_qkv;
  if (wg < qkv_groups)
    LoadStage<1, PA>(a.w.layers[0].qkv, a.hidden / 64, qkv_groups, 1, wg, stage_qkv);
  if (!GridBarrier(sync, base, ++index, quit, trace))
    return;

  for (int l = 0; l < a.layers; ++l) {
    const Layer layer = a.w.layers[l];
    const float* h_in = a.ws.h + static_cast<std::size_t>(2 * l) * h_size;
    float* h_mid = a.ws.h + static_cast<std::size_t>(2 * l + 1) * h_size;
    float* h_out = a.ws.h + static_cast<std::size_t>(2 * l + 2) * h_size;
    float* qkv = a.ws.qkv + static_cast<std::size_t>(l) * qkv_size;
    Bf16* attention = a.ws.attention + static_cast<std::size_t>(l) * attention_size;
    Bf16* swiglu = a.ws.swiglu + static_cast<std::size_t>(l) * swiglu_size;

    if (wg < qkv_groups)
      PhaseQkv<PA>(a, stage_qkv, h_in, layer.input_norm, qkv, wg, lds,
                   trace != nullptr ? trace + 4 * (index + 1) : nullptr,
                   sync + kArrivalsWord + a.layers * hidden_groups + l * a.heads, attention);
    WaitStores();
    Stage<1, PC> stage_o;
    if (wg < hidden_groups)
      LoadStage<1, PC>(layer.o, a.q_width / 64, hidden_groups, 1, wg, stage_o);
    if (!GridBarrier(sync, base, ++index, quit, trace))
      return;

    if (wg < hidden_groups)
      PhaseResidual<PC>(a, stage_o, attention, a.q_width, h_in, h_mid, wg, lds,
                        trace != nullptr ? trace + 4 * (index + 1) : nullptr);
    WaitStores();
    Stage<2, PA> stage_gate_up;
    if (wg < ffn_groups)
      LoadStage<2, PA>(layer.gate_up, a.hidden / 64, 2 * ffn_groups, ffn_groups, wg,
                       stage_gate_up);
    if (!GridBarrier(sync, base, ++index, quit, trace))
      return;

    if (wg < ffn_groups)
      PhaseGateUp<PA>(a, stage_gate_up, h_mid, layer.post_norm, swiglu, wg, lds,
                      trace != nullptr ? trace + 4 * (index + 1) : nullptr);
    WaitStores();
    Stage<1, PE> stage_down;
    const int per_split = a.ffn / 64 / kDownSplits;
    if (wg < down_tiles)
      LoadStage<1, PE>(layer.down, a.ffn / 64, hidden_groups, 1, wg % hidden_groups,
                       stage_down, (wg / hidden_groups) * per_split, per_split);
    if (!GridBarrier(sync, base, ++index, quit, trace))
      return;

    if (wg < down_tiles)
      PhaseDown<PE>(a, stage_down, swiglu, h_mid, h_out,
                    a.ws.partials + static_cast<std::size_t>(l) * kDownSplits * 32 * a.hidden,
                    sync + kArrivalsWord + l * hidden_groups + wg % hidden_groups,
                    wg % hidden_groups, wg / hidden_groups, lds,
                    trace != nullptr ? trace + 4 * (index + 1) : nullptr);
    WaitStores();
    if (l + 1 < a.layers && wg < qkv_groups)
      LoadStage<1, PA>(a.w.layers[l + 1].qkv, a.hidden / 64, qkv_groups, 1, wg, stage_qkv);
    if (!GridBarrier(sync, base, ++index, quit, trace))
      return;
  }

  if (wg == 0) {
    PhaseOut<PA>(a, a.ws.h + static_cast<std::size_t>(2 * a.layers) * h_size, lds);
    if (threadIdx.x == 0)
      StoreU32(sync + kGenerationWord, generation + 1U);
  }
  if (trace != nullptr && threadIdx.x == 0)
    trace[1] = __builtin_amdgcn_s_memrealtime();
}

using Kernel = void (*)(Args);

template<int PA, int PC, int PE>
Kernel Prepared() {
  static const hipError_t status = hipFuncSetAttribute(
      reinterpret_cast<const void*>(EvaluateKernel<PA, PC, PE>),
      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kLdsBytes));
  return status == hipSuccess ? EvaluateKernel<PA, PC, PE> : nullptr;
}

int PairsPerWave(int k) { return (k / 64 + kWaves - 1) / kWaves; }

Kernel Pick(const fused::Shape& s) {
  const int pa = PairsPerWave(s.hidden);
  const int pc = PairsPerWave(s.heads * s.head_dim);
  const int pe = PairsPerWave(s.ffn / kDownSplits);
  if (pa == 2 && pc == 2 && pe == 2)
    return Prepared<2, 2, 2>();
  if (pa == 2 && pc == 4 && pe == 2)
    return Prepared<2, 4, 2>();
  if (pa == 1 && pc == 1 && pe <= 2)
    return Prepared<1, 1, 2>();
  if (pa == 1 && pc == 2 && pe <= 2)
    return Prepared<1, 2, 2>();
  if (pa == 2 && pc <= 2 && pe <= 2)
    return Prepared<2, 2, 2>();
  if (pa <= 2 && pc <= 4 && pe <= 2)
    return Prepared<2, 4, 2>();
  return nullptr;
}

}  // namespace

std::size_t SyncWords(const fused::Shape& s, int layers) {
  return kArrivalsWord + static_cast<std::size_t>(layers) * (s.hidden / 16 + s.heads);
}
std::size_t ErrorWord() { return kErrorWord; }
std::size_t PartialElements(const fused::Shape& s, int layers) {
  return static_cast<std::size_t>(layers) * kDownSplits * 32 * s.hidden;
}

std::size_t HElements(const fused::Shape& s, int layers) {
  return static_cast<std::size_t>(2 * layers + 1) * Frag(s.hidden);
}
std::size_t QkvElements(const fused::Shape& s, int layers) {
  return static_cast<std::size_t>(layers) * 32 * (s.heads + 2 * s.kv_heads) * s.head_dim;
}
std::size_t AttentionElements(const fused::Shape& s, int layers) {
  return static_cast<std::size_t>(layers) * Frag(s.heads * s.head_dim);
}
std::size_t SwigluElements(const fused::Shape& s, int layers) {
  return static_cast<std::size_t>(layers) * Frag(s.ffn);
}

bool Supported(const fused::Shape& s, int layers, int grid) {
  if (!fused::Supported(s) || layers < 1 || layers > kMaxLayers || grid < 1 ||
      grid > kMaxGrid)
    return false;
  const int q_width = s.heads * s.head_dim;
  const int qkv_width = (s.heads + 2 * s.kv_heads) * s.head_dim;
  if (qkv_width % 16 != 0 || s.head_dim % 16 != 0 || s.heads / s.kv_heads > 8)
    return false;
  if (kDownSplits * (s.hidden / 16) > grid || qkv_width / 16 > grid ||
      s.ffn / 16 > grid || s.heads > grid)
    return false;
  if (PairsPerWave(s.hidden) > 2 || PairsPerWave(q_width) > 4 ||
      (s.ffn / 64) % kDownSplits != 0 || PairsPerWave(s.ffn / kDownSplits) > 2)
    return false;
  // The attention phase's LDS (queries, keys, values, weights, inverse
  // sums, the bf16 output block) ends before the flags.
  const int stage = 3 * 32 * (s.head_dim + 4) + 2 * kMaxLength * kMaxLength + 32 +
                    16 * s.head_dim;
  return stage <= kFlagsAt;
}

int GridSize() {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess)
    return 0;
  int units = 0;
  if (hipDeviceGetAttribute(&units, hipDeviceAttributeMultiprocessorCount, device) !=
      hipSuccess)
    return 0;
  return std::min(units, kMaxGrid);
}

bool Prepare(const fused::Shape& s) {
  const Kernel kernel = Pick(s);
  if (kernel == nullptr)
    return false;
  // Every workgroup of the grid must be resident at once, or the grid
  // barriers would wait for workgroups that cannot start: one workgroup
  // of this size and LDS per compute unit, and the grid no larger than
  // the compute units.
  int per_unit = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_unit, kernel, kThreads, kLdsBytes) !=
      hipSuccess)
    return false;
  int device = 0;
  int units = 0;
  if (hipGetDevice(&device) != hipSuccess ||
      hipDeviceGetAttribute(&units, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
    return false;
  return per_unit >= 1 && GridSize() <= units * per_unit;
}

std::size_t TraceWords(int layers, int grid) {
  return static_cast<std::size_t>(grid) * 4 * (2 + 4 * static_cast<std::size_t>(layers));
}

int Evaluate(const fused::Shape& s, int layers, int grid, const Weights& w,
             const Workspace& ws, const float* mu, const float* time,
             const float* cond_rows, const float* x, float* velocity,
             float* x_update, float cfg, float dt, int zero_star,
             unsigned long long* trace, hipStream_t stream) {
  const Kernel kernel = Pick(s);
  if (kernel == nullptr || !Supported(s, layers, grid))
    return Fail(VX_UNSUPPORTED, "persistent DiT evaluation: shape not supported");
  Args a{};
  a.rows = s.rows;
  a.length = s.length;
  a.patch = s.patch;
  a.hidden = s.hidden;
  a.heads = s.heads;
  a.kv_heads = s.kv_heads;
  a.head_dim = s.head_dim;
  a.ffn = s.ffn;
  a.feat = s.feat;
  a.layers = layers;
  a.q_width = s.heads * s.head_dim;
  a.qkv_width = (s.heads + 2 * s.kv_heads) * s.head_dim;
  a.eps = s.eps;
  a.attention_scale = 1.0F / std::sqrt(static_cast<float>(s.head_dim));
  a.w = w;
  a.mu = mu;
  a.time = time;
  a.cond = cond_rows;
  a.x = x;
  a.velocity = velocity;
  a.x_update = x_update;
  a.cfg = cfg;
  a.dt = dt;
  a.zero_star = zero_star;
  a.ws = ws;
  a.trace = trace;
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(grid)), dim3(kThreads),
                     kLdsBytes, stream, a);
  return LaunchStatus("persistent DiT evaluation");
}

}  // namespace vx::persistent
