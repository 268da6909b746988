// One DiT evaluation as one persistent launch (dit_persistent.hpp).
//
// Phases of a launch, each ended by a grid barrier:
//   in      in_proj of x and the assembly of the 2 (3 + 2 P) rows, with the
//           first layer's norm operand (generator.cpp:297-316;
//           kernels/generator_kernels.hip:320-340);
//   per layer (transformer.cpp:74-96):
//   qkv     (bf16(h gamma) Wqkv^T) rsqrt(mean(h^2) + eps): RMSNorm's row
//           factor after the product (generator_kernels.hip:91-108);
//   attn    rotary embedding and attention per (branch, head)
//           (generator_kernels.hip:110-241);
//   o       h += attn Wo^T, with the post-attention norm's operand;
//   gate_up swiglu of the normalised gate and up products
//           (generator_kernels.hip:243-254);
//   down    h += s Wdown^T, with the next layer's norm operand;
//   then the final norm, out_proj, its bias and the guided Euler step in
//   workgroup 0 (generator.cpp:318-324; generator_kernels.hip:342-360).
//
// Every phase is the body of the fused path's launch (dit_phases.hpp and
// the product engine of q8_tile.hpp) with the same work split, run by the
// first workgroups of the grid; its outputs are device-scope stores. The
// Q8_0 arithmetic is the products' (kernels/wmma_products.hip:192-215).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>

#include "common.hpp"
#include "dit_fused.hpp"
#include "dit_persistent.hpp"
#include "dit_phases.hpp"
#include "q8.hpp"
#include "q8_tile.hpp"

namespace vx::persistent {
namespace {

constexpr int kWaves = fused::kMaxWaves;
constexpr int kThreads = kWaves * kWave;
constexpr int kMaxGrid = 256;
// Barrier arrivals spread over 16 counters 256 bytes apart (workgroup w
// counts in slot w % 16), so no counter takes more than 16 atomics.
constexpr int kSlots = 16;
constexpr int kSlotStride = 64;
constexpr int kGenerationWord = kSlots * kSlotStride;
constexpr int kErrorWord = kGenerationWord + 64;
constexpr int kSyncWords = kErrorWord + 64;
// About a second of polling before a wait gives up (one poll is well under
// a microsecond).
constexpr int kSpinLimit = 1 << 21;
// LDS: the products' wave partial sums (64 KB for two row groups of 32
// rows) or the attention's staging; then the next product's first weights
// (EnginePrefetch: up to 16 waves x 4 units); then the flags. The output
// phase, after the last product, uses everything before the flags. The
// size keeps one workgroup per compute unit.
constexpr int kStageAt = 64 * 1024;  // bytes
constexpr int kStageBytes = q8::PrefetchBytes(1, 4, kWaves);
constexpr int kFlagsAt = (kStageAt + kStageBytes) / static_cast<int>(sizeof(float));
constexpr std::size_t kLdsBytes = static_cast<std::size_t>(kStageAt + kStageBytes) + 64;
static_assert(q8::EngineShared(2, 2, kWaves, q8::ASource::kScaledBf16) <= kStageAt,
              "LDS plan: products");
static_assert(q8::PrefetchBytes(2, 2, kWaves) <= kStageBytes, "LDS plan: staged weights");
static_assert(fused::kOutFloats <= kFlagsAt, "LDS plan: output phase");
static_assert(kLdsBytes > 80 * 1024, "one workgroup per compute unit");

struct Args {
  fused::Shape s;
  int layers, q_width, qkv_width;
  float attention_scale;
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
  // [workgroup][barrier + 1][arrive, leave, products, stores]: arrival at
  // and exit from the barrier, and inside the phase before it the times
  // its products (its work) and its stores were done; slot 0 holds the
  // kernel's start and end. Null: not recorded.
  unsigned long long* trace;
};

// ---- barrier --------------------------------------------------------------------

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

/// Records the time into trace word `at` (thread 0; no-op without a trace).
__device__ inline void Mark(unsigned long long* trace, int at) {
  if (trace != nullptr && threadIdx.x == 0)
    trace[at] = __builtin_amdgcn_s_memrealtime();
}

/// Grid barrier number `index` (1-based within the launch). Every wave has
/// waited for its stores (WaitStores); wave 0 counts the workgroup in and
/// polls the slot counters while the other waves' weight loads for the
/// next product are in flight. Returns false when the launch must stop:
/// the wait timed out (the error word is set) or another workgroup
/// stopped.
__device__ bool GridBarrier(unsigned* sync, unsigned base, int index, int* quit,
                            unsigned long long* trace) {
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
        const unsigned members = static_cast<unsigned>((grid - lane + kSlots - 1) / kSlots);
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

/// Grid barriers of a launch of `layers` layers: after the input assembly,
/// then after each of a layer's five phases.
__host__ __device__ constexpr int BarrierCount(int layers) { return 1 + 5 * layers; }

// ---- phase arguments ------------------------------------------------------------

__host__ __device__ inline std::size_t Frag(int columns) {
  return static_cast<std::size_t>(32) * ((columns + 63) / 64) * 64;
}

__device__ inline Bf16* NormOf(const Args& a, int slot) {
  return a.ws.norm + static_cast<std::size_t>(slot) * Frag(a.s.hidden);
}
__device__ inline float* SquaresOf(const Args& a, int slot) {
  return a.ws.squares + static_cast<std::size_t>(slot) * 32 * (a.s.hidden / 16);
}
__device__ inline float* HOf(const Args& a, int slot) {
  return a.ws.h + static_cast<std::size_t>(slot) * Frag(a.s.hidden);
}

/// `value` as the compiler cannot follow it (it stays in its scalar
/// register): phase arguments derived from a laundered layer index are
/// recomputed where a phase needs them instead of being held in registers
/// across the phases in between, where they would crowd out the products'.
__device__ inline int Opaque(int value) {
  asm volatile("" : "+s"(value));
  return value;
}

/// The thread index as the compiler cannot follow it: the per-lane index
/// arithmetic of each phase is recomputed in the phase instead of being
/// hoisted out of the layer loop and held in registers throughout.
__device__ inline int Thread() {
  int value = static_cast<int>(threadIdx.x);
  asm volatile("" : "+v"(value));
  return value;
}

/// qkv of layer l from the input norm's operand (fused::QkvScaled).
__device__ inline q8::TileArgs QkvArgs(const Args& a, int l) {
  q8::TileArgs t = fused::BaseArgs(a.w.layers[l].qkv, a.s.rows, a.s.hidden, a.qkv_width);
  t.x = NormOf(a, 2 * l);
  t.row_squares = SquaresOf(a, 2 * l);
  t.squares_groups = a.s.hidden / 16;
  t.eps = a.s.eps;
  t.y = a.ws.qkv + static_cast<std::size_t>(l) * 32 * a.qkv_width;
  return t;
}

/// A residual product of layer l (fused::Residual): o (h_mid = h_in +
/// attn Wo^T, with the post-attention norm's operand) or, kDown, down
/// (h_out = h_mid + s Wdown^T, with the next layer's input norm's operand).
template<bool kWide, bool kDown>
__device__ inline q8::TileArgs ResidualArgs(const Args& a, int l) {
  const Layer& layer = a.w.layers[l];
  const int k = kDown ? a.s.ffn : a.q_width;
  q8::TileArgs t = fused::BaseArgs(kDown ? layer.down : layer.o, a.s.rows, k, a.s.hidden);
  t.x = kDown ? a.ws.swiglu + static_cast<std::size_t>(l) * Frag(a.s.ffn)
              : a.ws.attention + static_cast<std::size_t>(l) * Frag(a.q_width);
  const int h_in = kDown ? 2 * l + 1 : 2 * l;
  t.residual_in = HOf(a, h_in);
  t.residual = HOf(a, h_in + 1);
  const Bf16* gamma = !kDown ? layer.post_norm
                             : l + 1 < a.layers ? a.w.layers[l + 1].input_norm : nullptr;
  if (gamma != nullptr) {
    t.norm_out = NormOf(a, h_in + 1);
    t.norm_gamma = gamma;
    t.norm_squares = SquaresOf(a, h_in + 1);
  }
  if constexpr (kWide)
    fused::SetTileBlocks(t, t.groups, a.s.rows);
  else
    fused::SetRowBlocks(t, t.groups, a.s.rows);
  return t;
}

/// gate_up of layer l from the post-attention norm's operand
/// (fused::GateUpScaled).
__device__ inline q8::TileArgs GateUpArgs(const Args& a, int l) {
  q8::TileArgs t = fused::BaseArgs(a.w.layers[l].gate_up, a.s.rows, a.s.hidden, 2 * a.s.ffn);
  t.x = NormOf(a, 2 * l + 1);
  t.row_squares = SquaresOf(a, 2 * l + 1);
  t.squares_groups = a.s.hidden / 16;
  t.eps = a.s.eps;
  t.frag_out = a.ws.swiglu + static_cast<std::size_t>(l) * Frag(a.s.ffn);
  t.group_stride = a.s.ffn / 16;
  return t;
}

// The products' phases. Each issues the first pass of its weights
// (Prefetch, before the grid barriers that precede it) and later runs the
// product on them (Run), with the fused launches' plan: qkv and gate_up
// one tile of 32 rows per workgroup, the residual products tile-aligned
// row blocks with four pairs per wave per pass above 32 pairs (one 16-row
// tile), else row blocks of the 32 rows with one pair per wave per pass.

template<bool kWide, bool kDown>
struct ResidualPlan {
  static constexpr int kMt = kWide ? 1 : 2;
  static constexpr int kPw = kWide ? 4 : 1;
  // The wide plan's four pairs per wave cover k in one pass (Supported
  // asks for at most 64 pairs).
  static constexpr bool kOnePass = kWide;
  __device__ static void Prefetch(const Args& a, int l, int wg, std::uint8_t* stage) {
    const q8::TileArgs t = ResidualArgs<kWide, kDown>(a, Opaque(l));
    const int grid = t.groups * t.row_blocks;
    if (wg < grid)
      q8::EnginePrefetch<kMt, 1, q8::Output::kResidual, kPw>(t, wg, grid, Thread(), stage);
  }
  __device__ static void Run(const Args& a, int l, int wg, const std::uint8_t* stage) {
    const q8::TileArgs t = ResidualArgs<kWide, kDown>(a, Opaque(l));
    const int grid = t.groups * t.row_blocks;
    if (wg < grid)
      q8::EngineBody<kMt, 1, q8::ASource::kFragBf16, q8::Output::kResidual, kPw, 2 * kMt,
                     q8::Weights::kQ8, 0, true, true, kOnePass>(t, wg, grid, Thread(), stage);
  }
};

template<int PA>
struct QkvPlan {
  __device__ static void Prefetch(const Args& a, int l, int wg, std::uint8_t* stage) {
    const q8::TileArgs t = QkvArgs(a, Opaque(l));
    if (wg < t.groups)
      q8::EnginePrefetch<2, 1, q8::Output::kStore, PA>(t, wg, t.groups, Thread(), stage);
  }
  __device__ static void Run(const Args& a, int l, int wg, const std::uint8_t* stage) {
    const q8::TileArgs t = QkvArgs(a, Opaque(l));
    if (wg < t.groups)
      q8::EngineBody<2, 1, q8::ASource::kScaledBf16, q8::Output::kStore, PA, 4,
                     q8::Weights::kQ8, 0, true, true, true>(t, wg, t.groups, Thread(), stage);
  }
};

template<int PA>
struct GateUpPlan {
  __device__ static void Prefetch(const Args& a, int l, int wg, std::uint8_t* stage) {
    const q8::TileArgs t = GateUpArgs(a, Opaque(l));
    if (wg < t.group_stride)
      q8::EnginePrefetch<2, 2, q8::Output::kSwiGlu, PA>(t, wg, t.group_stride, Thread(), stage);
  }
  __device__ static void Run(const Args& a, int l, int wg, const std::uint8_t* stage) {
    const q8::TileArgs t = GateUpArgs(a, Opaque(l));
    if (wg < t.group_stride)
      q8::EngineBody<2, 2, q8::ASource::kScaledBf16, q8::Output::kSwiGlu, PA, 4,
                     q8::Weights::kQ8, 0, true, true, true>(t, wg, t.group_stride, Thread(), stage);
  }
};

// ---- the kernel -------------------------------------------------------------------

/// PA: pairs per wave of qkv and gate_up (k = hidden); kOWide / kDWide:
/// the o / down products take the wide residual plan (k > 32 pairs).
template<int PA, bool kOWide, bool kDWide>
__global__ __launch_bounds__(kThreads) void EvaluateKernel(Args a) {
  extern __shared__ float lds[];
  using Qkv = QkvPlan<PA>;
  using GateUp = GateUpPlan<PA>;
  using OPlan = ResidualPlan<kOWide, false>;
  using DownPlan = ResidualPlan<kDWide, true>;
  int* quit = reinterpret_cast<int*>(lds + kFlagsAt);
  std::uint8_t* stage = reinterpret_cast<std::uint8_t*>(lds) + kStageAt;
  unsigned* sync = a.ws.sync;
  if (LoadU32(sync + kErrorWord) != 0U)
    return;  // a previous launch timed out: the host resets the area
  const unsigned generation = LoadU32(sync + kGenerationWord);
  const unsigned barriers = static_cast<unsigned>(BarrierCount(a.layers));
  unsigned long long* trace =
      a.trace != nullptr ? a.trace + static_cast<std::size_t>(blockIdx.x) * 4 * (barriers + 1)
                         : nullptr;
  Mark(trace, 0);
  const unsigned base = generation * barriers;
  int index = 0;
  const int wg = static_cast<int>(blockIdx.x);
  const int tid = static_cast<int>(threadIdx.x);
  const fused::Shape& s = a.s;
  const auto finish = [&](int next) {
    // The phase's products (or work) are done; then its stores.
    Mark(trace, 4 * next + 2);
    WaitStores();
    Mark(trace, 4 * next + 3);
  };

  // Input assembly, one wave per 16 hidden columns.
  if (wg < s.hidden / 16 && tid < kWave) {
    fused::InArgs in{};
    in.x = a.x;
    in.w = a.w.in_w;
    in.bias = a.w.in_b;
    in.mu = a.mu;
    in.time = a.time;
    in.cond = a.cond;
    in.h = HOf(a, 0);
    in.norm_out = NormOf(a, 0);
    in.norm_gamma = a.w.layers[0].input_norm;
    in.norm_squares = SquaresOf(a, 0);
    in.patch = s.patch;
    in.feat = s.feat;
    in.hidden = s.hidden;
    in.length = s.length;
    fused::InAssembleBody<q8::Weights::kQ8, true>(in, wg, Thread());
  }
  finish(index + 1);
  Qkv::Prefetch(a, 0, wg, stage);
  if (!GridBarrier(sync, base, ++index, quit, trace))
    return;

  for (int l = 0; l < a.layers; ++l) {
    Qkv::Run(a, l, wg, stage);
    finish(index + 1);
    // o's weights are in flight through the attention phase.
    OPlan::Prefetch(a, l, wg, stage);
    if (!GridBarrier(sync, base, ++index, quit, trace))
      return;

    if (wg < 2 * s.heads) {
      fused::AttentionArgs at{};
      at.qkv = a.ws.qkv + static_cast<std::size_t>(l) * 32 * a.qkv_width;
      at.rope = a.w.rope;
      at.out = a.ws.attention + static_cast<std::size_t>(l) * Frag(a.q_width);
      at.length = s.length;
      at.heads = s.heads;
      at.kv_heads = s.kv_heads;
      at.head_dim = s.head_dim;
      at.scale = a.attention_scale;
      fused::AttentionBody<true>(at, wg % 2, wg / 2, lds, Thread(), kThreads);
    }
    finish(index + 1);
    if (!GridBarrier(sync, base, ++index, quit, trace))
      return;

    OPlan::Run(a, l, wg, stage);
    finish(index + 1);
    GateUp::Prefetch(a, l, wg, stage);
    if (!GridBarrier(sync, base, ++index, quit, trace))
      return;

    GateUp::Run(a, l, wg, stage);
    finish(index + 1);
    DownPlan::Prefetch(a, l, wg, stage);
    if (!GridBarrier(sync, base, ++index, quit, trace))
      return;

    DownPlan::Run(a, l, wg, stage);
    finish(index + 1);
    if (l + 1 < a.layers)
      Qkv::Prefetch(a, l + 1, wg, stage);
    if (!GridBarrier(sync, base, ++index, quit, trace))
      return;
  }

  if (wg == 0) {
    fused::OutArgs out{};
    out.h = HOf(a, 2 * a.layers);
    out.norm = a.w.final_norm;
    out.w = a.w.out_w;
    out.bias = a.w.out_b;
    out.velocity = a.velocity;
    out.x = a.x_update;
    out.cfg = a.cfg;
    out.dt = a.dt;
    out.eps = s.eps;
    out.zero_star = a.zero_star;
    out.patch = s.patch;
    out.feat = s.feat;
    out.hidden = s.hidden;
    out.length = s.length;
    fused::OutEulerBody<q8::Weights::kQ8>(out, lds);
    if (threadIdx.x == 0)
      StoreU32(sync + kGenerationWord, generation + 1U);
  }
  if (trace != nullptr && threadIdx.x == 0)
    trace[1] = __builtin_amdgcn_s_memrealtime();
}

using Kernel = void (*)(Args);

template<int PA, bool kOWide, bool kDWide>
Kernel Prepared() {
  static const hipError_t status = hipFuncSetAttribute(
      reinterpret_cast<const void*>(EvaluateKernel<PA, kOWide, kDWide>),
      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kLdsBytes));
  return status == hipSuccess ? EvaluateKernel<PA, kOWide, kDWide> : nullptr;
}

/// The residual products' plan, as fused::Residual picks it.
bool Wide(int k) { return fused::PairsOf(k) > 2 * kWaves; }

Kernel Pick(const fused::Shape& s) {
  const int pa = fused::PairsOf(s.hidden) <= kWaves ? 1 : 2;
  const bool o_wide = Wide(s.heads * s.head_dim);
  const bool d_wide = Wide(s.ffn);
  if (pa == 1) {
    if (!o_wide && d_wide)
      return Prepared<1, false, true>();
    if (!o_wide && !d_wide)
      return Prepared<1, false, false>();
    return Prepared<1, true, true>();
  }
  if (!o_wide && d_wide)
    return Prepared<2, false, true>();
  if (!o_wide && !d_wide)
    return Prepared<2, false, false>();
  return Prepared<2, true, true>();
}

/// Workgroups of a residual product phase of k columns (fused::Residual's
/// grid).
int ResidualGrid(const fused::Shape& s, int k) {
  q8::TileArgs t = fused::BaseArgs(nullptr, s.rows, k, s.hidden);
  if (Wide(k))
    fused::SetTileBlocks(t, t.groups, s.rows);
  else
    fused::SetRowBlocks(t, t.groups, s.rows);
  return t.groups * t.row_blocks;
}

}  // namespace

int Barriers(int layers) { return BarrierCount(layers); }

std::size_t SyncWords(const fused::Shape& /*s*/, int /*layers*/) { return kSyncWords; }
std::size_t ErrorWord() { return kErrorWord; }

std::size_t HElements(const fused::Shape& s, int layers) {
  return static_cast<std::size_t>(2 * layers + 1) * Frag(s.hidden);
}
std::size_t NormElements(const fused::Shape& s, int layers) {
  return static_cast<std::size_t>(2 * layers) * Frag(s.hidden);
}
std::size_t SquaresElements(const fused::Shape& s, int layers) {
  return static_cast<std::size_t>(2 * layers) * 32 * (s.hidden / 16);
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
  if (!fused::Supported(s) || s.weights != q8::Weights::kQ8 || layers < 1 ||
      layers > kMaxLayers || grid < 1 || grid > kMaxGrid)
    return false;
  const int q_width = s.heads * s.head_dim;
  const int qkv_width = (s.heads + 2 * s.kv_heads) * s.head_dim;
  // qkv and gate_up take k = hidden in one pass of at most two pairs per
  // wave, the wide residual plan at most four.
  if (qkv_width % 16 != 0 || fused::PairsOf(s.hidden) > 2 * kWaves ||
      (Wide(q_width) && fused::PairsOf(q_width) > 4 * kWaves) ||
      (Wide(s.ffn) && fused::PairsOf(s.ffn) > 4 * kWaves))
    return false;
  // Every phase's workgroups fit the grid.
  if (s.hidden / 16 > grid || qkv_width / 16 > grid || 2 * s.heads > grid ||
      s.ffn / 16 > grid || ResidualGrid(s, q_width) > grid || ResidualGrid(s, s.ffn) > grid)
    return false;
  // The attention's staging fits the LDS before the flags.
  return fused::AttentionFloats(s.head_dim) <= kFlagsAt;
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
  return static_cast<std::size_t>(grid) * 4 * (static_cast<std::size_t>(Barriers(layers)) + 1);
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
  a.s = s;
  a.layers = layers;
  a.q_width = s.heads * s.head_dim;
  a.qkv_width = (s.heads + 2 * s.kv_heads) * s.head_dim;
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
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(grid)), dim3(kThreads), kLdsBytes,
                     stream, a);
  return LaunchStatus("persistent DiT evaluation");
}

}  // namespace vx::persistent
