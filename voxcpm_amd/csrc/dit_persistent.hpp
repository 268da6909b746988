// One DiT evaluation (the CFG pair through every layer, the output
// projection and the guided Euler step) as a single persistent launch: one
// workgroup of 16 waves per compute unit running the fused path's kernel
// bodies as phases (input assembly; per layer qkv, attention, o, gate_up,
// down; the output projection with the Euler step), separated by grid
// barriers. Each product phase's first Q8_0 weights are loaded into
// registers as soon as the previous product phase has stored its outputs,
// so that their latency overlaps the barriers in between. The arithmetic
// and the work split of every phase are the fused launches' (dit_fused.hip),
// so the two paths give the same bits.
//
// Workspace buffers are written once per launch (one buffer per layer and
// phase). Producers store with device-scope (relaxed atomic) stores, which
// write through the compute die's L2, and finish them before arriving at
// the barrier; consumers read with ordinary cached loads. A buffer is never
// read before the barrier after its producer, so no L2 holds a stale copy
// of it during the launch, and the kernel boundary clears the L2s between
// launches.
#ifndef VOXCPM_AMD_DIT_PERSISTENT_HPP_
#define VOXCPM_AMD_DIT_PERSISTENT_HPP_

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "common.hpp"
#include "dit_fused.hpp"

namespace vx::persistent {

/// Device pointers of one layer (vx_dit_layer on the device).
struct Layer {
  const Bf16* input_norm;
  const std::uint8_t* qkv;
  const std::uint8_t* o;
  const Bf16* post_norm;
  const std::uint8_t* gate_up;
  const std::uint8_t* down;
};

/// Layers a persistent launch takes: their pointers travel in the kernel
/// arguments, so that the kernel reads them with scalar loads.
constexpr int kMaxLayers = 32;

struct Weights {
  Layer layers[kMaxLayers];
  const std::uint8_t* in_w;
  const Bf16* in_b;
  const std::uint8_t* out_w;
  const Bf16* out_b;
  const Bf16* final_norm;
  const float* rope;  // or null
};

/// Workspace of one handle: write-once buffers per launch, the barrier
/// counters and the error word.
struct Workspace {
  float* h;          // [2 layers + 1][32 hidden] float32 fragment order: the
                     // assembly, then per layer after o and after down
  Bf16* norm;        // [2 layers][32 hidden] bf16 fragment order: the norm
                     // operands bf16(h gamma) of layer l's input norm (2 l)
                     // and post-attention norm (2 l + 1)
  float* squares;    // [2 layers][32][hidden / 16] their rows' sums of h^2
  float* qkv;        // [layers][32][qkv width] row-major
  Bf16* attention;   // [layers][32 q width] bf16 fragment order
  Bf16* swiglu;      // [layers][32 ffn] bf16 fragment order
  unsigned* sync;    // SyncWords() words, zero at creation
};

/// Words of the synchronisation area: the barrier slot counters, the
/// launch generation and the error word.
std::size_t SyncWords(const fused::Shape& s, int layers);
/// Offset (in words) of the error word in the synchronisation area; it
/// turns non-zero when a barrier wait times out, and every later launch
/// returns at once until the host clears the area.
std::size_t ErrorWord();

/// Elements of each workspace buffer for `layers` layers.
std::size_t HElements(const fused::Shape& s, int layers);
std::size_t NormElements(const fused::Shape& s, int layers);
std::size_t SquaresElements(const fused::Shape& s, int layers);
std::size_t QkvElements(const fused::Shape& s, int layers);
std::size_t AttentionElements(const fused::Shape& s, int layers);
std::size_t SwigluElements(const fused::Shape& s, int layers);

/// Whether the persistent kernel takes this shape on a grid of `grid`
/// workgroups (every phase's workgroups fit the grid, one pass of pairs
/// per wave, at most 32 rows).
bool Supported(const fused::Shape& s, int layers, int grid);

/// Workgroups of the launch on the current device: one per compute unit,
/// at most 256.
int GridSize();

/// Sets up the kernel for this shape (its LDS size limit) outside any
/// stream capture; false when there is no kernel for it or when its grid
/// cannot be resident on the device all at once.
bool Prepare(const fused::Shape& s);

/// 64-bit words of a launch's timestamp trace: [grid][barriers + 1][4]
/// (slot 0: kernel start and end; slot b: arrival at and exit from grid
/// barrier b, and in the phase before it the times its products and its
/// stores were done), s_memrealtime ticks of 10 ns.
std::size_t TraceWords(int layers, int grid);

/// Grid barriers of one launch: one after the input assembly and five per
/// layer.
int Barriers(int layers);

/// One evaluation: x [patch][feat] -> velocity [2][patch][feat]; with
/// x_update non-null also x_update -= dt (u s + cfg (c - u s)). `trace`
/// (TraceWords() words, or null) records the launch's timestamps.
int Evaluate(const fused::Shape& s, int layers, int grid, const Weights& w,
             const Workspace& ws, const float* mu, const float* time,
             const float* cond_rows, const float* x, float* velocity,
             float* x_update, float cfg, float dt, int zero_star,
             unsigned long long* trace, hipStream_t stream);

}  // namespace vx::persistent

#endif  // VOXCPM_AMD_DIT_PERSISTENT_HPP_
