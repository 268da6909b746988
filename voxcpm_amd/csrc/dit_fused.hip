// The DiT's fused layer kernels for up to 32 rows (the CFG pair of one
// patch). Between kernels the residual stream stays float32 and the product
// inputs bf16, both in the MFMA fragment order of q8_tile.hpp, so that every
// wave's operand load is 1 KB of contiguous bytes; the norms run inside the
// products that consume them and SwiGLU inside gate_up's epilogue.
//
// Arithmetic follows kernels/generator_kernels.hip (RMSNorm 91-108, rotary
// 110-158, attention 160-241, SwiGLU 243-254, bias 256-262, assembly
// 320-340, guided Euler 342-360) and transformer.cpp:55-100.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>

#include "common.hpp"
#include "dit_fused.hpp"
#include "dit_phases.hpp"
#include "q8.hpp"
#include "q8_tile.hpp"

namespace vx::fused {
namespace {

// ---- kernels over the phase bodies (dit_phases.hpp) ---------------------------

template<q8::Weights WK>
__global__ __launch_bounds__(kWave) void InAssembleKernel(InArgs a) {
  InAssembleBody<WK>(a, static_cast<int>(blockIdx.x), static_cast<int>(threadIdx.x));
}

__global__ __launch_bounds__(256) void AttentionKernel(AttentionArgs a) {
  extern __shared__ float stage[];
  AttentionBody(a, static_cast<int>(blockIdx.x), static_cast<int>(blockIdx.y), stage,
                static_cast<int>(threadIdx.x), static_cast<int>(blockDim.x));
}

template<q8::Weights WK>
__global__ __launch_bounds__(1024) void OutEulerKernel(OutArgs a) {
  __shared__ float lds[kOutFloats];
  OutEulerBody<WK>(a, lds);
}

// ---- the engine's fused instantiations -------------------------------------

/// One launch of the engine on weights of format WK. The norm products with
/// two pairs per wave (k = hidden of 1025-2048 columns, one pass by
/// Supported) take the one-pass kernel, which holds no registers for a next
/// pass: the two-pass kernel there needs more registers than 16 waves have.
/// The others keep the kernel with a next pass in flight, which measured
/// faster on MI355X even where one pass covers k (patch 2611 -> 2586 us).
template<q8::ASource SRC, q8::Output OUT, int RG, int PW, int MT, q8::Weights WK>
void LaunchEngineAs(const q8::TileArgs& args, int tiles, int waves, hipStream_t stream) {
  const std::size_t shared = q8::EngineShared(MT, RG, waves, SRC);
  constexpr bool kOnePass = SRC == q8::ASource::kScaledBf16 && PW >= 2;
  q8::EngineKernel<MT, RG, SRC, OUT, PW, 2 * MT, WK, 0, kOnePass>
      <<<tiles, waves * kWave, shared, stream>>>(args);
}

template<q8::ASource SRC, q8::Output OUT, int RG, int PW, int MT = 2>
void LaunchEngine(const q8::TileArgs& args, int tiles, int waves, q8::Weights kind,
                  hipStream_t stream) {
  if (kind == q8::Weights::kQ8)
    LaunchEngineAs<SRC, OUT, RG, PW, MT, q8::Weights::kQ8>(args, tiles, waves, stream);
  else
    LaunchEngineAs<SRC, OUT, RG, PW, MT, q8::Weights::kBf16>(args, tiles, waves, stream);
}

}  // namespace

bool Supported(const Shape& s) {
  return s.rows <= q8::kFragRows && s.length <= kMaxLength && s.patch >= 1 &&
         2 * s.patch <= 16 && s.head_dim % 8 == 0 &&
         s.hidden % 64 == 0 && s.hidden <= 2 * 64 * kMaxWaves &&
         (s.heads * s.head_dim) % 64 == 0 && s.ffn % 64 == 0 &&
         s.feat % 16 == 0 && s.feat <= 16 * kOutGroups && s.head_dim % 2 == 0 &&
         s.head_dim <= 256 && s.heads % s.kv_heads == 0;
}

bool StackSupported(const Shape& s) {
  return s.rows <= q8::kFragRows && s.hidden % 64 == 0 && s.hidden <= 2 * 64 * kMaxWaves &&
         (s.heads * s.head_dim) % 64 == 0 && s.ffn % 64 == 0 && s.heads % s.kv_heads == 0;
}

void InAssemble(const float* x, const void* in_weight, const Bf16* in_bias,
                const float* mu, const float* time, const float* cond_rows,
                float* h, const Shape& s, hipStream_t stream, const NormOperand& next) {
  InArgs a{};
  a.x = x;
  a.w = static_cast<const std::uint8_t*>(in_weight);
  a.bias = in_bias;
  a.mu = mu;
  a.time = time;
  a.cond = cond_rows;
  a.h = h;
  a.norm_out = next.x;
  a.norm_gamma = next.gamma;
  a.norm_squares = next.squares;
  a.patch = s.patch;
  a.feat = s.feat;
  a.hidden = s.hidden;
  a.length = s.length;
  if (s.weights == q8::Weights::kQ8)
    InAssembleKernel<q8::Weights::kQ8><<<s.hidden / 16, kWave, 0, stream>>>(a);
  else
    InAssembleKernel<q8::Weights::kBf16><<<s.hidden / 16, kWave, 0, stream>>>(a);
}

void Qkv(const float* h, const Bf16* norm, const void* weight, float* qkv,
         const Shape& s, hipStream_t stream) {
  const int n = (s.heads + 2 * s.kv_heads) * s.head_dim;
  q8::TileArgs args = BaseArgs(weight, s.rows, s.hidden, n);
  args.h = h;
  args.gamma = norm;
  args.eps = s.eps;
  args.y = qkv;
  if (args.pairs <= kMaxWaves)
    LaunchEngine<q8::ASource::kNormF32, q8::Output::kStore, 1, 1>(
        args, args.groups, kMaxWaves, s.weights, stream);
  else
    LaunchEngine<q8::ASource::kNormF32, q8::Output::kStore, 1, 2>(
        args, args.groups, kMaxWaves, s.weights, stream);
}

void QkvScaled(const NormOperand& x, const void* weight, float* qkv, const Shape& s,
               hipStream_t stream) {
  const int n = (s.heads + 2 * s.kv_heads) * s.head_dim;
  q8::TileArgs args = BaseArgs(weight, s.rows, s.hidden, n);
  args.x = x.x;
  args.row_squares = x.squares;
  args.squares_groups = s.hidden / 16;
  args.eps = s.eps;
  args.y = qkv;
  if (args.pairs <= kMaxWaves)
    LaunchEngine<q8::ASource::kScaledBf16, q8::Output::kStore, 1, 1>(
        args, args.groups, kMaxWaves, s.weights, stream);
  else
    LaunchEngine<q8::ASource::kScaledBf16, q8::Output::kStore, 1, 2>(
        args, args.groups, kMaxWaves, s.weights, stream);
}

void Attention(const float* qkv, const float* rope, Bf16* out, const Shape& s,
               hipStream_t stream) {
  AttentionArgs a{};
  a.qkv = qkv;
  a.rope = rope;
  a.out = out;
  a.length = s.length;
  a.heads = s.heads;
  a.kv_heads = s.kv_heads;
  a.head_dim = s.head_dim;
  a.scale = 1.0F / std::sqrt(static_cast<float>(s.head_dim));
  const std::size_t shared = static_cast<std::size_t>(AttentionFloats(s.head_dim)) * sizeof(float);
  AttentionKernel<<<dim3(2, static_cast<unsigned>(s.heads)), 256, shared,
                    stream>>>(a);
}

void Residual(const Bf16* act, const void* weight, int k, int n, float* h,
              const Shape& s, hipStream_t stream, const NormOperand& next) {
  q8::TileArgs args = BaseArgs(weight, s.rows, k, n);
  args.x = act;
  args.residual = h;
  args.norm_out = next.x;
  args.norm_gamma = next.gamma;
  args.norm_squares = next.squares;
  // o and down have few output groups (hidden / 16): row blocks spread
  // them over the compute units, each loading only its rows' activations.
  // With four or more pairs per wave (down) the operand loads bound the
  // workgroup: its blocks then lie within one 16-row tile, which halves
  // them (5.9 -> 4.9 us for k = 4096 on MI355X; o, k = 1024, measured
  // 3.35 us with 32-row blocks against 3.50 us).
  if (args.pairs > 2 * kMaxWaves) {
    // Q8_0: four pairs per wave per pass (k = 4096 in one pass: 2598 ->
    // 2588 us per patch); bf16 panels two (four spill 36 registers).
    SetTileBlocks(args, args.groups, s.rows);
    if (s.weights == q8::Weights::kQ8)
      LaunchEngineAs<q8::ASource::kFragBf16, q8::Output::kResidual, 1, 4, 1, q8::Weights::kQ8>(
          args, args.groups * args.row_blocks, kMaxWaves, stream);
    else
      LaunchEngineAs<q8::ASource::kFragBf16, q8::Output::kResidual, 1, 2, 1, q8::Weights::kBf16>(
          args, args.groups * args.row_blocks, kMaxWaves, stream);
  } else {
    SetRowBlocks(args, args.groups, s.rows);
    LaunchEngine<q8::ASource::kFragBf16, q8::Output::kResidual, 1, 1>(
        args, args.groups * args.row_blocks, kMaxWaves, s.weights, stream);
  }
}

void GateUp(const float* h, const Bf16* norm, const void* weight, Bf16* out,
            const Shape& s, hipStream_t stream) {
  q8::TileArgs args = BaseArgs(weight, s.rows, s.hidden, 2 * s.ffn);
  args.h = h;
  args.gamma = norm;
  args.eps = s.eps;
  args.frag_out = out;
  args.group_stride = s.ffn / 16;
  const int tiles = s.ffn / 16;
  if (args.pairs <= kMaxWaves)
    LaunchEngine<q8::ASource::kNormF32, q8::Output::kSwiGlu, 2, 1>(
        args, tiles, kMaxWaves, s.weights, stream);
  else
    LaunchEngine<q8::ASource::kNormF32, q8::Output::kSwiGlu, 2, 2>(
        args, tiles, kMaxWaves, s.weights, stream);
}

void GateUpScaled(const NormOperand& x, const void* weight, Bf16* out, const Shape& s,
                  hipStream_t stream) {
  q8::TileArgs args = BaseArgs(weight, s.rows, s.hidden, 2 * s.ffn);
  args.x = x.x;
  args.row_squares = x.squares;
  args.squares_groups = s.hidden / 16;
  args.eps = s.eps;
  args.frag_out = out;
  args.group_stride = s.ffn / 16;
  const int tiles = s.ffn / 16;
  if (args.pairs <= kMaxWaves)
    LaunchEngine<q8::ASource::kScaledBf16, q8::Output::kSwiGlu, 2, 1>(
        args, tiles, kMaxWaves, s.weights, stream);
  else
    LaunchEngine<q8::ASource::kScaledBf16, q8::Output::kSwiGlu, 2, 2>(
        args, tiles, kMaxWaves, s.weights, stream);
}

void OutEuler(const float* h, const Bf16* norm, const void* out_weight,
              const Bf16* out_bias, float* velocity, float* x, float cfg,
              float dt, int zero_star, const Shape& s, hipStream_t stream) {
  OutArgs a{};
  a.h = h;
  a.norm = norm;
  a.w = static_cast<const std::uint8_t*>(out_weight);
  a.bias = out_bias;
  a.velocity = velocity;
  a.x = x;
  a.cfg = cfg;
  a.dt = dt;
  a.eps = s.eps;
  a.zero_star = zero_star;
  a.patch = s.patch;
  a.feat = s.feat;
  a.hidden = s.hidden;
  a.length = s.length;
  const int pairs = PairsOf(s.hidden);
  const int waves = std::min(kMaxWaves, pairs);
  if (s.weights == q8::Weights::kQ8)
    OutEulerKernel<q8::Weights::kQ8><<<1, waves * kWave, 0, stream>>>(a);
  else
    OutEulerKernel<q8::Weights::kBf16><<<1, waves * kWave, 0, stream>>>(a);
}

}  // namespace vx::fused
