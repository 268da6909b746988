// Launchers of the DiT's fused layer kernels (dit_fused.hip): the CFG pair's
// rows (up to 32) kept in fragment order between kernels, five launches per
// layer (qkv with the input norm, attention with the rotary embedding, o
// with the residual add, gate_up with the post-attention norm and SwiGLU,
// down with the residual add) and one each for the input assembly and the
// output projection with the Euler update.
#ifndef VOXCPM_AMD_DIT_FUSED_HPP_
#define VOXCPM_AMD_DIT_FUSED_HPP_

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "common.hpp"
#include "q8.hpp"

namespace vx::fused {

struct Shape {
  int rows;      // 2 length
  int length;    // 3 + 2 patch
  int patch;
  int hidden;
  int heads;
  int kv_heads;
  int head_dim;
  int ffn;
  int feat;
  float eps;
  q8::Weights weights = q8::Weights::kQ8;  // Q8_0 or bf16 panels, every matrix
};

/// Whether the fused kernels take this shape: at most 32 rows (patch <= 6),
/// widths multiples of 64, hidden <= 2048 (the norm prologue's one pass),
/// feat <= 64, head_dim even and <= 256.
bool Supported(const Shape& s);

/// Whether the layer kernels (Qkv, Residual, GateUp) take a stack of this
/// shape, the DiT's input and output kernels aside: up to 32 rows, widths
/// multiples of 64, hidden <= 2048.
bool StackSupported(const Shape& s);

/// A norm operand in the form the producing epilogue leaves it: x =
/// bf16(h * gamma) in bf16 fragment order [32][hidden] and squares[row][g]
/// = the sum of h^2 over columns 16 g .. 16 g + 15 (float32 [32][hidden /
/// 16]); the consumer scales its outputs by rsqrt(sum / hidden + eps). With
/// x null the producer writes no operand.
struct NormOperand {
  Bf16* x = nullptr;
  const Bf16* gamma = nullptr;
  float* squares = nullptr;
};

/// Residual stream rows (float32 fragment order [32][hidden]) from in_proj
/// of x [patch][feat] (bf16 conversion, product, bias) and the assembly of
/// mu, the time vector and the condition rows (generator.cpp:297-316;
/// kernels/generator_kernels.hip:320-340).
void InAssemble(const float* x, const void* in_weight, const Bf16* in_bias,
                const float* mu, const float* time, const float* cond_rows,
                float* h, const Shape& s, hipStream_t stream,
                const NormOperand& next = NormOperand{});

/// qkv [rows][(heads + 2 kv_heads) head_dim] = rmsnorm(h) Wqkv^T.
void Qkv(const float* h, const Bf16* norm, const void* weight, float* qkv,
         const Shape& s, hipStream_t stream);

/// qkv = (bf16(h gamma) Wqkv^T) rsqrt(mean(h^2) + eps) from the norm
/// operand the producer of h left.
void QkvScaled(const NormOperand& x, const void* weight, float* qkv, const Shape& s,
               hipStream_t stream);

/// Rotary embedding and bidirectional attention within each branch from
/// the qkv rows; output bf16 fragment order [32][heads head_dim].
void Attention(const float* qkv, const float* rope, Bf16* out, const Shape& s,
               hipStream_t stream);

/// h += a W^T (a bf16 fragment order [32][k]; h float32 fragment order);
/// with next.x non-null also the next norm's operand of the new h.
void Residual(const Bf16* a, const void* weight, int k, int n, float* h,
              const Shape& s, hipStream_t stream, const NormOperand& next = NormOperand{});

/// s = swiglu(rmsnorm(h) Wgate_up^T), bf16 fragment order [32][ffn].
void GateUp(const float* h, const Bf16* norm, const void* weight, Bf16* out,
            const Shape& s, hipStream_t stream);

/// GateUp from the norm operand the producer of h left (outputs of both
/// halves scaled by the row's rsqrt(mean(h^2) + eps) before the SwiGLU).
void GateUpScaled(const NormOperand& x, const void* weight, Bf16* out, const Shape& s,
                  hipStream_t stream);

/// velocity [2][patch][feat] = out_proj(bf16(rmsnorm(h) of the output rows))
/// + bias; with `x` non-null also x -= dt (u s + cfg (c - u s))
/// (kernels/generator_kernels.hip:342-360).
void OutEuler(const float* h, const Bf16* norm, const void* out_weight,
              const Bf16* out_bias, float* velocity, float* x, float cfg,
              float dt, int zero_star, const Shape& s, hipStream_t stream);

}  // namespace vx::fused

#endif  // VOXCPM_AMD_DIT_FUSED_HPP_
