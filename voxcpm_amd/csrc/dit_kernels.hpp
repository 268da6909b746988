// Launchers of the DiT's non-product kernels (dit_kernels.hip), shared by the
// C ABI wrappers and the DiT orchestration. Same meaning as the reference's
// kernels:: launchers (kernels/generator_kernels.hpp).
#ifndef VOXCPM_AMD_DIT_KERNELS_HPP_
#define VOXCPM_AMD_DIT_KERNELS_HPP_

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "common.hpp"

namespace vx::kernels {

void RmsNorm(const float* input, const Bf16* weight, Bf16* output,
             float* output_f32, std::size_t rows, std::size_t width,
             float epsilon, hipStream_t stream);
void QkvRope(const float* qkv, const float* cos_sin,
             const std::int32_t* positions, const std::int32_t* cache_rows,
             float* q, float* k_cache, float* v_cache, std::size_t rows,
             std::size_t heads, std::size_t kv_heads, std::size_t head_dim,
             std::size_t capacity, hipStream_t stream);
void Attention(const float* q, const float* k_cache, const float* v_cache,
               Bf16* output, std::size_t rows, std::size_t rows_per_sequence,
               std::size_t keys_per_sequence, std::size_t past, bool causal,
               std::size_t heads, std::size_t kv_heads, std::size_t head_dim,
               std::size_t capacity, hipStream_t stream);
void SwiGlu(const float* gate_up, Bf16* output, std::size_t rows,
            std::size_t width, hipStream_t stream);
void AddBias(float* data, const Bf16* bias, std::size_t rows,
             std::size_t width, hipStream_t stream);
void ToBf16(const float* input, Bf16* output, std::size_t count, bool silu,
            hipStream_t stream);
void GatherRows(const float* input, const std::int32_t* indices,
                float* output, std::size_t rows, std::size_t width,
                hipStream_t stream);
void AssembleDit(const float* mu, const float* time, const float* cond,
                 const float* x, float* output, std::size_t patch,
                 std::size_t width, hipStream_t stream);
void GuidedEuler(const float* velocity, float* x, std::size_t count, float cfg,
                 float dt, bool zero_star, hipStream_t stream);
/// dst[i] = src[i] for `count` floats (a kernel, so that HIP graphs
/// capture no copy or memset nodes).
void CopyFloats(const float* src, float* dst, std::size_t count,
                hipStream_t stream);

}  // namespace vx::kernels

#endif  // VOXCPM_AMD_DIT_KERNELS_HPP_
