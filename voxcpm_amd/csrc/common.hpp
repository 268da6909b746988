// Shared helpers of the voxcpm_amd library: error reporting across the C
// ABI, bfloat16/float16 conversions and the wave64 reductions.
#ifndef VOXCPM_AMD_COMMON_HPP_
#define VOXCPM_AMD_COMMON_HPP_

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "voxcpm_amd.h"

namespace vx {

using Bf16 = std::uint16_t;

// ---- error reporting --------------------------------------------------

/// Records `message` as the calling thread's last error and returns `status`.
int Fail(int status, const std::string& message);
/// Records a HIP failure of `what`.
int FailHip(hipError_t error, const char* what);
/// Clears the calling thread's last error; returns VX_OK.
int Succeed();

/// Returns from the enclosing function when `status` is a failure.
#define VX_TRY(expression)                 \
  do {                                     \
    const int vx_status_ = (expression);   \
    if (vx_status_ != VX_OK)               \
      return vx_status_;                   \
  } while (0)

/// Returns VX_HIP_ERROR from the enclosing function on a HIP failure.
#define VX_HIP(expression, what)                 \
  do {                                           \
    const hipError_t vx_error_ = (expression);   \
    if (vx_error_ != hipSuccess)                 \
      return ::vx::FailHip(vx_error_, what);     \
  } while (0)

/// The status of the launches just enqueued.
int LaunchStatus(const char* what);

inline hipStream_t Stream(void* stream) {
  return static_cast<hipStream_t>(stream);
}

// ---- conversions ---------------------------------------------------------

/// float32 -> bfloat16 bits, nearest even; NaNs stay quiet NaNs.
__host__ __device__ inline Bf16 Bf16Bits(float value) {
  const std::uint32_t bits = __builtin_bit_cast(std::uint32_t, value);
  if ((bits & 0x7F800000U) == 0x7F800000U && (bits & 0x007FFFFFU) != 0)
    return static_cast<Bf16>((bits >> 16U) | 0x40U);
  return static_cast<Bf16>((bits + 0x7FFFU + ((bits >> 16U) & 1U)) >> 16U);
}

__host__ __device__ inline float Bf16Value(Bf16 bits) {
  return __builtin_bit_cast(float, static_cast<std::uint32_t>(bits) << 16U);
}

/// float16 bits -> float32 (subnormals included; the hardware conversion
/// keeps them).
__device__ inline float HalfValue(std::uint16_t bits) {
  return static_cast<float>(__builtin_bit_cast(_Float16, bits));
}

// ---- wave64 reductions -----------------------------------------------------

constexpr int kWave = 64;

__device__ inline float WaveSum(float value) {
#pragma unroll
  for (int offset = kWave / 2; offset > 0; offset /= 2)
    value += __shfl_xor(value, offset, kWave);
  return value;
}

__device__ inline float WaveMax(float value) {
#pragma unroll
  for (int offset = kWave / 2; offset > 0; offset /= 2)
    value = fmaxf(value, __shfl_xor(value, offset, kWave));
  return value;
}

/// `x` of the lane a DPP control picks within each row of 16 lanes (a VALU
/// move, no LDS round trip).
template<int kCtrl>
__device__ inline float RowDpp(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;         // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;  // lane i of 8 <- lane 7 - i
constexpr int kDppMirror = 0x140;      // lane i of 16 <- lane 15 - i
constexpr int kDppRotate8 = 0x128;     // lane i of 16 <- lane (i + 8) % 16

/// Sum over each row of 16 lanes by pairs at xor 1 and 2, then the
/// mirrored halves of 8 and of 16 lanes; every lane of the row receives the
/// same bits (each step adds the same two values).
__device__ inline float RowSum16(float value) {
  value += RowDpp<kDppXor1>(value);
  value += RowDpp<kDppXor2>(value);
  value += RowDpp<kDppHalfMirror>(value);
  value += RowDpp<kDppMirror>(value);
  return value;
}

__device__ inline float RowMax16(float value) {
  value = fmaxf(value, RowDpp<kDppXor1>(value));
  value = fmaxf(value, RowDpp<kDppXor2>(value));
  value = fmaxf(value, RowDpp<kDppHalfMirror>(value));
  value = fmaxf(value, RowDpp<kDppMirror>(value));
  return value;
}

/// x[l] + x[l ^ 16] by one v_permlane16_swap (rows 0 and 1, 2 and 3 meet);
/// both lanes of a pair receive the same bits.
__device__ inline float AddXor16(float x) {
  const auto swapped = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                        false, false);
  return __uint_as_float(swapped[0]) + __uint_as_float(swapped[1]);
}

/// x[l] + x[l ^ 32] by one v_permlane32_swap (the halves meet).
__device__ inline float AddXor32(float x) {
  const auto swapped = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                        false, false);
  return __uint_as_float(swapped[0]) + __uint_as_float(swapped[1]);
}

/// Lane l receives x[l % 16] (`row0`) and x[16 + l % 16] (`row1`): the first
/// two rows of 16 lanes broadcast over the wave by permlane swaps.
__device__ inline void BroadcastRows01(float x, float& row0, float& row1) {
  // [x0, x0, x2, x2] and [x1, x1, x3, x3] (rows of 16 lanes) ...
  const auto rows = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                     false, false);
  // ... then each one's low half over both halves.
  const auto even = __builtin_amdgcn_permlane32_swap(rows[0], rows[0], false, false);
  const auto odd = __builtin_amdgcn_permlane32_swap(rows[1], rows[1], false, false);
  row0 = __uint_as_float(even[0]);
  row1 = __uint_as_float(odd[0]);
}

/// Sum over a block of up to 1024 threads; `scratch` holds one float per
/// wave. Every thread receives the total, added in wave order.
__device__ inline float BlockSum(float value, float* scratch) {
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int waves = (blockDim.x + kWave - 1) / kWave;
  value = WaveSum(value);
  __syncthreads();
  if (lane == 0)
    scratch[wave] = value;
  __syncthreads();
  float total = scratch[0];
  for (int w = 1; w < waves; ++w)
    total += scratch[w];
  return total;
}

}  // namespace vx

#endif  // VOXCPM_AMD_COMMON_HPP_
