// The Q8_0 panel layout and the device pieces shared by every kernel that
// reads it (products, the DiT).
//
// A panel unit covers 16 weight rows (a row group) and 64 columns (two
// GGML Q8_0 blocks, a pair) in 1088 bytes:
//
//   bytes [0, 1024): lane L of a wave (0..63) owns bytes [16 L, 16 L + 16):
//     row r = L % 16 of the group, column octet j = L / 16:
//     q[r][64 p + 8 j + 0..7]       (first block of the pair), then
//     q[r][64 p + 32 + 8 j + 0..7]  (second block),
//     int8 two's complement, exactly as in the GGML block;
//   bytes [1024, 1088): 16 dwords, dword r = the float16 scales of row r:
//     scale[r][block 2 p] | scale[r][block 2 p + 1] << 16.
//
// Units run along the columns (pairs), then down the row groups. Rows past
// n and columns past k are zero (values and scales), so they add nothing.
//
// One 16-byte load per lane reads the bf16 MFMA B operands of both blocks
// of a pair for 16 weight rows (v_mfma_f32_16x16x32_bf16 takes 8 values
// per lane: column L % 16, reduction index 8 (L / 16) + i); a wave's load
// is 1024 contiguous bytes.
#ifndef VOXCPM_AMD_Q8_HPP_
#define VOXCPM_AMD_Q8_HPP_

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "common.hpp"

namespace vx::q8 {

constexpr int kGroupRows = 16;
constexpr int kPairColumns = 64;
constexpr int kValueBytes = 1024;
constexpr int kUnitBytes = 1088;
constexpr int kBlockBytes = 34;  // GGML Q8_0

inline std::size_t Groups(std::size_t n) { return (n + 15) / 16; }
inline std::size_t Pairs(std::size_t k) { return (k + 63) / 64; }
inline std::size_t PackedBytes(std::size_t n, std::size_t k) {
  return Groups(n) * Pairs(k) * kUnitBytes;
}

// bfloat16 weights take the same units at 2048 bytes: two halves of 1024
// bytes, one per 32-column block of the pair; in half h lane L owns bytes
// [16 L, 16 L + 16) = w[r][64 p + 32 h + 8 j + 0..7] (bf16 bits) for
// r = L % 16, j = L / 16. Rows past n and columns past k are zero. One
// 16-byte load per lane and half is the MFMA B operand of one block.
constexpr int kBf16UnitBytes = 2048;
constexpr int kBf16HalfBytes = 1024;
inline std::size_t Bf16PackedBytes(std::size_t n, std::size_t k) {
  return Groups(n) * Pairs(k) * kBf16UnitBytes;
}

/// Weight formats the product kernels read: Q8_0 panels (the exact per-block
/// arithmetic), bf16 panels, bf16 rows [n][k] as they come (row-major, k a
/// multiple of 8), or Q8_0 panels expanded on the fly to bf16(scale * q)
/// with one float32 sum over k (the reference's arithmetic beyond 128
/// rows, gemm.cpp:305-312).
enum class Weights : int { kQ8 = 0, kBf16 = 1, kBf16Rows = 2, kQ8Expanded = 3 };

/// Whether the weights are Q8_0 panels (either arithmetic).
__host__ __device__ constexpr bool IsQ8(Weights w) {
  return w == Weights::kQ8 || w == Weights::kQ8Expanded;
}

typedef __bf16 Bf16x8 __attribute__((ext_vector_type(8)));
typedef float F32x4 __attribute__((ext_vector_type(4)));

/// bf16 encodings of the sign-extended bytes `lo` and `hi` packed low/high:
/// an int8 has at most 8 significant bits, so its float32 value has a zero
/// low half and the high half is its exact bf16 encoding.
__device__ inline std::uint32_t Int8PairBf16(std::int32_t lo, std::int32_t hi) {
  return __builtin_amdgcn_perm(__float_as_uint(static_cast<float>(hi)),
                               __float_as_uint(static_cast<float>(lo)),
                               0x07060302U);
}

/// Eight int8 values (two little-endian dwords) -> eight exact bf16.
__device__ inline Bf16x8 Int8x8ToBf16(std::uint32_t w0, std::uint32_t w1) {
  const auto s = [](std::uint32_t word, int byte) {
    return static_cast<std::int32_t>(static_cast<std::int8_t>(word >> (8 * byte)));
  };
  union {
    std::uint32_t u[4];
    Bf16x8 v;
  } out;
  out.u[0] = Int8PairBf16(s(w0, 0), s(w0, 1));
  out.u[1] = Int8PairBf16(s(w0, 2), s(w0, 3));
  out.u[2] = Int8PairBf16(s(w1, 0), s(w1, 1));
  out.u[3] = Int8PairBf16(s(w1, 2), s(w1, 3));
  return out.v;
}

__device__ inline Bf16x8 AsBf16x8(const uint4& bits) {
  return __builtin_bit_cast(Bf16x8, bits);
}

/// C (16 x 16, float32) += A (16 x 32, bf16) B (32 x 16, bf16): lane L holds
/// A row L % 16 and B column L % 16, each at reduction indices
/// 8 (L / 16) .. + 7; C element i of lane L is row 4 (L / 16) + i, column
/// L % 16.
__device__ inline F32x4 Mfma16x16x32(const Bf16x8& a, const Bf16x8& b,
                                     const F32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

}  // namespace vx::q8

#endif  // VOXCPM_AMD_Q8_HPP_
