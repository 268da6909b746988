// Load-time conversions of Q8_0 weights: GGML blocks <-> panels, and panels
// -> bfloat16 rows (the reference's expansion for products of more than
// 128 rows).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.hpp"
#include "q8.hpp"

namespace vx {
namespace {

using q8::kBlockBytes;
using q8::kUnitBytes;
using q8::kValueBytes;

// One thread per (unit, lane): gathers the lane's 16 value bytes from two
// GGML blocks, and lanes of octet 0 also the row's pair of scales.
__global__ void PackKernel(const std::uint8_t* blocks, int n, int k,
                           std::uint8_t* packed, int pairs,
                           std::size_t threads) {
  const std::size_t index =
      static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (index >= threads)
    return;
  const int lane = static_cast<int>(index % 64);
  const std::size_t unit = index / 64;
  const int pair = static_cast<int>(unit % pairs);
  const int group = static_cast<int>(unit / pairs);
  const int row = group * 16 + lane % 16;
  const int octet = lane / 16;
  const int blocks_per_row = k / 32;
  std::uint8_t values[16];
  std::uint16_t scales[2] = {0, 0};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int block = 2 * pair + h;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      values[8 * h + i] = 0;
    if (row < n && block < blocks_per_row) {
      const std::uint8_t* source =
          blocks + (static_cast<std::size_t>(row) * blocks_per_row + block) *
                       kBlockBytes;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        values[8 * h + i] = source[2 + 8 * octet + i];
      scales[h] = static_cast<std::uint16_t>(source[0] | (source[1] << 8));
    }
  }
  std::uint8_t* target = packed + unit * kUnitBytes;
  uint4 word;
  __builtin_memcpy(&word, values, 16);
  *reinterpret_cast<uint4*>(target + 16 * lane) = word;
  if (octet == 0)
    *reinterpret_cast<std::uint32_t*>(target + kValueBytes + 4 * (lane % 16)) =
        scales[0] | (static_cast<std::uint32_t>(scales[1]) << 16);
}

// One thread per GGML block.
__global__ void UnpackBlocksKernel(const std::uint8_t* packed, int n, int k,
                                   std::uint8_t* blocks, int pairs) {
  const std::size_t index =
      static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int blocks_per_row = k / 32;
  if (index >= static_cast<std::size_t>(n) * blocks_per_row)
    return;
  const int row = static_cast<int>(index / blocks_per_row);
  const int block = static_cast<int>(index % blocks_per_row);
  const int pair = block / 2;
  const int h = block % 2;
  const std::uint8_t* unit =
      packed + (static_cast<std::size_t>(row / 16) * pairs + pair) * kUnitBytes;
  const int r = row % 16;
  std::uint8_t* target = blocks + index * kBlockBytes;
  const std::uint32_t scales =
      *reinterpret_cast<const std::uint32_t*>(unit + kValueBytes + 4 * r);
  const std::uint16_t scale =
      static_cast<std::uint16_t>(h == 0 ? scales & 0xFFFFU : scales >> 16);
  target[0] = static_cast<std::uint8_t>(scale & 0xFFU);
  target[1] = static_cast<std::uint8_t>(scale >> 8);
  for (int octet = 0; octet < 4; ++octet) {
    const std::uint8_t* source = unit + 16 * (octet * 16 + r) + 8 * h;
    for (int i = 0; i < 8; ++i)
      target[2 + 8 * octet + i] = source[i];
  }
}

// One thread per 8 output values (a row's octet of one block):
// bf16_rne(f32(scale) * q).
__global__ void UnpackBf16Kernel(const std::uint8_t* packed, int n, int k,
                                 Bf16* out, int pairs) {
  const std::size_t index =
      static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int octets = k / 8;
  if (index >= static_cast<std::size_t>(n) * octets)
    return;
  const int row = static_cast<int>(index / octets);
  const int column = static_cast<int>(index % octets) * 8;
  const int pair = column / 64;
  const int h = (column % 64) / 32;
  const int octet = (column % 32) / 8;
  const std::uint8_t* unit =
      packed + (static_cast<std::size_t>(row / 16) * pairs + pair) * kUnitBytes;
  const int r = row % 16;
  const std::uint32_t scales =
      *reinterpret_cast<const std::uint32_t*>(unit + kValueBytes + 4 * r);
  const float scale = HalfValue(
      static_cast<std::uint16_t>(h == 0 ? scales & 0xFFFFU : scales >> 16));
  const uint2 bytes =
      *reinterpret_cast<const uint2*>(unit + 16 * (octet * 16 + r) + 8 * h);
  Bf16 values[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const std::uint32_t word = i < 4 ? bytes.x : bytes.y;
    const float q = static_cast<float>(
        static_cast<std::int8_t>(word >> (8 * (i % 4))));
    values[i] = Bf16Bits(scale * q);
  }
  uint4 word;
  __builtin_memcpy(&word, values, 16);
  *reinterpret_cast<uint4*>(out + static_cast<std::size_t>(row) * k + column) =
      word;
}

// bf16 panels (q8.hpp): one thread per (unit, half, lane) gathers 16 bytes
// of one weight row.
__global__ void PackBf16PanelsKernel(const Bf16* rows, int n, int k, std::uint8_t* packed,
                                     int pairs, std::size_t threads) {
  const std::size_t index =
      static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (index >= threads)
    return;
  const int lane = static_cast<int>(index % 64);
  const int half = static_cast<int>((index / 64) % 2);
  const std::size_t unit = index / 128;
  const int pair = static_cast<int>(unit % pairs);
  const int group = static_cast<int>(unit / pairs);
  const int row = group * 16 + lane % 16;
  const int column = 64 * pair + 32 * half + 8 * (lane / 16);
  uint4 word{0U, 0U, 0U, 0U};
  if (row < n && column < k)
    word = *reinterpret_cast<const uint4*>(rows + static_cast<std::size_t>(row) * k + column);
  *reinterpret_cast<uint4*>(packed + unit * q8::kBf16UnitBytes + half * q8::kBf16HalfBytes +
                            16 * lane) = word;
}

// One thread per 8 values of a row.
__global__ void UnpackBf16PanelsKernel(const std::uint8_t* packed, int n, int k, Bf16* rows,
                                       int pairs) {
  const std::size_t index =
      static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int octets = k / 8;
  if (index >= static_cast<std::size_t>(n) * octets)
    return;
  const int row = static_cast<int>(index / octets);
  const int column = static_cast<int>(index % octets) * 8;
  const int pair = column / 64;
  const int half = (column % 64) / 32;
  const int lane = 16 * ((column % 32) / 8) + row % 16;
  const std::uint8_t* source =
      packed + (static_cast<std::size_t>(row / 16) * pairs + pair) * q8::kBf16UnitBytes +
      half * q8::kBf16HalfBytes + 16 * lane;
  *reinterpret_cast<uint4*>(rows + static_cast<std::size_t>(row) * k + column) =
      *reinterpret_cast<const uint4*>(source);
}

int CheckShape(std::size_t n, std::size_t k, const char* what) {
  if (n == 0 || k == 0 || k % 32 != 0)
    return Fail(VX_BAD_ARG, std::string(what) +
                                ": n must be positive and k a positive "
                                "multiple of 32");
  if (n > (1U << 30) || k > (1U << 30))
    return Fail(VX_BAD_ARG, std::string(what) + ": shape too large");
  return VX_OK;
}

dim3 Grid(std::size_t threads, int block) {
  return dim3(static_cast<unsigned>((threads + block - 1) / block));
}

}  // namespace
}  // namespace vx

extern "C" {

size_t vx_q8_packed_bytes(size_t n, size_t k) {
  return vx::q8::PackedBytes(n, k);
}

int vx_q8_pack(const uint8_t* blocks, size_t n, size_t k, void* packed,
               void* stream) {
  VX_TRY(vx::CheckShape(n, k, "vx_q8_pack"));
  if (blocks == nullptr || packed == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_q8_pack: null pointer");
  if (reinterpret_cast<std::uintptr_t>(packed) % 16 != 0)
    return vx::Fail(VX_BAD_ARG, "vx_q8_pack: packed must be 16-byte aligned");
  const int pairs = static_cast<int>(vx::q8::Pairs(k));
  const std::size_t threads = vx::q8::Groups(n) * pairs * 64;
  vx::PackKernel<<<vx::Grid(threads, 256), 256, 0, vx::Stream(stream)>>>(
      blocks, static_cast<int>(n), static_cast<int>(k),
      static_cast<std::uint8_t*>(packed), pairs, threads);
  return vx::LaunchStatus("vx_q8_pack");
}

int vx_q8_unpack_blocks(const void* packed, size_t n, size_t k,
                        uint8_t* blocks, void* stream) {
  VX_TRY(vx::CheckShape(n, k, "vx_q8_unpack_blocks"));
  if (blocks == nullptr || packed == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_q8_unpack_blocks: null pointer");
  const int pairs = static_cast<int>(vx::q8::Pairs(k));
  vx::UnpackBlocksKernel<<<vx::Grid(n * (k / 32), 256), 256, 0,
                           vx::Stream(stream)>>>(
      static_cast<const std::uint8_t*>(packed), static_cast<int>(n),
      static_cast<int>(k), blocks, pairs);
  return vx::LaunchStatus("vx_q8_unpack_blocks");
}

int vx_q8_unpack_bf16(const void* packed, size_t n, size_t k, uint16_t* out,
                      void* stream) {
  VX_TRY(vx::CheckShape(n, k, "vx_q8_unpack_bf16"));
  if (out == nullptr || packed == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_q8_unpack_bf16: null pointer");
  if (reinterpret_cast<std::uintptr_t>(out) % 16 != 0 ||
      reinterpret_cast<std::uintptr_t>(packed) % 16 != 0)
    return vx::Fail(VX_BAD_ARG,
                    "vx_q8_unpack_bf16: pointers must be 16-byte aligned");
  const int pairs = static_cast<int>(vx::q8::Pairs(k));
  vx::UnpackBf16Kernel<<<vx::Grid(n * (k / 8), 256), 256, 0,
                         vx::Stream(stream)>>>(
      static_cast<const std::uint8_t*>(packed), static_cast<int>(n),
      static_cast<int>(k), out, pairs);
  return vx::LaunchStatus("vx_q8_unpack_bf16");
}

size_t vx_bf16_packed_bytes(size_t n, size_t k) {
  return vx::q8::Bf16PackedBytes(n, k);
}

int vx_bf16_pack(const uint16_t* rows, size_t n, size_t k, void* packed, void* stream) {
  VX_TRY(vx::CheckShape(n, k, "vx_bf16_pack"));
  if (rows == nullptr || packed == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_bf16_pack: null pointer");
  if (reinterpret_cast<std::uintptr_t>(packed) % 16 != 0 ||
      reinterpret_cast<std::uintptr_t>(rows) % 16 != 0)
    return vx::Fail(VX_BAD_ARG, "vx_bf16_pack: pointers must be 16-byte aligned");
  const int pairs = static_cast<int>(vx::q8::Pairs(k));
  const std::size_t threads = vx::q8::Groups(n) * pairs * 128;
  vx::PackBf16PanelsKernel<<<vx::Grid(threads, 256), 256, 0, vx::Stream(stream)>>>(
      rows, static_cast<int>(n), static_cast<int>(k), static_cast<std::uint8_t*>(packed),
      pairs, threads);
  return vx::LaunchStatus("vx_bf16_pack");
}

int vx_bf16_unpack(const void* packed, size_t n, size_t k, uint16_t* rows, void* stream) {
  VX_TRY(vx::CheckShape(n, k, "vx_bf16_unpack"));
  if (rows == nullptr || packed == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_bf16_unpack: null pointer");
  if (reinterpret_cast<std::uintptr_t>(packed) % 16 != 0 ||
      reinterpret_cast<std::uintptr_t>(rows) % 16 != 0)
    return vx::Fail(VX_BAD_ARG, "vx_bf16_unpack: pointers must be 16-byte aligned");
  const int pairs = static_cast<int>(vx::q8::Pairs(k));
  vx::UnpackBf16PanelsKernel<<<vx::Grid(n * (k / 8), 256), 256, 0, vx::Stream(stream)>>>(
      static_cast<const std::uint8_t*>(packed), static_cast<int>(n), static_cast<int>(k),
      rows, pairs);
  return vx::LaunchStatus("vx_bf16_unpack");
}

}  // extern "C"
