// The bodies of the DiT's non-product kernels (input assembly, rotary
// attention, output projection with the Euler step), shared by the fused
// per-layer launches (dit_fused.hip) and the persistent evaluation
// (dit_persistent.hip), which runs them as phases of one launch.
//
// Arithmetic follows kernels/generator_kernels.hip (RMSNorm 91-108, rotary
// 110-158, attention 160-241, bias 256-262, assembly 320-340, guided Euler
// 342-360).
#ifndef VOXCPM_AMD_DIT_PHASES_HPP_
#define VOXCPM_AMD_DIT_PHASES_HPP_

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "common.hpp"
#include "q8.hpp"
#include "q8_tile.hpp"

namespace vx::fused {

using q8::AsBf16x8;
using q8::Bf16x8;
using q8::BfFragIndex;
using q8::F32FragIndex;
using q8::F32x4;
using q8::Int8x8ToBf16;
using q8::kUnitBytes;
using q8::kValueBytes;
using q8::Mfma16x16x32;

constexpr int kMaxWaves = 16;

__host__ __device__ inline int PairsOf(int columns) { return (columns + 63) / 64; }

// ---- input assembly -----------------------------------------------------------

struct InArgs {
  const float* x;          // [patch][feat]
  const std::uint8_t* w;   // in_proj panels [hidden][feat]
  const Bf16* bias;        // [hidden] or null
  const float* mu;         // [2][hidden]
  const float* time;       // [hidden]
  const float* cond;       // [patch][hidden]
  float* h;                // fragment order [32][hidden]
  // With norm_out non-null also the first layer's norm operand
  // bf16(h * norm_gamma) (bf16 fragment order) and each row's sum of h^2
  // over the wave's 16 columns, norm_squares[row][column / 16].
  Bf16* norm_out;
  const Bf16* norm_gamma;
  float* norm_squares;
  int patch, feat, hidden, length;
};

// One wave per 16 hidden columns (`group`): in_proj of the patch rows (x
// rounded to bf16, the exact Q8_0 product or the bf16 one, then the bias),
// written to both branches' x rows, and the mu / time / condition rows of
// those columns. kCoherent: device-scope stores (q8::Put).
template<q8::Weights WK, bool kCoherent = false>
__device__ __forceinline__ void InAssembleBody(const InArgs& a, int group, int lane) {
  constexpr int kUnit = WK == q8::Weights::kQ8 ? kUnitBytes : q8::kBf16UnitBytes;
  const int r16 = lane % 16;
  const int octet = lane / 16;
  const int pairs = PairsOf(a.feat);
  const int column = 16 * group + r16;
  const int groups = a.hidden / 16;
  // Every value the wave stores after its product is loaded first, so that
  // all its loads are in flight together instead of one round trip per
  // store: the bias, the norm weight of its column (lane % 16 is the column
  // of every row the lane writes) and its mu / time / condition values,
  // pass p holding element 64 p + lane of the 2 (3 + patch) rows x 16
  // columns (branch-major).
  // Buffer loads: a value a lane does not need (a null bias, a source row
  // it does not take) is read as zero with no access and no branch, so the
  // compiler issues every load before it waits for the first.
  const std::uint32_t hidden_bytes = 4U * static_cast<std::uint32_t>(a.hidden);
  const auto bf16_at = [&](const Bf16* base) {
    const std::uint32_t word = q8::BufferLoad4(
        q8::BufferOf(base, base != nullptr ? hidden_bytes / 2 : 0U),
        4U * static_cast<std::uint32_t>(column / 2), base != nullptr);
    return Bf16Value(static_cast<Bf16>(column % 2 != 0 ? word >> 16 : word & 0xFFFFU));
  };
  const float bias = bf16_at(a.bias);
  const float gamma = bf16_at(a.norm_out != nullptr ? a.norm_gamma : nullptr);
  const int fixed = 3 + a.patch;  // mu, mu, time, condition rows
  constexpr int kFixedPasses = 6;  // 2 (3 + patch) 16 <= 384 for patch <= 8
  const __amdgpu_buffer_rsrc_t mu_buffer = q8::BufferOf(a.mu, 2U * hidden_bytes);
  const __amdgpu_buffer_rsrc_t time_buffer = q8::BufferOf(a.time, hidden_bytes);
  const __amdgpu_buffer_rsrc_t cond_buffer =
      q8::BufferOf(a.cond, static_cast<std::uint32_t>(a.patch) * hidden_bytes);
  float fixed_value[kFixedPasses];
#pragma unroll
  for (int pass = 0; pass < kFixedPasses; ++pass) {
    const int e = kWave * pass + lane;
    const bool live = e < 2 * fixed * 16;
    const int branch = e / (fixed * 16);
    const int row = (e / 16) % fixed;
    const std::uint32_t at = 4U * static_cast<std::uint32_t>(column);
    const std::uint32_t mu = q8::BufferLoad4(
        mu_buffer, at + static_cast<std::uint32_t>(row) * hidden_bytes,
        live && row < 2 && branch == 0);
    const std::uint32_t time = q8::BufferLoad4(time_buffer, at, live && row == 2);
    const std::uint32_t cond = q8::BufferLoad4(
        cond_buffer, at + static_cast<std::uint32_t>(row - 3) * hidden_bytes, live && row > 2);
    fixed_value[pass] = __uint_as_float(row < 2 ? mu : row == 2 ? time : cond);
  }
  const std::uint8_t* unit =
      a.w + static_cast<std::size_t>(group) * pairs * kUnit;
  F32x4 acc{0.0F, 0.0F, 0.0F, 0.0F};
  const F32x4 zero{0.0F, 0.0F, 0.0F, 0.0F};
  for (int pair = 0; pair < pairs; ++pair) {
    const std::uint8_t* u = unit + static_cast<std::size_t>(pair) * kUnit;
    const uint4 wv = *reinterpret_cast<const uint4*>(u + 16 * lane);
    const std::uint32_t scales =
        WK == q8::Weights::kQ8
            ? *reinterpret_cast<const std::uint32_t*>(u + kValueBytes + 4 * r16)
            : 0U;
    uint4 xa[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int x_column = 64 * pair + 32 * hf + 8 * octet;
      float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      if (r16 < a.patch && x_column < a.feat) {
        const float4* source = reinterpret_cast<const float4*>(
            a.x + static_cast<std::size_t>(r16) * a.feat + x_column);
        const float4 lo = source[0];
        const float4 hi = source[1];
        v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
        v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
      }
      xa[hf] = q8::PackBf16x8(v);
    }
    if constexpr (WK != q8::Weights::kQ8) {
      // bf16 panels: each block's products accumulate straight into the sums.
      const uint4 wv2 = *reinterpret_cast<const uint4*>(u + q8::kBf16HalfBytes + 16 * lane);
      acc = Mfma16x16x32(AsBf16x8(xa[0]), AsBf16x8(wv), acc);
      acc = Mfma16x16x32(AsBf16x8(xa[1]), AsBf16x8(wv2), acc);
      continue;
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
  // The norm operand and the row's sum over the wave's 16 columns: the 16
  // lanes of a DPP row hold one row's 16 columns (uniform control flow;
  // dead lanes add zeros and write nothing).
  const auto emit_norm = [&](bool live, int row, float value) {
    if (a.norm_out == nullptr)
      return;
    const float square = RowSum16(live ? value * value : 0.0F);
    if (live) {
      q8::Put<kCoherent>(a.norm_out + BfFragIndex(row, column), q8::Bf16Fast(value * gamma));
      if (column % 16 == 0)
        q8::Put<kCoherent>(a.norm_squares + row * groups + column / 16, square);
    }
  };
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 4 * octet + i;
    const bool live = row < a.patch;
    const float value = acc[i] + bias;
    if (live) {
      q8::Put<kCoherent>(a.h + F32FragIndex(3 + a.patch + row, column), value);
      q8::Put<kCoherent>(a.h + F32FragIndex(a.length + 3 + a.patch + row, column), value);
    }
    emit_norm(live, 3 + a.patch + row, value);
    emit_norm(live, a.length + 3 + a.patch + row, value);
  }
#pragma unroll
  for (int pass = 0; pass < kFixedPasses; ++pass) {
    if (kWave * pass >= 2 * fixed * 16)  // uniform
      break;
    const int e = kWave * pass + lane;
    const bool live = e < 2 * fixed * 16;
    const int branch = e / (fixed * 16);
    const int row = (e / 16) % fixed;
    if (live)
      q8::Put<kCoherent>(a.h + F32FragIndex(branch * a.length + row, column), fixed_value[pass]);
    emit_norm(live, branch * a.length + row, fixed_value[pass]);
  }
}

// ---- attention ----------------------------------------------------------------

struct AttentionArgs {
  const float* qkv;   // [rows][(heads + 2 kv_heads) head_dim]
  const float* rope;  // [length][head_dim] cos | sin, or null
  Bf16* out;          // fragment order [32][heads head_dim]
  int length, heads, kv_heads, head_dim;
  float scale;
};

// One workgroup per (branch, head). Every thread issues its loads at once:
// for query/key row r and dimensions d..d+3 (d < head_dim / 2) the pair
// halves of q and k, the two halves of v and the row's cos / sin. The
// rotated, scaled queries, rotated keys and values go to LDS; then the
// scores of all (query, key) pairs (16 lanes per query row), the softmax
// over the keys (max, exp, sum within the 16 lanes by DPP moves) and the
// weighted values (4 consecutive dimensions per thread). The dot
// products and the weighted sums read LDS 16 bytes at a time, unrolled, so
// that their reads are in flight together instead of one latency per term;
// the terms are still added in index order.
constexpr int kMaxLength = 16;

/// LDS floats of AttentionBody.
__host__ __device__ inline int AttentionFloats(int head_dim) {
  return kMaxLength * (3 * head_dim + 8) + kMaxLength * kMaxLength + kMaxLength;
}

/// (branch, head) on `threads` (>= 256, a multiple of 64) threads, thread
/// `tid`, `stage` AttentionFloats() floats of LDS. kCoherent: device-scope
/// output stores.
template<bool kCoherent = false>
__device__ __forceinline__ void AttentionBody(const AttentionArgs& a, int branch, int head,
                                              float* stage, int tid, int threads) {
  const int dims = a.head_dim;
  const int half = dims / 2;
  const int width = (a.heads + 2 * a.kv_heads) * dims;
  const int kv_head = head / (a.heads / a.kv_heads);
  // Rows padded by 16 bytes: 16-byte reads stay aligned and consecutive
  // keys start 4 banks apart.
  const int stride = dims + 4;
  float* qs = stage;                              // [length][stride]
  float* ks = qs + kMaxLength * stride;           // [length][stride]
  float* vs = ks + kMaxLength * stride;           // [kMaxLength][dims], zero past length
  float* weights = vs + kMaxLength * dims;        // [length][kMaxLength]
  float* inverse = weights + kMaxLength * kMaxLength;  // [length]
  const int quads = half / 4;
  const int items = a.length * quads;
  for (int e = tid; e < items; e += threads) {
    const int r = e / quads;
    const int d = 4 * (e % quads);
    const float* source =
        a.qkv + static_cast<std::size_t>(branch * a.length + r) * width;
    const float4 q0 = *reinterpret_cast<const float4*>(source + head * dims + d);
    const float4 q1 = *reinterpret_cast<const float4*>(source + head * dims + half + d);
    const float4 k0 = *reinterpret_cast<const float4*>(source + (a.heads + kv_head) * dims + d);
    const float4 k1 =
        *reinterpret_cast<const float4*>(source + (a.heads + kv_head) * dims + half + d);
    const float4 v0 =
        *reinterpret_cast<const float4*>(source + (a.heads + a.kv_heads + kv_head) * dims + d);
    const float4 v1 = *reinterpret_cast<const float4*>(
        source + (a.heads + a.kv_heads + kv_head) * dims + half + d);
    float4 c{1.0F, 1.0F, 1.0F, 1.0F};
    float4 sn{0.0F, 0.0F, 0.0F, 0.0F};
    if (a.rope != nullptr) {
      const float* table = a.rope + static_cast<std::size_t>(r) * dims;
      c = *reinterpret_cast<const float4*>(table + d);
      sn = *reinterpret_cast<const float4*>(table + half + d);
    }
    const float qa[4] = {q0.x, q0.y, q0.z, q0.w};
    const float qb[4] = {q1.x, q1.y, q1.z, q1.w};
    const float ka[4] = {k0.x, k0.y, k0.z, k0.w};
    const float kb[4] = {k1.x, k1.y, k1.z, k1.w};
    const float cs[4] = {c.x, c.y, c.z, c.w};
    const float ss[4] = {sn.x, sn.y, sn.z, sn.w};
    const float va[4] = {v0.x, v0.y, v0.z, v0.w};
    const float vb[4] = {v1.x, v1.y, v1.z, v1.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float q_first = qa[j], q_second = qb[j], k_first = ka[j], k_second = kb[j];
      if (a.rope != nullptr) {
        // (a, b) at (i, i + half) -> (a c - b s, b c + a s)
        q_first = qa[j] * cs[j] - qb[j] * ss[j];
        q_second = qb[j] * cs[j] + qa[j] * ss[j];
        k_first = ka[j] * cs[j] - kb[j] * ss[j];
        k_second = kb[j] * cs[j] + ka[j] * ss[j];
      }
      qs[r * stride + d + j] = q_first * a.scale;
      qs[r * stride + half + d + j] = q_second * a.scale;
      ks[r * stride + d + j] = k_first;
      ks[r * stride + half + d + j] = k_second;
      vs[r * dims + d + j] = va[j];
      vs[r * dims + half + d + j] = vb[j];
    }
  }
  for (int e = tid; e < (kMaxLength - a.length) * dims; e += threads)
    vs[a.length * dims + e] = 0.0F;
  __syncthreads();
  {
    // Scores: thread (query i, key j) = (t / 16, t % 16).
    const int i = tid / kMaxLength;
    const int j = tid % kMaxLength;
    const bool valid = i < a.length && j < a.length;
    float score = -INFINITY;
    if (valid) {
      const float4* query = reinterpret_cast<const float4*>(qs + i * stride);
      const float4* key = reinterpret_cast<const float4*>(ks + j * stride);
      float dot = 0.0F;
#pragma unroll 4
      for (int d4 = 0; d4 < dims / 4; ++d4) {
        const float4 q = query[d4];
        const float4 k = key[d4];
        dot += q.x * k.x;
        dot += q.y * k.y;
        dot += q.z * k.z;
        dot += q.w * k.w;
      }
      score = dot;
    }
    static_assert(kMaxLength == 16, "one query's keys are one DPP row");
    const float maximum = RowMax16(score);
    const float weight = valid ? expf(score - maximum) : 0.0F;
    const float sum = RowSum16(weight);
    if (!kCoherent && dims == 4 * kMaxLength) {
      // A query's 16 quarters of the dimensions sit on the same 16 lanes as
      // its 16 keys: each lane takes the row's weights from its neighbours
      // (no LDS round trip, no barrier), then the weighted values as below
      // (bit for bit). The attention launch of the fused path only: 10 x 12
      // launches per patch 2577 -> 2561 us; inside the persistent kernel's
      // 1024-thread phase it measured 17 us slower per patch.
      float w[kMaxLength];
#pragma unroll
      for (int jj = 0; jj < kMaxLength; ++jj)
        w[jj] = __shfl(weight, jj, kMaxLength);
      if (i >= a.length)
        return;
      const int d = 4 * j;
      float out[4] = {0, 0, 0, 0};
#pragma unroll
      for (int jj = 0; jj < kMaxLength; ++jj) {
        const float4 v = *reinterpret_cast<const float4*>(vs + jj * dims + d);
        out[0] += w[jj] * v.x;
        out[1] += w[jj] * v.y;
        out[2] += w[jj] * v.z;
        out[3] += w[jj] * v.w;
      }
      const float inv = 1.0F / sum;
      const int row = branch * a.length + i;
      const std::uint64_t pair =
          static_cast<std::uint64_t>(q8::PackBf16x2(out[0] * inv, out[1] * inv)) |
          static_cast<std::uint64_t>(q8::PackBf16x2(out[2] * inv, out[3] * inv)) << 32;
      q8::Put<kCoherent>(
          reinterpret_cast<std::uint64_t*>(a.out + BfFragIndex(row, head * dims + d)), pair);
      return;
    }
    if (i < kMaxLength) {
      weights[i * kMaxLength + j] = weight;
      if (j == 0)
        inverse[i] = 1.0F / sum;
    }
  }
  __syncthreads();
  // Weighted values: four consecutive dimensions per thread.
  const int quarters = dims / 4;
  for (int e = tid; e < a.length * quarters; e += threads) {
    const int i = e / quarters;
    const int d = 4 * (e % quarters);
    const float4* w4 = reinterpret_cast<const float4*>(weights + i * kMaxLength);
    float w[kMaxLength];
#pragma unroll
    for (int j4 = 0; j4 < kMaxLength / 4; ++j4) {
      const float4 v = w4[j4];
      w[4 * j4] = v.x;
      w[4 * j4 + 1] = v.y;
      w[4 * j4 + 2] = v.z;
      w[4 * j4 + 3] = v.w;
    }
    float out[4] = {0, 0, 0, 0};
    // Keys past the length have weight 0 and zero values: they add +0.
#pragma unroll
    for (int j = 0; j < kMaxLength; ++j) {
      const float4 v = *reinterpret_cast<const float4*>(vs + j * dims + d);
      out[0] += w[j] * v.x;
      out[1] += w[j] * v.y;
      out[2] += w[j] * v.z;
      out[3] += w[j] * v.w;
    }
    const float inv = inverse[i];
    const int row = branch * a.length + i;
    const std::uint64_t pair =
        static_cast<std::uint64_t>(q8::PackBf16x2(out[0] * inv, out[1] * inv)) |
        static_cast<std::uint64_t>(q8::PackBf16x2(out[2] * inv, out[3] * inv)) << 32;
    q8::Put<kCoherent>(reinterpret_cast<std::uint64_t*>(a.out + BfFragIndex(row, head * dims + d)),
                       pair);
  }
}

// ---- output projection and Euler update ------------------------------------

struct OutArgs {
  const float* h;          // fragment order [32][hidden]
  const Bf16* norm;        // [hidden]
  const std::uint8_t* w;   // out_proj panels [feat][hidden]
  const Bf16* bias;        // [feat] or null
  float* velocity;         // [2][patch][feat]
  float* x;                // [patch][feat] or null
  float cfg, dt, eps;
  int zero_star;
  int patch, feat, hidden, length;
};

constexpr int kOutGroups = 4;  // feat <= 64

/// LDS floats of OutEulerBody.
constexpr int kOutFloats = kMaxWaves * 16 + kMaxWaves * kOutGroups * 4 * kWave + 2 * 8 * 64 +
                           kMaxWaves;

// One workgroup: the 2 patch output rows of both branches normalised with
// the final norm (bf16 after the float32 scale, as RmsNorm then ToBf16),
// the out_proj product (Q8_0 or bf16 panels) split over the waves by pairs,
// the bias, and with x given the guided Euler step over the whole velocity.
// `lds`: kOutFloats floats.
template<q8::Weights WK>
__device__ __forceinline__ void OutEulerBody(const OutArgs& a, float* lds) {
  constexpr bool kBf16 = WK != q8::Weights::kQ8;
  constexpr int kUnit = kBf16 ? q8::kBf16UnitBytes : kUnitBytes;
  auto* squares = reinterpret_cast<float(*)[16]>(lds);
  auto* reduce = reinterpret_cast<float(*)[kOutGroups][4][kWave]>(lds + kMaxWaves * 16);
  float* velocity = lds + kMaxWaves * 16 + kMaxWaves * kOutGroups * 4 * kWave;
  float* block = velocity + 2 * 8 * 64;
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int waves = blockDim.x / kWave;
  const int r16 = lane % 16;
  const int octet = lane / 16;
  const int pairs = PairsOf(a.hidden);
  const int groups = (a.feat + 15) / 16;
  const int out_rows = 2 * a.patch;
  // A row r16 (< 2 patch) is branch r16 / patch, output row r16 % patch.
  const bool row_ok = r16 < out_rows;
  const int h_row = row_ok ? (r16 / a.patch) * a.length + 3 + a.patch + r16 % a.patch : 0;
  constexpr int kPw = 2;  // pairs per wave: hidden <= 2048
  uint4 wv[kPw][kOutGroups];
  uint4 wv2[kPw][kOutGroups];  // bf16: the pair's second block
  std::uint32_t sc[kPw][kOutGroups];
  float4 hv[kPw][2][2];
#pragma unroll
  for (int p = 0; p < kPw; ++p) {
    const int pair = wave + p * waves;
    const bool ok = pair < pairs;
#pragma unroll
    for (int g = 0; g < kOutGroups; ++g) {
      const bool use = ok && g < groups;
      const std::uint8_t* u =
          a.w + (static_cast<std::size_t>(use ? g : 0) * pairs + (use ? pair : 0)) * kUnit;
      wv[p][g] = use ? *reinterpret_cast<const uint4*>(u + 16 * lane) : uint4{0U, 0U, 0U, 0U};
      if constexpr (kBf16) {
        wv2[p][g] = use ? *reinterpret_cast<const uint4*>(u + q8::kBf16HalfBytes + 16 * lane)
                        : uint4{0U, 0U, 0U, 0U};
        sc[p][g] = 0U;
      } else {
        sc[p][g] =
            use ? *reinterpret_cast<const std::uint32_t*>(u + kValueBytes + 4 * r16) : 0U;
      }
    }
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        float4 v{0.0F, 0.0F, 0.0F, 0.0F};
        if (ok && row_ok)
          v = *reinterpret_cast<const float4*>(
              a.h + F32FragIndex(h_row, 64 * pair + 32 * hf + 8 * octet + 4 * q));
        hv[p][hf][q] = v;
      }
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
  partial = AddXor32(AddXor16(partial));
  if (octet == 0)
    squares[wave][r16] = partial;
  __syncthreads();
  float total = 0.0F;
  for (int w = 0; w < waves; ++w)
    total += squares[w][r16];
  const float inverse = rsqrtf(total / static_cast<float>(a.hidden) + a.eps);
  F32x4 acc[kOutGroups];
#pragma unroll
  for (int g = 0; g < kOutGroups; ++g)
    acc[g] = F32x4{0.0F, 0.0F, 0.0F, 0.0F};
  const F32x4 zero{0.0F, 0.0F, 0.0F, 0.0F};
#pragma unroll
  for (int p = 0; p < kPw; ++p) {
    const int pair = wave + p * waves;
    if (pair >= pairs)
      continue;
    uint4 xa[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const uint4 gw = *reinterpret_cast<const uint4*>(a.norm + 64 * pair + 32 * hf + 8 * octet);
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
      if constexpr (kBf16) {
        acc[g] = Mfma16x16x32(AsBf16x8(xa[0]), AsBf16x8(wv[p][g]), acc[g]);
        acc[g] = Mfma16x16x32(AsBf16x8(xa[1]), AsBf16x8(wv2[p][g]), acc[g]);
        continue;
      }
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
      reduce[wave][g][i][lane] = acc[g][i];
  __syncthreads();
  const int values = a.patch * a.feat;  // per branch
  for (int e = threadIdx.x; e < kOutGroups * 256; e += blockDim.x) {
    const int g = e / 256;
    const int i = (e / 64) % 4;
    const int l = e % 64;
    const int row = 4 * (l / 16) + i;
    const int column = 16 * g + l % 16;
    if (row >= out_rows || column >= a.feat)
      continue;
    float v = reduce[0][g][i][l];
    for (int w = 1; w < waves; ++w)
      v += reduce[w][g][i][l];
    if (a.bias != nullptr)
      v += Bf16Value(a.bias[column]);
    const int at = row * a.feat + column;  // [branch][patch][feat]
    a.velocity[at] = v;
    velocity[at] = v;
  }
  if (a.x == nullptr)
    return;
  __syncthreads();
  const float* c = velocity;
  const float* u = velocity + values;
  float s = 1.0F;
  if (a.zero_star) {
    float dot = 0.0F;
    float norm = 0.0F;
    for (int i = threadIdx.x; i < values; i += blockDim.x) {
      dot += c[i] * u[i];
      norm += u[i] * u[i];
    }
    dot = BlockSum(dot, block);
    norm = BlockSum(norm, block);
    s = dot / (norm + 1e-8F);
  }
  for (int i = threadIdx.x; i < values; i += blockDim.x) {
    const float guided = u[i] * s + a.cfg * (c[i] - u[i] * s);
    a.x[i] -= a.dt * guided;
  }
}

// ---- the products' work split (shared by both paths) -------------------------

/// Product arguments of m rows of k columns times n weight rows (panels).
__host__ __device__ inline q8::TileArgs BaseArgs(const void* weight, int m, int k, int n) {
  q8::TileArgs args{};
  args.w = static_cast<const std::uint8_t*>(weight);
  args.m = m;
  args.k = k;
  args.n = n;
  args.pairs = PairsOf(k);
  args.groups = (n + 15) / 16;
  args.group_stride = 1;
  args.row_blocks = 1;
  args.rows_per_block = m;
  return args;
}

/// Row blocks of a launch of `tiles` tiles over `rows` rows: up to 4 while
/// the grid stays within one workgroup per compute unit (256) and blocks
/// keep at least 5 rows; tiles a multiple of 8 keep a tile's blocks on one
/// compute die.
__host__ __device__ inline void SetRowBlocks(q8::TileArgs& args, int tiles, int rows) {
  int blocks = 1;
  while (tiles % 8 == 0 && blocks < 4 && tiles * 2 * blocks <= 256 &&
         (rows + 2 * blocks - 1) / (2 * blocks) >= 5)
    blocks *= 2;
  args.row_blocks = blocks;
  args.rows_per_block = (rows + blocks - 1) / blocks;
}

/// Tile-aligned row blocks (one 16-row tile of the fragment order per
/// workgroup): up to 4 blocks per tile while the grid stays within one
/// workgroup per compute unit; tiles a multiple of 8 keep a tile's blocks
/// on one compute die, whose L2 serves their weights.
__host__ __device__ inline void SetTileBlocks(q8::TileArgs& args, int tiles, int rows) {
  const int row_tiles = (rows + 15) / 16;
  int blocks = 1;
  while (tiles % 8 == 0 && blocks < 4 && tiles * row_tiles * 2 * blocks <= 256)
    blocks *= 2;
  args.tile_blocks = blocks;
  args.row_blocks = row_tiles * blocks;
}

}  // namespace vx::fused

#endif  // VOXCPM_AMD_DIT_PHASES_HPP_
