// One MiniCPM4 stack with a key/value cache on one stream: VoxCPM2's base
// and residual LMs (one row per decode step) and the local encoder (five
// rows per patch), ForwardStack of transformer.cpp:55-100.
//
// Up to 32 rows take the fused layer kernels of the DiT (dit_fused.hip: the
// residual stream in fragment order, the norms folded into the qkv and
// gate_up products, SwiGLU into gate_up's epilogue, the residual adds into
// o's and down's) around the rotary/cache kernel and a split-key attention:
// the keys of each (row, KV head) are cut into chunks of 64 that separate
// workgroups score, so that a one-row decode step over a long cache still
// spreads over the compute units; a second launch merges the chunks'
// softmax statistics in chunk order. More rows take the reference's launch
// sequence.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <vector>

#include "common.hpp"
#include "dit_fused.hpp"
#include "dit_kernels.hpp"
#include "products.hpp"
#include "q8.hpp"
#include "q8_tile.hpp"
#include "voxcpm_amd.h"
#include "voxcpm_amd_internal.h"

namespace vx::stack {
namespace {

constexpr int kChunk = 64;     // keys per workgroup of the split attention
constexpr int kThreads = 256;  // four waves, 16 keys each when scoring
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxGroup = 16;  // query heads per KV head

struct AttentionArgs {
  const float* q;        // [rows][heads][D], rotated, unscaled
  const float* k;        // [kv_heads][capacity][D]
  const float* v;
  Bf16* out;             // [rows][heads D] row-major, or fragment order
  float* partials;       // [rows][heads][splits][D + 2] when splits > 1
  int rows_per_sequence;
  int keys_per_sequence;
  int past;
  int causal;
  int heads;
  int kv_heads;
  int capacity;
  int splits;
  float scale;
  int fragment;  // bf16 fragment order (rows <= 32) instead of row-major
};

__device__ inline std::size_t OutIndex(const AttentionArgs& a, int row, int column, int width) {
  return a.fragment != 0 ? q8::BfFragIndex(row, column)
                         : static_cast<std::size_t>(row) * width + column;
}

/// LDS floats of a workgroup: the group's scaled queries, the chunk's
/// scores, the per-head statistics and the waves' value sums.
constexpr std::size_t SharedFloats(int group, int d) {
  return static_cast<std::size_t>(group) * d + static_cast<std::size_t>(group) * kChunk +
         2 * group + static_cast<std::size_t>(kWaves) * group * d;
}

/// One chunk of keys of one (row, KV head) for the KV head's `group` query
/// heads (kernels/generator_kernels.hip:160-241 in the chunk): scores
/// q . k scale with lanes over (key, quarter of the dimensions) and the
/// quarters met by permlane swaps; the chunk's maximum and sum per head;
/// the values weighted by exp(score - max) with lanes over dimensions and
/// the four waves' sums added in wave order. One chunk writes the output
/// itself; several leave (max, sum, values) for MergeKernel.
template<int D>
__global__ __launch_bounds__(kThreads) void SplitAttentionKernel(AttentionArgs a) {
  constexpr int kQuarter = D / 4;
  constexpr int kPerLane = D / kWave;
  extern __shared__ float lds[];
  const int group = a.heads / a.kv_heads;
  float* qs = lds;                                  // [group][D]
  float* ps = qs + group * D;                       // [group][kChunk]
  float* stats = ps + group * kChunk;               // [group][2]
  float* parts = stats + 2 * group;                 // [waves][group][D]
  const int split = static_cast<int>(blockIdx.x);
  const int row = static_cast<int>(blockIdx.y);
  const int g = static_cast<int>(blockIdx.z);
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int sequence = row / a.rows_per_sequence;
  const int local = row % a.rows_per_sequence;
  const int count = a.past + (a.causal != 0 ? local + 1 : a.rows_per_sequence);
  const int first = sequence * a.keys_per_sequence;
  const int key0 = split * kChunk;
  const int key1 = min(count, key0 + kChunk);
  const std::size_t stride = static_cast<std::size_t>(D) + 2;
  const std::size_t partial0 =
      (static_cast<std::size_t>(row) * a.heads + g * group) * a.splits + split;

  if (key0 >= key1) {  // past this row's keys: an empty chunk
    for (int e = static_cast<int>(threadIdx.x); e < group * static_cast<int>(stride);
         e += kThreads) {
      const int hh = e / static_cast<int>(stride);
      const int i = e % static_cast<int>(stride);
      a.partials[(partial0 + static_cast<std::size_t>(hh) * a.splits) * stride + i] =
          i == 0 ? -INFINITY : 0.0F;
    }
    return;
  }

  for (int e = static_cast<int>(threadIdx.x); e < group * D; e += kThreads) {
    const int hh = e / D;
    qs[e] = a.q[(static_cast<std::size_t>(row) * a.heads + g * group + hh) * D + e % D] *
            a.scale;
  }
  __syncthreads();

  // Scores: lane (key 16 wave + lane % 16, quarter lane / 16).
  {
    const int key_local = 16 * wave + lane % 16;
    const int quarter = lane / 16;
    const int key = key0 + key_local;
    const bool valid = key < key1;
    const float4* krow = reinterpret_cast<const float4*>(
        a.k + (static_cast<std::size_t>(g) * a.capacity + first + (valid ? key : key0)) * D +
        quarter * kQuarter);
    float kv[kQuarter];
#pragma unroll
    for (int i = 0; i < kQuarter / 4; ++i) {
      const float4 f = krow[i];
      kv[4 * i] = f.x;
      kv[4 * i + 1] = f.y;
      kv[4 * i + 2] = f.z;
      kv[4 * i + 3] = f.w;
    }
    for (int hh = 0; hh < group; ++hh) {
      const float4* qrow = reinterpret_cast<const float4*>(qs + hh * D + quarter * kQuarter);
      float s = 0.0F;
#pragma unroll
      for (int i = 0; i < kQuarter / 4; ++i) {
        const float4 qv = qrow[i];
        s += qv.x * kv[4 * i] + qv.y * kv[4 * i + 1] + qv.z * kv[4 * i + 2] +
             qv.w * kv[4 * i + 3];
      }
      s = AddXor32(AddXor16(s));
      if (quarter == 0)
        ps[hh * kChunk + key_local] = valid ? s : -INFINITY;
    }
  }
  __syncthreads();

  // The chunk's softmax statistics per head (wave w: heads w, w + 4, ...).
  for (int hh = wave; hh < group; hh += kWaves) {
    const float s = ps[hh * kChunk + lane];
    const float m = WaveMax(s);
    const float p = s == -INFINITY ? 0.0F : expf(s - m);
    const float l = WaveSum(p);
    ps[hh * kChunk + lane] = p;
    if (lane == 0) {
      stats[2 * hh] = m;
      stats[2 * hh + 1] = l;
    }
  }
  __syncthreads();

  // Values: wave w adds keys 16 w .. 16 w + 15 of the chunk, lanes over
  // dimensions.
  float o[kMaxGroup][kPerLane];
#pragma unroll
  for (int hh = 0; hh < kMaxGroup; ++hh)
#pragma unroll
    for (int j = 0; j < kPerLane; ++j)
      o[hh][j] = 0.0F;
  for (int kk = 0; kk < 16; ++kk) {
    const int key_local = 16 * wave + kk;
    const int key = key0 + key_local;
    if (key >= key1)
      break;
    const float* vrow =
        a.v + (static_cast<std::size_t>(g) * a.capacity + first + key) * D + lane * kPerLane;
    float vv[kPerLane];
#pragma unroll
    for (int j = 0; j < kPerLane; ++j)
      vv[j] = vrow[j];
#pragma unroll
    for (int hh = 0; hh < kMaxGroup; ++hh) {
      if (hh >= group)
        break;
      const float p = ps[hh * kChunk + key_local];
#pragma unroll
      for (int j = 0; j < kPerLane; ++j)
        o[hh][j] += p * vv[j];
    }
  }
#pragma unroll
  for (int hh = 0; hh < kMaxGroup; ++hh) {
    if (hh >= group)
      break;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j)
      parts[(wave * group + hh) * D + lane * kPerLane + j] = o[hh][j];
  }
  __syncthreads();
  const int width = a.heads * D;
  for (int e = static_cast<int>(threadIdx.x); e < group * D; e += kThreads) {
    float total = parts[e];
#pragma unroll
    for (int w = 1; w < kWaves; ++w)
      total += parts[w * group * D + e];
    const int hh = e / D;
    const int d = e % D;
    if (a.splits == 1) {
      a.out[OutIndex(a, row, (g * group + hh) * D + d, width)] =
          Bf16Bits(total * (1.0F / stats[2 * hh + 1]));
    } else {
      float* target = a.partials + (partial0 + static_cast<std::size_t>(hh) * a.splits) * stride;
      target[2 + d] = total;
      if (d == 0) {
        target[0] = stats[2 * hh];
        target[1] = stats[2 * hh + 1];
      }
    }
  }
}

/// The chunks of one (row, head) met in chunk order: M = max m_c,
/// L = sum l_c exp(m_c - M), out = bf16(sum o_c exp(m_c - M) / L).
template<int D>
__global__ __launch_bounds__(kWave) void MergeKernel(AttentionArgs a) {
  constexpr int kPerLane = D / kWave;
  const int row = static_cast<int>(blockIdx.x);
  const int head = static_cast<int>(blockIdx.y);
  const int lane = static_cast<int>(threadIdx.x);
  const std::size_t stride = static_cast<std::size_t>(D) + 2;
  const float* base =
      a.partials + (static_cast<std::size_t>(row) * a.heads + head) * a.splits * stride;
  float m = -INFINITY;
  for (int c = 0; c < a.splits; ++c)
    m = fmaxf(m, base[c * stride]);
  float l = 0.0F;
  float o[kPerLane];
#pragma unroll
  for (int j = 0; j < kPerLane; ++j)
    o[j] = 0.0F;
  for (int c = 0; c < a.splits; ++c) {
    const float* part = base + c * stride;
    if (part[1] == 0.0F)
      continue;  // an empty chunk
    const float factor = expf(part[0] - m);
    l += part[1] * factor;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j)
      o[j] += part[2 + lane * kPerLane + j] * factor;
  }
  const float inverse = 1.0F / l;
  const int width = a.heads * D;
#pragma unroll
  for (int j = 0; j < kPerLane; ++j)
    a.out[OutIndex(a, row, head * D + lane * kPerLane + j, width)] = Bf16Bits(o[j] * inverse);
}

template<int D>
void LaunchAttention(const AttentionArgs& a, int rows, hipStream_t stream) {
  const int group = a.heads / a.kv_heads;
  const std::size_t shared = SharedFloats(group, D) * sizeof(float);
  SplitAttentionKernel<D><<<dim3(static_cast<unsigned>(a.splits), static_cast<unsigned>(rows),
                                 static_cast<unsigned>(a.kv_heads)),
                            kThreads, shared, stream>>>(a);
  if (a.splits > 1)
    MergeKernel<D><<<dim3(static_cast<unsigned>(rows), static_cast<unsigned>(a.heads)), kWave, 0,
                     stream>>>(a);
}

}  // namespace

/// Chunks per (row, KV head) for rows that attend to at most
/// past + rows_per_sequence keys.
int AttentionSplits(std::size_t past, std::size_t rows_per_sequence) {
  return static_cast<int>((past + rows_per_sequence + kChunk - 1) / kChunk);
}

/// Floats of the chunks' partial results of `rows` rows.
std::size_t AttentionPartialFloats(std::size_t rows, std::size_t heads, std::size_t head_dim,
                                   int splits) {
  return splits > 1 ? rows * heads * static_cast<std::size_t>(splits) * (head_dim + 2) : 0;
}

/// Checks the shape the split attention takes: head_dim 64 or 128 (VoxCPM2's
/// stacks take 128), at most 16 query heads per KV head, its LDS within
/// 64 KB.
bool AttentionSupported(std::size_t heads, std::size_t kv_heads, std::size_t head_dim) {
  if (kv_heads == 0 || heads % kv_heads != 0 || heads / kv_heads > kMaxGroup)
    return false;
  if (head_dim != 64 && head_dim != 128)
    return false;
  return SharedFloats(static_cast<int>(heads / kv_heads), static_cast<int>(head_dim)) *
             sizeof(float) <=
         65536;
}

/// The split attention over one layer's cache (the caller has checked the
/// shape, the bounds and the partials' size).
void Attention(const float* q, const float* k_cache, const float* v_cache, Bf16* out,
               bool fragment, float* partials, std::size_t rows,
               std::size_t rows_per_sequence, std::size_t keys_per_sequence, std::size_t past,
               bool causal, std::size_t heads, std::size_t kv_heads, std::size_t head_dim,
               std::size_t capacity, hipStream_t stream) {
  AttentionArgs a{};
  a.q = q;
  a.k = k_cache;
  a.v = v_cache;
  a.out = out;
  a.partials = partials;
  a.rows_per_sequence = static_cast<int>(rows_per_sequence);
  a.keys_per_sequence = static_cast<int>(keys_per_sequence);
  a.past = static_cast<int>(past);
  a.causal = causal ? 1 : 0;
  a.heads = static_cast<int>(heads);
  a.kv_heads = static_cast<int>(kv_heads);
  a.capacity = static_cast<int>(capacity);
  a.splits = AttentionSplits(past, rows_per_sequence);
  a.scale = 1.0F / std::sqrt(static_cast<float>(head_dim));
  a.fragment = fragment ? 1 : 0;
  const int r = static_cast<int>(rows);
  if (head_dim == 64)
    LaunchAttention<64>(a, r, stream);
  else
    LaunchAttention<128>(a, r, stream);
}

namespace {

/// h (fragment order [32][hidden]) from row-major rows.
__global__ void ToFragmentsKernel(const float* rows_in, float* h, int rows, int width) {
  const int e = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
  if (e >= rows * width)
    return;
  h[q8::F32FragIndex(e / width, e % width)] = rows_in[e];
}

/// Row-major rows from h (fragment order).
__global__ void FromFragmentsKernel(const float* h, float* rows_out, int rows, int width) {
  const int e = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
  if (e >= rows * width)
    return;
  rows_out[e] = h[q8::F32FragIndex(e / width, e % width)];
}

}  // namespace

void ToFragments(const float* rows_in, float* h, int rows, int width, hipStream_t stream) {
  const int count = rows * width;
  ToFragmentsKernel<<<(count + 255) / 256, 256, 0, stream>>>(rows_in, h, rows, width);
}

void FromFragments(const float* h, float* rows_out, int rows, int width, hipStream_t stream) {
  const int count = rows * width;
  FromFragmentsKernel<<<(count + 255) / 256, 256, 0, stream>>>(h, rows_out, rows, width);
}

}  // namespace vx::stack

namespace {

using vx::Bf16;

template<typename T>
int Grow(T** pointer, std::size_t* have, std::size_t need, const char* what) {
  if (need <= *have)
    return VX_OK;
  if (*pointer != nullptr)
    (void)hipFree(*pointer);
  *pointer = nullptr;
  *have = 0;
  const hipError_t error =
      hipMalloc(reinterpret_cast<void**>(pointer), std::max<std::size_t>(need, 1) * sizeof(T));
  if (error != hipSuccess)
    return vx::FailHip(error, what);
  *have = need;
  return VX_OK;
}

}  // namespace

struct vx_stack {
  vx_stack_shape shape{};
  vx_stack_weights weights{};
  std::vector<vx_dit_layer> layers;
  std::size_t q_width = 0;
  std::size_t kv_width = 0;
  std::size_t qkv_width = 0;
  bool fused = false;
  vx::fused::Shape fs{};
  int path = VX_STACK_PATH_AUTO;

  // Row-major scratch of the per-kernel path (grown to the rows seen).
  float* qkv = nullptr;
  std::size_t qkv_floats = 0;
  float* q = nullptr;
  std::size_t q_floats = 0;
  Bf16* bf16 = nullptr;
  std::size_t bf16_count = 0;
  float* gate_up = nullptr;
  std::size_t gate_up_floats = 0;
  float* attention_partials = nullptr;
  std::size_t attention_partial_floats = 0;
  float* product_partials = nullptr;  // products beyond 128 rows
  std::size_t product_partial_floats = 0;

  // The fused path: 32-row fragment-order buffers.
  float* h_frag = nullptr;
  Bf16* attention_frag = nullptr;
  Bf16* swiglu_frag = nullptr;

  ~vx_stack() {
    for (void* pointer :
         {static_cast<void*>(qkv), static_cast<void*>(q), static_cast<void*>(bf16),
          static_cast<void*>(gate_up), static_cast<void*>(attention_partials),
          static_cast<void*>(product_partials), static_cast<void*>(h_frag),
          static_cast<void*>(attention_frag), static_cast<void*>(swiglu_frag)})
      if (pointer != nullptr)
        (void)hipFree(pointer);
  }

  vx::q8::Weights Kind() const {
    return weights.format == VX_WEIGHTS_BF16 ? vx::q8::Weights::kBf16 : vx::q8::Weights::kQ8;
  }

  /// Bf16Gemm::Linear (gemm.cpp:259-313): y[m][n] (+)= x W^T.
  int Linear(const Bf16* x, const void* w, float* y, std::size_t m, std::size_t k,
             std::size_t n, bool accumulate, hipStream_t stream) {
    if (m > vx::kExactRows) {
      VX_TRY(Grow(&product_partials, &product_partial_floats, 2 * m * n,
                  "vx_stack_forward: hipMalloc"));
      return vx::RunTiled(x, w, y, nullptr, m, k, n, accumulate,
                          Kind() == vx::q8::Weights::kQ8 ? vx::TiledMode::kQ8Expanded
                                                         : vx::TiledMode::kBf16,
                          product_partials, product_partial_floats, stream);
    }
    const vx::ProductPlan plan = vx::PlanSkinny(m, k, n, 0, 0);
    return vx::RunSkinny(x, w, y, nullptr, m, k, n, accumulate, plan, nullptr, nullptr,
                         stream, Kind());
  }

  int Resolved(std::size_t rows) const {
    if (path == VX_STACK_PATH_UNFUSED || !fused || rows > vx::q8::kFragRows)
      return VX_STACK_PATH_UNFUSED;
    return VX_STACK_PATH_FUSED;
  }

  int Forward(float* hidden, float* output, std::size_t rows, const std::int32_t* positions,
              const std::int32_t* cache_rows, std::size_t rows_per_sequence,
              std::size_t keys_per_sequence, std::size_t past, bool causal, float* k_cache,
              float* v_cache, std::size_t capacity, hipStream_t stream) {
    const std::size_t width = shape.hidden;
    const std::size_t ffn = shape.ffn;
    const std::size_t layer_stride = shape.kv_heads * capacity * shape.head_dim;
    const int splits = vx::stack::AttentionSplits(past, rows_per_sequence);
    VX_TRY(Grow(&attention_partials, &attention_partial_floats,
                vx::stack::AttentionPartialFloats(rows, shape.heads, shape.head_dim, splits),
                "vx_stack_forward: hipMalloc"));
    VX_TRY(Grow(&q, &q_floats, rows * q_width, "vx_stack_forward: hipMalloc"));
    VX_TRY(Grow(&qkv, &qkv_floats, rows * qkv_width, "vx_stack_forward: hipMalloc"));
    const float* rope = shape.rope != 0 ? weights.rope : nullptr;

    if (Resolved(rows) == VX_STACK_PATH_FUSED) {
      vx::fused::Shape s = fs;
      s.rows = static_cast<int>(rows);
      vx::stack::ToFragments(hidden, h_frag, s.rows, s.hidden, stream);
      for (std::size_t l = 0; l < layers.size(); ++l) {
        const vx_dit_layer& layer = layers[l];
        float* keys = k_cache + l * layer_stride;
        float* values = v_cache + l * layer_stride;
        vx::fused::Qkv(h_frag, layer.input_norm, layer.qkv, qkv, s, stream);
        vx::kernels::QkvRope(qkv, rope, positions, cache_rows, q, keys, values, rows,
                             shape.heads, shape.kv_heads, shape.head_dim, capacity, stream);
        vx::stack::Attention(q, keys, values, attention_frag, true, attention_partials, rows,
                             rows_per_sequence, keys_per_sequence, past, causal, shape.heads,
                             shape.kv_heads, shape.head_dim, capacity, stream);
        vx::fused::Residual(attention_frag, layer.o, static_cast<int>(q_width), s.hidden,
                            h_frag, s, stream);
        vx::fused::GateUp(h_frag, layer.post_norm, layer.gate_up, swiglu_frag, s, stream);
        vx::fused::Residual(swiglu_frag, layer.down, s.ffn, s.hidden, h_frag, s, stream);
      }
      vx::stack::FromFragments(h_frag, hidden, s.rows, s.hidden, stream);
      VX_TRY(Grow(&bf16, &bf16_count, rows * width, "vx_stack_forward: hipMalloc"));
      vx::kernels::RmsNorm(hidden, weights.norm, bf16, output, rows, width, shape.eps, stream);
      return vx::LaunchStatus("vx_stack_forward");
    }

    const std::size_t wide = std::max({width, qkv_width, ffn});
    VX_TRY(Grow(&bf16, &bf16_count, rows * wide, "vx_stack_forward: hipMalloc"));
    VX_TRY(Grow(&gate_up, &gate_up_floats, rows * 2 * ffn, "vx_stack_forward: hipMalloc"));
    for (std::size_t l = 0; l < layers.size(); ++l) {
      const vx_dit_layer& layer = layers[l];
      float* keys = k_cache + l * layer_stride;
      float* values = v_cache + l * layer_stride;
      vx::kernels::RmsNorm(hidden, layer.input_norm, bf16, nullptr, rows, width, shape.eps,
                           stream);
      VX_TRY(Linear(bf16, layer.qkv, qkv, rows, width, qkv_width, false, stream));
      vx::kernels::QkvRope(qkv, rope, positions, cache_rows, q, keys, values, rows,
                           shape.heads, shape.kv_heads, shape.head_dim, capacity, stream);
      vx::stack::Attention(q, keys, values, bf16, false, attention_partials, rows,
                           rows_per_sequence, keys_per_sequence, past, causal, shape.heads,
                           shape.kv_heads, shape.head_dim, capacity, stream);
      VX_TRY(Linear(bf16, layer.o, hidden, rows, q_width, width, true, stream));
      vx::kernels::RmsNorm(hidden, layer.post_norm, bf16, nullptr, rows, width, shape.eps,
                           stream);
      VX_TRY(Linear(bf16, layer.gate_up, gate_up, rows, width, 2 * ffn, false, stream));
      vx::kernels::SwiGlu(gate_up, bf16, rows, ffn, stream);
      VX_TRY(Linear(bf16, layer.down, hidden, rows, ffn, width, true, stream));
    }
    vx::kernels::RmsNorm(hidden, weights.norm, bf16, output, rows, width, shape.eps, stream);
    return vx::LaunchStatus("vx_stack_forward");
  }
};

namespace {

int CheckStack(const vx_stack_shape& s, const vx_stack_weights& w) {
  if (s.hidden == 0 || s.heads == 0 || s.kv_heads == 0 || s.head_dim == 0 || s.ffn == 0 ||
      s.layers == 0)
    return vx::Fail(VX_BAD_ARG, "vx_stack_create: zero dimension");
  if (s.hidden % 32 != 0 || (s.heads * s.head_dim) % 32 != 0 || s.ffn % 32 != 0)
    return vx::Fail(VX_BAD_ARG,
                    "vx_stack_create: hidden, heads x head_dim and ffn must be multiples "
                    "of 32 (Q8_0 blocks)");
  if (s.head_dim % 2 != 0)
    return vx::Fail(VX_BAD_ARG, "vx_stack_create: head_dim must be even");
  if (!vx::stack::AttentionSupported(s.heads, s.kv_heads, s.head_dim))
    return vx::Fail(VX_UNSUPPORTED,
                    "vx_stack_create: attention takes head_dim 64 or 128 and at most 16 "
                    "query heads per KV head");
  if (w.layers == nullptr || w.norm == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_stack_create: null weights");
  if (s.rope != 0 && w.rope == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_stack_create: rotary stack without a table");
  if (w.format != VX_WEIGHTS_Q8_0 && w.format != VX_WEIGHTS_BF16)
    return vx::Fail(VX_BAD_ARG, "vx_stack_create: unknown weight format");
  for (std::size_t l = 0; l < s.layers; ++l) {
    const vx_dit_layer& layer = w.layers[l];
    if (layer.input_norm == nullptr || layer.qkv == nullptr || layer.o == nullptr ||
        layer.post_norm == nullptr || layer.gate_up == nullptr || layer.down == nullptr)
      return vx::Fail(VX_BAD_ARG, "vx_stack_create: null layer weights");
  }
  return VX_OK;
}

template<typename T>
int Allocate(T** pointer, std::size_t count) {
  const hipError_t error = hipMalloc(reinterpret_cast<void**>(pointer),
                                     std::max<std::size_t>(count, 1) * sizeof(T));
  if (error != hipSuccess)
    return vx::FailHip(error, "vx_stack_create: hipMalloc");
  return VX_OK;
}

}  // namespace

extern "C" {

int vx_stack_create(vx_stack** stack, const vx_stack_shape* shape,
                    const vx_stack_weights* weights) {
  if (stack == nullptr || shape == nullptr || weights == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_stack_create: null argument");
  *stack = nullptr;
  VX_TRY(CheckStack(*shape, *weights));
  auto* created = new vx_stack();
  created->shape = *shape;
  created->weights = *weights;
  created->layers.assign(weights->layers, weights->layers + shape->layers);
  created->weights.layers = created->layers.data();
  created->q_width = shape->heads * shape->head_dim;
  created->kv_width = shape->kv_heads * shape->head_dim;
  created->qkv_width = created->q_width + 2 * created->kv_width;
  vx::fused::Shape& fs = created->fs;
  fs.rows = vx::q8::kFragRows;
  fs.hidden = static_cast<int>(shape->hidden);
  fs.heads = static_cast<int>(shape->heads);
  fs.kv_heads = static_cast<int>(shape->kv_heads);
  fs.head_dim = static_cast<int>(shape->head_dim);
  fs.ffn = static_cast<int>(shape->ffn);
  fs.eps = shape->eps;
  fs.weights = created->Kind();
  created->fused = vx::fused::StackSupported(fs);
  int status = VX_OK;
  if (created->fused) {
    status = Allocate(&created->h_frag, vx::q8::FragElements(shape->hidden));
    if (status == VX_OK)
      status = Allocate(&created->attention_frag, vx::q8::FragElements(created->q_width));
    if (status == VX_OK)
      status = Allocate(&created->swiglu_frag, vx::q8::FragElements(shape->ffn));
  }
  if (status != VX_OK) {
    delete created;
    return status;
  }
  *stack = created;
  return VX_OK;
}

int vx_stack_forward(vx_stack* stack, float* hidden, float* output, size_t rows,
                     const int32_t* positions, const int32_t* cache_rows,
                     size_t rows_per_sequence, size_t keys_per_sequence, size_t past,
                     int causal, float* k_cache, float* v_cache, size_t capacity,
                     void* stream) {
  if (stack == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_stack_forward: null handle");
  if (hidden == nullptr || output == nullptr || positions == nullptr ||
      cache_rows == nullptr || k_cache == nullptr || v_cache == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_stack_forward: null pointer");
  if (rows == 0 || rows_per_sequence == 0 || rows % rows_per_sequence != 0)
    return vx::Fail(VX_BAD_ARG,
                    "vx_stack_forward: rows must be a positive multiple of rows_per_sequence");
  // Every key a row attends to lies in the cache: sequence s reads keys
  // s keys_per_sequence .. + past + rows_per_sequence.
  const std::size_t sequences = rows / rows_per_sequence;
  if ((sequences - 1) * keys_per_sequence + past + rows_per_sequence > capacity)
    return vx::Fail(VX_BAD_ARG, "vx_stack_forward: the attended keys exceed the cache");
  if (capacity > (1U << 24) || rows > (1U << 16))
    return vx::Fail(VX_BAD_ARG, "vx_stack_forward: capacity or rows too large");
  return stack->Forward(hidden, output, rows, positions, cache_rows, rows_per_sequence,
                        keys_per_sequence, past, causal != 0, k_cache, v_cache, capacity,
                        vx::Stream(stream));
}

void vx_stack_destroy(vx_stack* stack) { delete stack; }

int vx_stack_set_path(vx_stack* stack, int path) {
  if (stack == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_stack_set_path: null handle");
  if (path == VX_STACK_PATH_FUSED && !stack->fused)
    return vx::Fail(VX_UNSUPPORTED, "vx_stack_set_path: no fused kernels for this shape");
  if (path != VX_STACK_PATH_AUTO && path != VX_STACK_PATH_FUSED &&
      path != VX_STACK_PATH_UNFUSED)
    return vx::Fail(VX_BAD_ARG, "vx_stack_set_path: unknown path");
  stack->path = path;
  return VX_OK;
}

int vx_stack_path(const vx_stack* stack, size_t rows) {
  return stack == nullptr ? -1 : stack->Resolved(rows);
}

int vx_split_attention(const float* q, const float* k_cache, const float* v_cache,
                       uint16_t* output, size_t rows, size_t rows_per_sequence,
                       size_t keys_per_sequence, size_t past, int causal, size_t heads,
                       size_t kv_heads, size_t head_dim, size_t capacity, float* partials,
                       size_t partial_floats, void* stream) {
  if (q == nullptr || k_cache == nullptr || v_cache == nullptr || output == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_split_attention: null pointer");
  if (rows == 0 || rows_per_sequence == 0 || rows % rows_per_sequence != 0)
    return vx::Fail(VX_BAD_ARG, "vx_split_attention: bad rows");
  if (!vx::stack::AttentionSupported(heads, kv_heads, head_dim))
    return vx::Fail(VX_UNSUPPORTED, "vx_split_attention: unsupported heads or head_dim");
  const std::size_t sequences = rows / rows_per_sequence;
  if ((sequences - 1) * keys_per_sequence + past + rows_per_sequence > capacity)
    return vx::Fail(VX_BAD_ARG, "vx_split_attention: the attended keys exceed the cache");
  const int splits = vx::stack::AttentionSplits(past, rows_per_sequence);
  if (vx::stack::AttentionPartialFloats(rows, heads, head_dim, splits) > partial_floats ||
      (splits > 1 && partials == nullptr))
    return vx::Fail(VX_BAD_ARG, "vx_split_attention: partials too small");
  vx::stack::Attention(q, k_cache, v_cache, output, false, partials, rows, rows_per_sequence,
                       keys_per_sequence, past, causal != 0, heads, kv_heads, head_dim,
                       capacity, vx::Stream(stream));
  return vx::LaunchStatus("vx_split_attention");
}

size_t vx_split_attention_floats(size_t rows, size_t heads, size_t head_dim, size_t past,
                                 size_t rows_per_sequence) {
  if (rows_per_sequence == 0)
    return 0;
  return vx::stack::AttentionPartialFloats(
      rows, heads, head_dim, vx::stack::AttentionSplits(past, rows_per_sequence));
}

}  // extern "C"
