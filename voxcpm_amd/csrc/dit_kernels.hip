// The DiT's non-product kernels for wave64 (gfx950): RMSNorm, the q/k/v
// split with rotary embedding, bidirectional attention over a branch's
// rows, SwiGLU, bias, bf16 conversion, row gather and assembly, and the
// guided Euler update. Each follows the reference kernel cited at its
// launcher; reductions use 64-lane waves.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>

#include "common.hpp"
#include "dit_kernels.hpp"

namespace vx::kernels {
namespace {

constexpr int kThreads = 256;

dim3 Blocks(std::size_t count, int threads = kThreads) {
  return dim3(static_cast<unsigned>((count + threads - 1) / threads));
}

__device__ inline float Silu(float value) {
  return value / (1.0F + expf(-value));
}

__global__ void RmsNormKernel(const float* input, const Bf16* weight,
                              Bf16* output, float* output_f32, int width,
                              float epsilon) {
  __shared__ float scratch[kThreads / kWave];
  const std::size_t row = blockIdx.x;
  const float* x = input + row * width;
  float sum = 0.0F;
  for (int i = threadIdx.x; i < width; i += blockDim.x)
    sum += x[i] * x[i];
  sum = BlockSum(sum, scratch);
  const float inverse = rsqrtf(sum / static_cast<float>(width) + epsilon);
  for (int i = threadIdx.x; i < width; i += blockDim.x) {
    const float value = x[i] * inverse * Bf16Value(weight[i]);
    output[row * width + i] = Bf16Bits(value);
    if (output_f32 != nullptr)
      output_f32[row * width + i] = value;
  }
}

/// One workgroup per (row, head of q | k | v), one thread per rotated pair
/// (i, i + head_dim / 2): every load of a pair is issued at once. q and k
/// heads rotate (when a table is given) into q and the key cache; v heads
/// copy into the value cache.
__global__ void QkvRopeKernel(const float* qkv, const float* cos_sin,
                              const std::int32_t* positions,
                              const std::int32_t* cache_rows, float* q,
                              float* k_cache, float* v_cache, int heads,
                              int kv_heads, int head_dim, int capacity) {
  const std::size_t row = blockIdx.x;
  const int head = static_cast<int>(blockIdx.y);
  const int half = head_dim / 2;
  const int width = (heads + 2 * kv_heads) * head_dim;
  const float* source = qkv + row * width + static_cast<std::size_t>(head) * head_dim;
  const std::size_t cache_row = static_cast<std::size_t>(cache_rows[row]);
  for (int i = threadIdx.x; i < half; i += blockDim.x) {
    const float a = source[i];
    const float b = source[half + i];
    if (head >= heads + kv_heads) {  // a value head
      float* target = v_cache +
                      (static_cast<std::size_t>(head - heads - kv_heads) * capacity + cache_row) *
                          head_dim;
      target[i] = a;
      target[half + i] = b;
      continue;
    }
    float first = a;
    float second = b;
    if (cos_sin != nullptr) {
      const float* table = cos_sin + static_cast<std::size_t>(positions[row]) * head_dim;
      const float c = table[i];
      const float s = table[half + i];
      first = a * c - b * s;
      second = b * c + a * s;
    }
    float* target =
        head < heads
            ? q + (row * heads + head) * head_dim
            : k_cache + ((static_cast<std::size_t>(head - heads) * capacity) + cache_row) *
                            head_dim;
    target[i] = first;
    target[half + i] = second;
  }
}

// One wave per (row, head); lane d holds dimensions d, d + 64, ... of the
// scaled query, its keys and the output. Keys run in order with an online
// softmax (running maximum and sum).
constexpr int kMaxDimsPerLane = 4;  // head_dim <= 256

__global__ __launch_bounds__(kWave) void AttentionKernel(
    const float* q, const float* k_cache, const float* v_cache, Bf16* output,
    int rows_per_sequence, int keys_per_sequence, int past, int causal,
    int heads, int kv_heads, int head_dim, int capacity, float scale) {
  const int lane = threadIdx.x;
  const std::size_t row = blockIdx.x;
  const int head = blockIdx.y;
  const int sequence = static_cast<int>(row) / rows_per_sequence;
  const int local = static_cast<int>(row) % rows_per_sequence;
  const int count = past + (causal ? local + 1 : rows_per_sequence);
  const int first_key = sequence * keys_per_sequence;
  const int kv_head = head / (heads / kv_heads);
  const float* keys =
      k_cache + (static_cast<std::size_t>(kv_head) * capacity + first_key) *
                    head_dim;
  const float* values =
      v_cache + (static_cast<std::size_t>(kv_head) * capacity + first_key) *
                    head_dim;
  const float* query = q + (row * heads + head) * head_dim;
  float qd[kMaxDimsPerLane];
  float out[kMaxDimsPerLane];
#pragma unroll
  for (int j = 0; j < kMaxDimsPerLane; ++j) {
    const int d = lane + kWave * j;
    qd[j] = d < head_dim ? query[d] * scale : 0.0F;
    out[j] = 0.0F;
  }
  float maximum = -INFINITY;
  float sum = 0.0F;
  for (int key = 0; key < count; ++key) {
    float partial = 0.0F;
#pragma unroll
    for (int j = 0; j < kMaxDimsPerLane; ++j) {
      const int d = lane + kWave * j;
      if (d < head_dim)
        partial += qd[j] * keys[static_cast<std::size_t>(key) * head_dim + d];
    }
    const float score = WaveSum(partial);
    const float next = fmaxf(maximum, score);
    const float decay = expf(maximum - next);
    const float weight = expf(score - next);
    sum = sum * decay + weight;
#pragma unroll
    for (int j = 0; j < kMaxDimsPerLane; ++j) {
      const int d = lane + kWave * j;
      if (d < head_dim)
        out[j] = out[j] * decay +
                 weight * values[static_cast<std::size_t>(key) * head_dim + d];
    }
    maximum = next;
  }
  const float inverse = 1.0F / sum;
  Bf16* target = output + (row * heads + head) * head_dim;
#pragma unroll
  for (int j = 0; j < kMaxDimsPerLane; ++j) {
    const int d = lane + kWave * j;
    if (d < head_dim)
      target[d] = Bf16Bits(out[j] * inverse);
  }
}

__global__ void SwiGluKernel(const float* gate_up, Bf16* output,
                             std::size_t rows, std::size_t width) {
  const std::size_t index =
      static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (index >= rows * width)
    return;
  const std::size_t row = index / width;
  const std::size_t i = index % width;
  const float gate = gate_up[row * 2 * width + i];
  const float up = gate_up[row * 2 * width + width + i];
  output[index] = Bf16Bits(Silu(gate) * up);
}

__global__ void AddBiasKernel(float* data, const Bf16* bias, std::size_t rows,
                              std::size_t width) {
  const std::size_t index =
      static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (index < rows * width)
    data[index] += Bf16Value(bias[index % width]);
}

__global__ void ToBf16Kernel(const float* input, Bf16* output,
                             std::size_t count, int silu) {
  const std::size_t index =
      static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (index >= count)
    return;
  float value = input[index];
  if (silu)
    value = Silu(value);
  output[index] = Bf16Bits(value);
}

__global__ void GatherRowsKernel(const float* input,
                                 const std::int32_t* indices, float* output,
                                 int width) {
  const std::size_t row = blockIdx.x;
  const std::size_t source = static_cast<std::size_t>(indices[row]);
  for (int i = threadIdx.x; i < width; i += blockDim.x)
    output[row * width + i] = input[source * width + i];
}

__global__ void AssembleDitKernel(const float* mu, const float* time,
                                  const float* cond, const float* x,
                                  float* output, int patch, int width) {
  const int sequence = blockIdx.x;  // 0 conditional, 1 unconditional
  const int row = blockIdx.y;
  const int length = 3 + 2 * patch;
  float* target =
      output + (static_cast<std::size_t>(sequence) * length + row) * width;
  for (int i = threadIdx.x; i < width; i += blockDim.x) {
    float value;
    if (row < 2)
      value = sequence == 0 ? mu[row * width + i] : 0.0F;
    else if (row == 2)
      value = time[i];
    else if (row < 3 + patch)
      value = cond[(row - 3) * width + i];
    else
      value = x[(row - 3 - patch) * width + i];
    target[i] = value;
  }
}

__global__ void GuidedEulerKernel(const float* velocity, float* x, int count,
                                  float cfg, float dt, int zero_star) {
  __shared__ float scratch[kThreads / kWave];
  const float* c = velocity;
  const float* u = velocity + count;
  float s = 1.0F;
  if (zero_star) {
    float dot = 0.0F;
    float norm = 0.0F;
    for (int i = threadIdx.x; i < count; i += blockDim.x) {
      dot += c[i] * u[i];
      norm += u[i] * u[i];
    }
    dot = BlockSum(dot, scratch);
    norm = BlockSum(norm, scratch);
    s = dot / (norm + 1e-8F);
  }
  for (int i = threadIdx.x; i < count; i += blockDim.x) {
    const float guided = u[i] * s + cfg * (c[i] - u[i] * s);
    x[i] -= dt * guided;
  }
}

__global__ void CopyKernel(const float* src, float* dst, std::size_t count) {
  const std::size_t index =
      static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (index < count)
    dst[index] = src[index];
}

}  // namespace

// kernels/generator_kernels.hip:91-108
void RmsNorm(const float* input, const Bf16* weight, Bf16* output,
             float* output_f32, std::size_t rows, std::size_t width,
             float epsilon, hipStream_t stream) {
  if (rows == 0)
    return;
  RmsNormKernel<<<static_cast<unsigned>(rows), kThreads, 0, stream>>>(
      input, weight, output, output_f32, static_cast<int>(width), epsilon);
}

// kernels/generator_kernels.hip:110-158
void QkvRope(const float* qkv, const float* cos_sin,
             const std::int32_t* positions, const std::int32_t* cache_rows,
             float* q, float* k_cache, float* v_cache, std::size_t rows,
             std::size_t heads, std::size_t kv_heads, std::size_t head_dim,
             std::size_t capacity, hipStream_t stream) {
  if (rows == 0)
    return;
  const unsigned threads = static_cast<unsigned>(
      std::min<std::size_t>(256, (head_dim / 2 + kWave - 1) / kWave * kWave));
  QkvRopeKernel<<<dim3(static_cast<unsigned>(rows), static_cast<unsigned>(heads + 2 * kv_heads)),
                  threads, 0, stream>>>(
      qkv, cos_sin, positions, cache_rows, q, k_cache, v_cache,
      static_cast<int>(heads), static_cast<int>(kv_heads),
      static_cast<int>(head_dim), static_cast<int>(capacity));
}

// kernels/generator_kernels.hip:160-241, 408-420
void Attention(const float* q, const float* k_cache, const float* v_cache,
               Bf16* output, std::size_t rows, std::size_t rows_per_sequence,
               std::size_t keys_per_sequence, std::size_t past, bool causal,
               std::size_t heads, std::size_t kv_heads, std::size_t head_dim,
               std::size_t capacity, hipStream_t stream) {
  if (rows == 0)
    return;
  AttentionKernel<<<dim3(static_cast<unsigned>(rows),
                         static_cast<unsigned>(heads)),
                    kWave, 0, stream>>>(
      q, k_cache, v_cache, output, static_cast<int>(rows_per_sequence),
      static_cast<int>(keys_per_sequence), static_cast<int>(past),
      causal ? 1 : 0, static_cast<int>(heads), static_cast<int>(kv_heads),
      static_cast<int>(head_dim), static_cast<int>(capacity),
      1.0F / std::sqrt(static_cast<float>(head_dim)));
}

// kernels/generator_kernels.hip:243-254
void SwiGlu(const float* gate_up, Bf16* output, std::size_t rows,
            std::size_t width, hipStream_t stream) {
  if (rows * width == 0)
    return;
  SwiGluKernel<<<Blocks(rows * width), kThreads, 0, stream>>>(gate_up, output,
                                                              rows, width);
}

// kernels/generator_kernels.hip:256-262
void AddBias(float* data, const Bf16* bias, std::size_t rows,
             std::size_t width, hipStream_t stream) {
  if (rows * width == 0)
    return;
  AddBiasKernel<<<Blocks(rows * width), kThreads, 0, stream>>>(data, bias,
                                                               rows, width);
}

// kernels/generator_kernels.hip:264-274
void ToBf16(const float* input, Bf16* output, std::size_t count, bool silu,
            hipStream_t stream) {
  if (count == 0)
    return;
  ToBf16Kernel<<<Blocks(count), kThreads, 0, stream>>>(input, output, count,
                                                       silu ? 1 : 0);
}

// kernels/generator_kernels.hip:82-89
void GatherRows(const float* input, const std::int32_t* indices,
                float* output, std::size_t rows, std::size_t width,
                hipStream_t stream) {
  if (rows == 0)
    return;
  GatherRowsKernel<<<static_cast<unsigned>(rows), kThreads, 0, stream>>>(
      input, indices, output, static_cast<int>(width));
}

// kernels/generator_kernels.hip:320-340
void AssembleDit(const float* mu, const float* time, const float* cond,
                 const float* x, float* output, std::size_t patch,
                 std::size_t width, hipStream_t stream) {
  AssembleDitKernel<<<dim3(2, static_cast<unsigned>(3 + 2 * patch)), kThreads,
                      0, stream>>>(mu, time, cond, x, output,
                                   static_cast<int>(patch),
                                   static_cast<int>(width));
}

// kernels/generator_kernels.hip:342-360
void GuidedEuler(const float* velocity, float* x, std::size_t count, float cfg,
                 float dt, bool zero_star, hipStream_t stream) {
  GuidedEulerKernel<<<1, kThreads, 0, stream>>>(
      velocity, x, static_cast<int>(count), cfg, dt, zero_star ? 1 : 0);
}

void CopyFloats(const float* src, float* dst, std::size_t count,
                hipStream_t stream) {
  if (count == 0)
    return;
  CopyKernel<<<Blocks(count), kThreads, 0, stream>>>(src, dst, count);
}

}  // namespace vx::kernels

// ---- C ABI wrappers --------------------------------------------------------

namespace {

int Null(const char* what) {
  return vx::Fail(VX_BAD_ARG, std::string(what) + ": null pointer");
}

}  // namespace

extern "C" {

int vx_rms_norm(const float* input, const uint16_t* weight, uint16_t* output,
                float* output_f32, size_t rows, size_t width, float epsilon,
                void* stream) {
  if (input == nullptr || weight == nullptr || output == nullptr)
    return Null("vx_rms_norm");
  if (width == 0)
    return vx::Fail(VX_BAD_ARG, "vx_rms_norm: zero width");
  vx::kernels::RmsNorm(input, weight, output, output_f32, rows, width, epsilon,
                       vx::Stream(stream));
  return vx::LaunchStatus("vx_rms_norm");
}

int vx_qkv_rope(const float* qkv, const float* cos_sin,
                const int32_t* positions, const int32_t* cache_rows, float* q,
                float* k_cache, float* v_cache, size_t rows, size_t heads,
                size_t kv_heads, size_t head_dim, size_t capacity,
                void* stream) {
  if (qkv == nullptr || cache_rows == nullptr || q == nullptr ||
      k_cache == nullptr || v_cache == nullptr ||
      (cos_sin != nullptr && positions == nullptr))
    return Null("vx_qkv_rope");
  if (heads == 0 || kv_heads == 0 || head_dim == 0 || head_dim % 2 != 0)
    return vx::Fail(VX_BAD_ARG, "vx_qkv_rope: bad head shape");
  vx::kernels::QkvRope(qkv, cos_sin, positions, cache_rows, q, k_cache,
                       v_cache, rows, heads, kv_heads, head_dim, capacity,
                       vx::Stream(stream));
  return vx::LaunchStatus("vx_qkv_rope");
}

int vx_attention(const float* q, const float* k_cache, const float* v_cache,
                 uint16_t* output, size_t rows, size_t rows_per_sequence,
                 size_t keys_per_sequence, size_t past, int causal,
                 size_t heads, size_t kv_heads, size_t head_dim,
                 size_t capacity, void* stream) {
  if (q == nullptr || k_cache == nullptr || v_cache == nullptr ||
      output == nullptr)
    return Null("vx_attention");
  if (heads == 0 || kv_heads == 0 || heads % kv_heads != 0)
    return vx::Fail(VX_BAD_ARG,
                    "vx_attention: heads must be a multiple of kv_heads");
  if (head_dim == 0 || head_dim > 256 || rows_per_sequence == 0)
    return vx::Fail(VX_UNSUPPORTED,
                    "vx_attention: head_dim must be in 1..256");
  const std::size_t sequences =
      (rows + rows_per_sequence - 1) / rows_per_sequence;
  if (rows > 0 &&
      (sequences - 1) * keys_per_sequence + past + rows_per_sequence >
          capacity)
    return vx::Fail(VX_BAD_ARG, "vx_attention: keys exceed the cache");
  vx::kernels::Attention(q, k_cache, v_cache, output, rows, rows_per_sequence,
                         keys_per_sequence, past, causal != 0, heads,
                         kv_heads, head_dim, capacity, vx::Stream(stream));
  return vx::LaunchStatus("vx_attention");
}

int vx_swiglu(const float* gate_up, uint16_t* output, size_t rows,
              size_t width, void* stream) {
  if (gate_up == nullptr || output == nullptr)
    return Null("vx_swiglu");
  vx::kernels::SwiGlu(gate_up, output, rows, width, vx::Stream(stream));
  return vx::LaunchStatus("vx_swiglu");
}

int vx_add_bias(float* data, const uint16_t* bias, size_t rows, size_t width,
                void* stream) {
  if (data == nullptr || bias == nullptr)
    return Null("vx_add_bias");
  vx::kernels::AddBias(data, bias, rows, width, vx::Stream(stream));
  return vx::LaunchStatus("vx_add_bias");
}

int vx_to_bf16(const float* input, uint16_t* output, size_t count, int silu,
               void* stream) {
  if (input == nullptr || output == nullptr)
    return Null("vx_to_bf16");
  vx::kernels::ToBf16(input, output, count, silu != 0, vx::Stream(stream));
  return vx::LaunchStatus("vx_to_bf16");
}

int vx_gather_rows(const float* input, const int32_t* indices, float* output,
                   size_t rows, size_t width, void* stream) {
  if (input == nullptr || indices == nullptr || output == nullptr)
    return Null("vx_gather_rows");
  vx::kernels::GatherRows(input, indices, output, rows, width,
                          vx::Stream(stream));
  return vx::LaunchStatus("vx_gather_rows");
}

int vx_assemble_dit(const float* mu, const float* time, const float* cond,
                    const float* x, float* output, size_t patch_size,
                    size_t width, void* stream) {
  if (mu == nullptr || time == nullptr || cond == nullptr || x == nullptr ||
      output == nullptr)
    return Null("vx_assemble_dit");
  vx::kernels::AssembleDit(mu, time, cond, x, output, patch_size, width,
                           vx::Stream(stream));
  return vx::LaunchStatus("vx_assemble_dit");
}

int vx_guided_euler(const float* velocity, float* x, size_t count, float cfg,
                    float dt, int zero_star, void* stream) {
  if (velocity == nullptr || x == nullptr)
    return Null("vx_guided_euler");
  vx::kernels::GuidedEuler(velocity, x, count, cfg, dt, zero_star != 0,
                           vx::Stream(stream));
  return vx::LaunchStatus("vx_guided_euler");
}

}  // extern "C"
