// The DiT's non-product kernels for wave64 (gfx950): RMSNorm, the q/k/v
// split with rotary embedding, bidirectional attention over a branch's
// rows, SwiGLU, bias, bf16 conversion, row gather and assembly, and the
// guided Euler update. Each follows the reference kernel cited at its
// launcher; reductions use 64-lane waves.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <initializer_list>

#include "common.hpp"
#include "dit_kernels.hpp"
#include "q8_tile.hpp"

namespace vx::kernels {
namespace {

constexpr int kThreads = 256;

dim3 Blocks(std::size_t count, int threads = kThreads) {
  return dim3(static_cast<unsigned>((count + threads - 1) / threads));
}

/// One access per thread over `accesses`, at most 4096 workgroups (the
/// kernels loop over the rest).
dim3 Grid(std::size_t accesses) {
  return dim3(static_cast<unsigned>(std::min<std::size_t>((accesses + kThreads - 1) / kThreads,
                                                          4096)));
}

/// Workgroups along a row of `accesses` accesses (grid x of the row copies).
unsigned RowBlocks(std::size_t accesses) {
  return static_cast<unsigned>(std::max<std::size_t>(1, (accesses + kThreads - 1) / kThreads));
}

__device__ inline float Silu(float value) {
  return value / (1.0F + expf(-value));
}

// ---- vector access -------------------------------------------------------
//
// The elementwise kernels move V consecutive values per access: V = 4 when
// every pointer is aligned for it and the widths are multiples of 4 (16-byte
// float32 and 8-byte bf16 accesses), else V = 1.

template<int V>
struct Lanes {
  float v[V];
};

template<int V>
__device__ inline Lanes<V> LoadF(const float* at) {
  Lanes<V> out;
  if constexpr (V == 4) {
    const float4 f = *reinterpret_cast<const float4*>(at);
    out.v[0] = f.x;
    out.v[1] = f.y;
    out.v[2] = f.z;
    out.v[3] = f.w;
  } else {
    out.v[0] = *at;
  }
  return out;
}

template<int V>
__device__ inline void StoreF(float* at, const Lanes<V>& in) {
  if constexpr (V == 4)
    *reinterpret_cast<float4*>(at) = float4{in.v[0], in.v[1], in.v[2], in.v[3]};
  else
    *at = in.v[0];
}

/// V bf16 values at `at` as float32.
template<int V>
__device__ inline Lanes<V> LoadB(const Bf16* at) {
  Lanes<V> out;
  if constexpr (V == 4) {
    const uint2 b = *reinterpret_cast<const uint2*>(at);
    out.v[0] = q8::Bf16Lo(b.x);
    out.v[1] = q8::Bf16Hi(b.x);
    out.v[2] = q8::Bf16Lo(b.y);
    out.v[3] = q8::Bf16Hi(b.y);
  } else {
    out.v[0] = Bf16Value(*at);
  }
  return out;
}

/// V float32 values rounded to bf16 (nearest even, quiet NaNs) at `at`.
template<int V>
__device__ inline void StoreB(Bf16* at, const Lanes<V>& in) {
  if constexpr (V == 4)
    *reinterpret_cast<uint2*>(at) =
        uint2{q8::PackBf16x2(in.v[0], in.v[1]), q8::PackBf16x2(in.v[2], in.v[3])};
  else
    *at = Bf16Bits(in.v[0]);
}

/// V float32 values at byte `offset` of `buffer`, zero (no access) unless
/// `keep`: a masked buffer load, no branch, so a wave's loads stay in
/// flight together.
template<int V>
__device__ inline Lanes<V> BufferF(__amdgpu_buffer_rsrc_t buffer, std::uint32_t offset,
                                   bool keep) {
  Lanes<V> out;
  if constexpr (V == 4) {
    const float4 f = __builtin_bit_cast(float4, q8::BufferLoad16(buffer, offset, keep));
    out.v[0] = f.x;
    out.v[1] = f.y;
    out.v[2] = f.z;
    out.v[3] = f.w;
  } else {
    out.v[0] = __builtin_bit_cast(float, q8::BufferLoad4(buffer, offset, keep));
  }
  return out;
}

/// V bf16 values at byte `offset` of `buffer` as float32, zero unless
/// `keep`.
template<int V>
__device__ inline Lanes<V> BufferB(__amdgpu_buffer_rsrc_t buffer, std::uint32_t offset,
                                   bool keep) {
  Lanes<V> out;
  const int at = static_cast<int>(keep ? offset : q8::kPastBuffer);
  if constexpr (V == 4) {
    const auto b = __builtin_amdgcn_raw_buffer_load_b64(buffer, at, 0, 0);
    out.v[0] = q8::Bf16Lo(b[0]);
    out.v[1] = q8::Bf16Hi(b[0]);
    out.v[2] = q8::Bf16Lo(b[1]);
    out.v[3] = q8::Bf16Hi(b[1]);
  } else {
    out.v[0] = q8::Bf16Lo(__builtin_amdgcn_raw_buffer_load_b16(buffer, at, 0, 0));
  }
  return out;
}

bool Aligned(const void* pointer, std::size_t bytes) {
  return reinterpret_cast<std::uintptr_t>(pointer) % bytes == 0;
}

/// Whether float32 arrays (16 bytes) and bf16 arrays (8 bytes) allow V = 4.
bool Quads(std::initializer_list<const float*> floats, std::initializer_list<const Bf16*> halves,
           std::size_t width) {
  if (width % 4 != 0)
    return false;
  for (const float* f : floats)
    if (f != nullptr && !Aligned(f, 16))
      return false;
  for (const Bf16* h : halves)
    if (h != nullptr && !Aligned(h, 8))
      return false;
  return true;
}

// ---- RMSNorm ----------------------------------------------------------------

constexpr int kNormWaves = 4;  // rows per workgroup, one per wave

/// One row per wave. Lane l reads accesses l, l + 64, ... of the row (V
/// values each) and keeps the first kHeld of them, with their norm weights,
/// in registers for the second pass (rows up to 2048 values; longer rows
/// read the rest again). The held accesses are masked buffer loads issued
/// together, so the row arrives in one memory round trip.
/// The lanes' sums of squares meet by a wave butterfly; the output is
/// bf16((x * inv) * gamma) with inv = rsqrt(mean(x^2) + eps), the
/// reference's arithmetic (kernels/generator_kernels.hip:91-108), and its
/// float32 value when asked for.
template<int V>
__global__ __launch_bounds__(kNormWaves * kWave) void WaveNormKernel(
    const float* input, const Bf16* weight, Bf16* output, float* output_f32, int rows,
    int width, float epsilon) {
  constexpr int kHeld = 32 / V;
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  // One row per wave: readfirstlane puts the row (and the buffer made from
  // it) in scalar registers, which buffer loads need.
  const int row = __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x) * kNormWaves +
                                                 static_cast<int>(threadIdx.x) / kWave);
  if (row >= rows)
    return;
  const std::size_t base = static_cast<std::size_t>(row) * width;
  const int accesses = width / V;
  const __amdgpu_buffer_rsrc_t row_buffer =
      q8::BufferOf(input + base, 4U * static_cast<std::uint32_t>(width));
  const __amdgpu_buffer_rsrc_t gamma_buffer =
      q8::BufferOf(weight, 2U * static_cast<std::uint32_t>(width));
  Lanes<V> held[kHeld];
  Lanes<V> held_gamma[kHeld];
#pragma unroll
  for (int j = 0; j < kHeld; ++j) {
    const int c = lane + kWave * j;
    held[j] = BufferF<V>(row_buffer, 4U * V * static_cast<std::uint32_t>(c), c < accesses);
  }
#pragma unroll
  for (int j = 0; j < kHeld; ++j) {
    const int c = lane + kWave * j;
    held_gamma[j] =
        BufferB<V>(gamma_buffer, 2U * V * static_cast<std::uint32_t>(c), c < accesses);
  }
  float squares = 0.0F;
#pragma unroll
  for (int j = 0; j < kHeld; ++j)
#pragma unroll
    for (int i = 0; i < V; ++i)
      squares += held[j].v[i] * held[j].v[i];
  for (int c = lane + kWave * kHeld; c < accesses; c += kWave) {
    const Lanes<V> x = LoadF<V>(input + base + V * c);
#pragma unroll
    for (int i = 0; i < V; ++i)
      squares += x.v[i] * x.v[i];
  }
  const float inverse = rsqrtf(WaveSum(squares) / static_cast<float>(width) + epsilon);
  const auto emit = [&](int c, const Lanes<V>& x, const Lanes<V>& gamma) {
    Lanes<V> y;
#pragma unroll
    for (int i = 0; i < V; ++i)
      y.v[i] = x.v[i] * inverse * gamma.v[i];
    StoreB<V>(output + base + V * c, y);
    if (output_f32 != nullptr)
      StoreF<V>(output_f32 + base + V * c, y);
  };
#pragma unroll
  for (int j = 0; j < kHeld; ++j) {
    const int c = lane + kWave * j;
    if (c < accesses)
      emit(c, held[j], held_gamma[j]);
  }
  for (int c = lane + kWave * kHeld; c < accesses; c += kWave)
    emit(c, LoadF<V>(input + base + V * c), LoadB<V>(weight + V * c));
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

// ---- elementwise -------------------------------------------------------------
//
// Grid-stride loops over V-value accesses (the grid is sized for one access
// per thread and capped).

__device__ inline std::size_t FirstIndex() {
  return static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
}
__device__ inline std::size_t Stride() {
  return static_cast<std::size_t>(gridDim.x) * blockDim.x;
}

/// bf16(silu(gate) * up) over rows of [gate | up] (each `width` wide), the
/// reference's SwiGLU (kernels/generator_kernels.hip:243-254).
template<int V>
__global__ __launch_bounds__(kThreads) void GatedKernel(const float* gate_up, Bf16* output,
                                                        std::size_t rows, std::size_t width) {
  const std::size_t per_row = width / V;
  for (std::size_t e = FirstIndex(); e < rows * per_row; e += Stride()) {
    const std::size_t row = e / per_row;
    const std::size_t column = V * (e % per_row);
    const Lanes<V> gate = LoadF<V>(gate_up + 2 * width * row + column);
    const Lanes<V> up = LoadF<V>(gate_up + 2 * width * row + width + column);
    Lanes<V> y;
#pragma unroll
    for (int i = 0; i < V; ++i)
      y.v[i] = Silu(gate.v[i]) * up.v[i];
    StoreB<V>(output + width * row + column, y);
  }
}

/// data[r][c] += f32(bias[c]) (kernels/generator_kernels.hip:256-262).
template<int V>
__global__ __launch_bounds__(kThreads) void BiasKernel(float* data, const Bf16* bias,
                                                       std::size_t rows, std::size_t width) {
  const std::size_t per_row = width / V;
  for (std::size_t e = FirstIndex(); e < rows * per_row; e += Stride()) {
    const std::size_t column = V * (e % per_row);
    Lanes<V> x = LoadF<V>(data + V * e);
    const Lanes<V> b = LoadB<V>(bias + column);
#pragma unroll
    for (int i = 0; i < V; ++i)
      x.v[i] += b.v[i];
    StoreF<V>(data + V * e, x);
  }
}

/// bf16(x) or bf16(silu(x)) (kernels/generator_kernels.hip:264-274).
template<int V>
__global__ __launch_bounds__(kThreads) void RoundKernel(const float* input, Bf16* output,
                                                        std::size_t count, int silu) {
  for (std::size_t e = FirstIndex(); e < count / V; e += Stride()) {
    Lanes<V> x = LoadF<V>(input + V * e);
    if (silu) {
#pragma unroll
      for (int i = 0; i < V; ++i)
        x.v[i] = Silu(x.v[i]);
    }
    StoreB<V>(output + V * e, x);
  }
}

/// Row copies: output row blockIdx.y <- `source(row)`, V values per access.
/// Gather: the source row is indices[row] of `input`
/// (kernels/generator_kernels.hip:82-89).
template<int V>
__global__ __launch_bounds__(kThreads) void GatherKernel(const float* input,
                                                         const std::int32_t* indices,
                                                         float* output, int width) {
  const int row = static_cast<int>(blockIdx.y);
  const float* from = input + static_cast<std::size_t>(indices[row]) * width;
  float* to = output + static_cast<std::size_t>(row) * width;
  for (int c = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x); c < width / V;
       c += static_cast<int>(gridDim.x * blockDim.x))
    StoreF<V>(to + V * c, LoadF<V>(from + V * c));
}

/// The DiT input rows of both branches (generator.cpp:111-121): each output
/// row of [2][3 + 2 patch][width] picks its source once (mu halves for the
/// conditional branch, zeros for the unconditional one, then the time
/// vector, the condition rows and the projected x rows, the layout of
/// kernels/generator_kernels.hip:320-340) and its threads copy V values
/// per access.
template<int V>
__global__ __launch_bounds__(kThreads) void InputRowsKernel(const float* mu, const float* time,
                                                            const float* cond, const float* x,
                                                            float* output, int patch,
                                                            int width) {
  const int length = 3 + 2 * patch;
  const int branch = static_cast<int>(blockIdx.y) / length;
  const int row = static_cast<int>(blockIdx.y) % length;
  const float* from = nullptr;  // null: zeros
  if (row < 2)
    from = branch == 0 ? mu + static_cast<std::size_t>(row) * width : nullptr;
  else if (row == 2)
    from = time;
  else if (row < 3 + patch)
    from = cond + static_cast<std::size_t>(row - 3) * width;
  else
    from = x + static_cast<std::size_t>(row - 3 - patch) * width;
  float* to = output + static_cast<std::size_t>(blockIdx.y) * width;
  for (int c = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x); c < width / V;
       c += static_cast<int>(gridDim.x * blockDim.x))
    StoreF<V>(to + V * c, from != nullptr ? LoadF<V>(from + V * c) : Lanes<V>{});
}

/// The guided Euler step over one velocity pair (conditional c, then
/// unconditional u, `count` values each), in one workgroup:
/// x -= dt (u s + cfg (c - u s)), with s = <c, u> / (|u|^2 + 1e-8) under
/// CFG-Zero* and s = 1 otherwise (kernels/generator_kernels.hip:342-360).
/// Both sums are carried together: lane partials, a wave butterfly each,
/// then the waves' pairs added in wave order from LDS.
template<int V>
__global__ __launch_bounds__(kThreads) void EulerKernel(const float* velocity, float* x,
                                                        int count, float cfg, float dt,
                                                        int zero_star) {
  __shared__ float2 waves[kThreads / kWave];
  const float* c = velocity;
  const float* u = velocity + count;
  const int accesses = count / V;
  float s = 1.0F;
  if (zero_star) {
    float dot = 0.0F;
    float norm = 0.0F;
    for (int e = static_cast<int>(threadIdx.x); e < accesses; e += kThreads) {
      const Lanes<V> cv = LoadF<V>(c + V * e);
      const Lanes<V> uv = LoadF<V>(u + V * e);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        dot += cv.v[i] * uv.v[i];
        norm += uv.v[i] * uv.v[i];
      }
    }
    dot = WaveSum(dot);
    norm = WaveSum(norm);
    if (threadIdx.x % kWave == 0)
      waves[threadIdx.x / kWave] = float2{dot, norm};
    __syncthreads();
    float2 total = waves[0];
#pragma unroll
    for (int w = 1; w < kThreads / kWave; ++w) {
      total.x += waves[w].x;
      total.y += waves[w].y;
    }
    s = total.x / (total.y + 1e-8F);
  }
  for (int e = static_cast<int>(threadIdx.x); e < accesses; e += kThreads) {
    const Lanes<V> cv = LoadF<V>(c + V * e);
    const Lanes<V> uv = LoadF<V>(u + V * e);
    Lanes<V> xv = LoadF<V>(x + V * e);
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float guided = uv.v[i] * s + cfg * (cv.v[i] - uv.v[i] * s);
      xv.v[i] -= dt * guided;
    }
    StoreF<V>(x + V * e, xv);
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
  const dim3 grid(static_cast<unsigned>((rows + kNormWaves - 1) / kNormWaves));
  if (Quads({input, output_f32}, {weight, output}, width))
    WaveNormKernel<4><<<grid, kNormWaves * kWave, 0, stream>>>(
        input, weight, output, output_f32, static_cast<int>(rows), static_cast<int>(width),
        epsilon);
  else
    WaveNormKernel<1><<<grid, kNormWaves * kWave, 0, stream>>>(
        input, weight, output, output_f32, static_cast<int>(rows), static_cast<int>(width),
        epsilon);
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
  if (Quads({gate_up}, {output}, width))
    GatedKernel<4><<<Grid(rows * width / 4), kThreads, 0, stream>>>(gate_up, output, rows, width);
  else
    GatedKernel<1><<<Grid(rows * width), kThreads, 0, stream>>>(gate_up, output, rows, width);
}

// kernels/generator_kernels.hip:256-262
void AddBias(float* data, const Bf16* bias, std::size_t rows,
             std::size_t width, hipStream_t stream) {
  if (rows * width == 0)
    return;
  if (Quads({data}, {bias}, width))
    BiasKernel<4><<<Grid(rows * width / 4), kThreads, 0, stream>>>(data, bias, rows, width);
  else
    BiasKernel<1><<<Grid(rows * width), kThreads, 0, stream>>>(data, bias, rows, width);
}

// kernels/generator_kernels.hip:264-274
void ToBf16(const float* input, Bf16* output, std::size_t count, bool silu,
            hipStream_t stream) {
  if (count == 0)
    return;
  if (Quads({input}, {output}, count))
    RoundKernel<4><<<Grid(count / 4), kThreads, 0, stream>>>(input, output, count, silu ? 1 : 0);
  else
    RoundKernel<1><<<Grid(count), kThreads, 0, stream>>>(input, output, count, silu ? 1 : 0);
}

// kernels/generator_kernels.hip:82-89
void GatherRows(const float* input, const std::int32_t* indices,
                float* output, std::size_t rows, std::size_t width,
                hipStream_t stream) {
  if (rows == 0 || width == 0)
    return;
  const bool quads = Quads({input, output}, {}, width);
  const dim3 grid(RowBlocks(quads ? width / 4 : width), static_cast<unsigned>(rows));
  if (quads)
    GatherKernel<4><<<grid, kThreads, 0, stream>>>(input, indices, output,
                                                   static_cast<int>(width));
  else
    GatherKernel<1><<<grid, kThreads, 0, stream>>>(input, indices, output,
                                                   static_cast<int>(width));
}

// kernels/generator_kernels.hip:320-340
void AssembleDit(const float* mu, const float* time, const float* cond,
                 const float* x, float* output, std::size_t patch,
                 std::size_t width, hipStream_t stream) {
  if (width == 0)
    return;
  const bool quads = Quads({mu, time, cond, x, output}, {}, width);
  const dim3 grid(RowBlocks(quads ? width / 4 : width),
                  static_cast<unsigned>(2 * (3 + 2 * patch)));
  if (quads)
    InputRowsKernel<4><<<grid, kThreads, 0, stream>>>(mu, time, cond, x, output,
                                                      static_cast<int>(patch),
                                                      static_cast<int>(width));
  else
    InputRowsKernel<1><<<grid, kThreads, 0, stream>>>(mu, time, cond, x, output,
                                                      static_cast<int>(patch),
                                                      static_cast<int>(width));
}

// kernels/generator_kernels.hip:342-360
void GuidedEuler(const float* velocity, float* x, std::size_t count, float cfg,
                 float dt, bool zero_star, hipStream_t stream) {
  if (count == 0)
    return;
  if (Quads({velocity, velocity + count, x}, {}, count))
    EulerKernel<4><<<1, kThreads, 0, stream>>>(velocity, x, static_cast<int>(count), cfg, dt,
                                               zero_star ? 1 : 0);
  else
    EulerKernel<1><<<1, kThreads, 0, stream>>>(velocity, x, static_cast<int>(count), cfg, dt,
                                               zero_star ? 1 : 0);
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
