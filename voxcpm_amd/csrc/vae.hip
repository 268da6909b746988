// AudioVAE V2's causal decoder on one stream, float32, time-major [t][c]:
// the consumer of each patch's latents (vae.cpp:415-481). Chunk by chunk
// with every causal convolution's history carried in a state buffer, which
// equals decoding at once.
//
// Per chunk: the latents' depthwise and pointwise input convolutions, then
// per decoder block the rate-conditioned Snake, the causal transposed
// convolution as ONE product over [x(t) | x(t-1)] (the two taps' weights
// side by side, K = 2 in), and three residual units (Snake, dilated
// depthwise conv fused with the second Snake, pointwise product added into
// the stream), then Snake and the 7-tap convolution to mono with tanh.
// Over at most 256 channels (and for the latents' input convolutions) the
// depthwise convolution and its Snake are made in the pointwise product's
// operand loads, staged through LDS, and the units' windows alternate
// between two buffers; wider units keep a depthwise launch.
// Each product's epilogue applies its bias and makes its consumer's input
// (a residual unit's window: bias, Snake, history; a block's input; the
// output window); each state is filled by the kernel that first reads it
// and refreshed by a later kernel that does not, so no copies remain. The
// products (the reference calls hipblasSgemm) take float32 MFMA kernels:
// 16-column, 32-row tiles that read the weights in place, or, where those
// tiles would re-read over 32 MiB of activations between them, 32 x 32
// tiles staged through LDS. Up to 16 latent frames per chunk the launches
// replay as one HIP graph.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <vector>

#include "common.hpp"
#include "q8_tile.hpp"
#include "voxcpm_amd.h"

namespace {

using vx::kWave;

constexpr int kThreads = 256;
constexpr int kTaps = 7;
constexpr int kDilations[3] = {1, 3, 9};
constexpr std::size_t kMaxGraphFrames = 16;
// Output samples per decode call: a product's row blocks of 32 rows are
// grid rows, at most 65535 of them.
constexpr std::size_t kMaxSamples = std::size_t{65535} * 32;

dim3 Blocks(std::size_t count) {
  return dim3(static_cast<unsigned>((count + kThreads - 1) / kThreads));
}

// One-wave workgroups for the per-element launches between the products:
// spread over more compute units they end sooner (a patch's six depthwise
// launches 1.0 us faster than with 256 threads, 2.1 us slower with 1024).
constexpr int kWaveThreads = kWave;
dim3 WaveBlocks(std::size_t count) {
  return dim3(static_cast<unsigned>((count + kWaveThreads - 1) / kWaveThreads));
}

/// A channel's 1 / (a + 1e-9) in Snake.
__device__ inline float SnakeScale(float a) { return 1.0F / (a + 1e-9F); }
/// Snake(y) = y + sin^2(a y) / (a + 1e-9), `inverse` the channel's
/// SnakeScale(a). The sine is the hardware's (v_sin_f32 takes turns:
/// sin(2 pi r)) of a y in turns reduced to [-1/2, 1/2]: the decoder
/// evaluates Snake on every element of every unit and block input, and the
/// library sine's range reduction and polynomial made the units' products
/// bound by their vector instructions.
__device__ inline float Snake(float y, float a, float inverse) {
  const float turns = a * y * 0.159154943091895336F;  // 1 / (2 pi)
  const float s = __builtin_amdgcn_sinf(turns - rintf(turns));
  return y + inverse * (s * s);
}
__device__ inline float Snake(float y, float a) { return Snake(y, a, SnakeScale(a)); }

/// Up to N copies (to[e] = from[e], e < count) spread over every thread of
/// a grid: each thread's first element is loaded by Load() beside the
/// kernel's first loads and stored by Store() at its end, so that no load
/// of the kernel waits behind a copy's round trip; elements past the
/// grid's threads go in a loop after them.
template<int N>
struct SideCopies {
  float* to[N] = {};
  const float* from[N] = {};
  int count[N] = {};
  float first[N] = {};
  int flat = 0;
  int threads = 0;
  __device__ SideCopies()
      : flat(static_cast<int>((blockIdx.y * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x)),
        threads(static_cast<int>(gridDim.x * gridDim.y * blockDim.x)) {}
  __device__ void Add(int i, float* into, const float* source, int n) {
    to[i] = into;
    from[i] = source;
    count[i] = n;
  }
  __device__ void Load() {
#pragma unroll
    for (int i = 0; i < N; ++i)
      first[i] = __builtin_bit_cast(
          float, vx::q8::BufferLoad4(
                     vx::q8::BufferOf(from[i], 4U * static_cast<std::uint32_t>(count[i])),
                     4U * static_cast<std::uint32_t>(flat), flat < count[i]));
  }
  __device__ void Store() const {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (flat < count[i])
        to[i][flat] = first[i];
      for (int e = flat + threads; e < count[i]; e += threads)
        to[i][e] = from[i][e];
    }
  }
};

/// p[0 .. count) = 0.
__global__ void ZeroKernel(float* p, std::size_t count) {
  const std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < count)
    p[i] = 0.0F;
}

/// work = [state (kTaps - 1 rows) | latents (t rows)] of `c` channels.
__global__ void StageKernel(const float* state, const float* latents, float* work,
                            std::size_t t, std::size_t c) {
  const std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const std::size_t head = (kTaps - 1) * c;
  if (i < head)
    work[i] = state[i];
  else if (i < head + t * c)
    work[i] = latents[i - head];
}

/// out[f][c] = b[c] + sum_j w[c][j] work[f + j d][c] (work holds 6 d rows
/// of history first), optionally through Snake(alpha); also state =
/// work's last 6 d rows (this kernel never reads the state).
__global__ void DepthwiseKernel(const float* work, const float* w, const float* b,
                                const float* alpha, float* out, float* state, std::size_t t,
                                std::size_t c, int d, const float* copy_from = nullptr,
                                float* copy_to = nullptr, std::size_t copy_count = 0) {
  const std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const std::size_t rows = static_cast<std::size_t>(kTaps - 1) * d;
  // The state refresh and a refresh for a kernel before this one (the
  // block input's state), loaded beside the taps.
  SideCopies<2> copies;
  copies.Add(0, state, work + t * c, static_cast<int>(rows * c));
  copies.Add(1, copy_to, copy_from, static_cast<int>(copy_count));
  copies.Load();
  if (i < t * c) {
    const std::size_t f = i / c;
    const std::size_t ch = i % c;
    float sum = b[ch];
#pragma unroll
    for (int j = 0; j < kTaps; ++j)
      sum += w[ch * kTaps + j] * work[(f + static_cast<std::size_t>(j) * d) * c + ch];
    out[i] = alpha != nullptr ? Snake(sum, alpha[ch]) : sum;
  }
  copies.Store();
}

/// samples[f] = tanh(b + sum_c sum_j w[c][j] work[f + j][c]) with `lanes`
/// lanes per frame (a power of two up to 64, at least c / 4 where it can
/// be): lane q takes channel quads q, q + lanes, .., each with one 16-byte
/// load per tap and its four channels' 28 taps as seven 16-byte loads, and
/// the frame's lanes add their sums by butterfly. Also state = work's last
/// 6 rows (this kernel never reads the state) and copy_to = copy_from
/// (copy_count floats: the latents' history, which the first product of
/// the chunk read). c a multiple of 4.
__global__ void ToMonoKernel(const float* work, const float* w, float b, float* samples,
                             float* state, std::size_t t, std::size_t c, int lanes,
                             const float* copy_from, float* copy_to, int copy_count) {
  const std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  SideCopies<2> copies;  // the state refreshes, loaded beside the window
  copies.Add(0, state, work + t * c, static_cast<int>((kTaps - 1) * c));
  copies.Add(1, copy_to, copy_from, copy_count);
  copies.Load();
  const std::size_t f = i / static_cast<std::size_t>(lanes);
  const int q = static_cast<int>(i % static_cast<std::size_t>(lanes));
  const int quads = static_cast<int>(c / 4);
  float sum = 0.0F;
  if (f < t)
    for (int quad = q; quad < quads; quad += lanes) {
      // Channel 4 quad + s's taps are taps[7 s .. 7 s + 6].
      const float4* packed =
          reinterpret_cast<const float4*>(w + static_cast<std::size_t>(quad) * 4 * kTaps);
      float taps[4 * kTaps];
#pragma unroll
      for (int e = 0; e < kTaps; ++e) {
        const float4 v = packed[e];
        taps[4 * e] = v.x;
        taps[4 * e + 1] = v.y;
        taps[4 * e + 2] = v.z;
        taps[4 * e + 3] = v.w;
      }
      float4 rows[kTaps];
#pragma unroll
      for (int j = 0; j < kTaps; ++j)
        rows[j] = *reinterpret_cast<const float4*>(work + (f + j) * c + 4 * quad);
#pragma unroll
      for (int j = 0; j < kTaps; ++j) {
        sum += taps[j] * rows[j].x;
        sum += taps[kTaps + j] * rows[j].y;
        sum += taps[2 * kTaps + j] * rows[j].z;
        sum += taps[3 * kTaps + j] * rows[j].w;
      }
    }
  for (int offset = lanes / 2; offset > 0; offset /= 2)
    sum += __shfl_xor(sum, offset, kWave);
  if (q == 0 && f < t)
    samples[f] = tanhf(sum + b);
  copies.Store();
}

// ---- float32 products of few rows ------------------------------------------
//
// y[t][n] (+)= x[t][k] W[n][k]^T on v_mfma_f32_16x16x4_f32, float32
// throughout. A workgroup owns 16 columns of W and a block of 16 MT rows
// (grid y: the row blocks); its W waves split k in groups of 16. Within a
// group lane L (r = L % 16, g = L / 16) loads W[n0 + r][k0 + 4 g .. + 3]
// and x[16 m + r][k0 + 4 g .. + 3] as float4 and step s of four multiplies
// the k-slots {k0 + 4 g + s}: the weights are read in place, 64 contiguous
// bytes per row per load. The waves' sums meet in LDS in wave order.

constexpr int kF32Waves = 16;  // most waves per workgroup
typedef float F32x4 __attribute__((ext_vector_type(4)));

/// A residual unit's input made in a product's epilogue. y's linear
/// element i is (frame i / channels, channel i % channels), also for a
/// transposed convolution's [t][stride channels] output: v = y[i] +
/// bias[channel], y[i] = v, window[head + i] = Snake(v, alpha[channel]), and
/// window[0 .. head) = state (copied by the first row block's workgroups).
/// Unused when window is null.
///
/// With `scale` set it makes a decoder block's input instead:
/// u = Snake(v scale + shift, alpha) per frame f
/// and channel c of a [frames][channels] output, window = x2 [frames][2
/// channels] with x2[f] = [u(f) | u(f - 1)] and u(-1) = state (copied into
/// x2[0]'s second half by the first row block's workgroups; a later kernel
/// refreshes the state from x2's last frame).
struct UnitWindow {
  const float* bias = nullptr;
  const float* alpha = nullptr;
  float* window = nullptr;
  const float* state = nullptr;
  int head = 0;  // floats of history: 6 d rows of `channels`
  int channels = 1;
  const float* scale = nullptr;
  const float* shift = nullptr;
  int frames = 0;
};

/// A residual unit's pointwise operand made from the unit's window as the
/// product reads it, in place of a depthwise launch and its output buffer
/// (vae.cpp:489-500, vae_kernels.hip:36-51): x[f][c] = Snake(b[c] +
/// sum_j w[c][j] win[f + j d][c], alpha[c]) over the window [6 d history
/// rows | t rows], with no Snake when alpha is null. The product's
/// workgroups also refresh the unit's state from the window's last 6 d
/// rows and copy `copy_count` floats (a block input's state refresh),
/// memory that no workgroup of the launch reads.
struct DwOperand {
  const float* weights = nullptr;  // [c][7]
  const float* bias = nullptr;     // [c]
  const float* alpha = nullptr;    // [c], or null
  int dilation = 1;
  float* state = nullptr;          // [6 d][c]
  // When set, the window's first 6 d rows come from here and the rest from
  // x ([t][c]); `state` is then a buffer of its own, which a later kernel
  // copies into head.
  const float* head = nullptr;
  const float* copy_from = nullptr;
  float* copy_to = nullptr;
  int copy_count = 0;
};

/// Floats of dynamic LDS a fused unit operand takes: the tap table [10][k]
/// (seven taps, bias, alpha, Snake's 1 / (alpha + 1e-9)) and the operand
/// rows [16 MT][k + 4].
constexpr std::size_t DwLdsFloats(std::size_t k, int mt) {
  return 10 * k + static_cast<std::size_t>(16 * mt) * (k + 4);
}
constexpr std::size_t kDwLdsBytes = 60 * 1024;  // under the default 64 KiB

/// With kDw the operand is made from a window (DwOperand) into LDS before
/// the products; k then takes one pass of KA groups per wave.
template<int MT, int W, int KA, bool kDw>
__global__ __launch_bounds__(W * kWave) void F32SkinnyKernel(
    const float* x, const float* w, float* y, int t, int k, int n, int accumulate,
    UnitWindow unit, DwOperand dw) {
  // The waves' partial sums; with kDw they meet in the operand rows' LDS.
  __shared__ float reduce_static[kDw ? 1 : W][MT][4][kWave];
  extern __shared__ float staged[];  // kDw: tap table [10][k], operand rows [16 MT][k + 4]
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int r = lane % 16;
  const int g = lane / 16;
  const int n0 = 16 * static_cast<int>(blockIdx.x);
  const bool column_ok = n0 + r < n;
  // This workgroup's rows: x and y from row0 on, t rows of them.
  const int row0 = 16 * MT * static_cast<int>(blockIdx.y);
  const bool block_input = unit.scale != nullptr;
  const int d = dw.dilation;
  const int halo = kDw ? (kTaps - 1) * d : 0;  // window rows before the first frame
  // Copies beside the product, spread over every workgroup of the grid:
  // the next window's history and, with kDw, the unit's state (the
  // window's last 6 d rows) and a block input's state.
  // (Issuing these copies' loads beside the operands' and storing them at
  // the end, as the depthwise kernel does, measured slower here.)
  const int grid_threads = static_cast<int>(gridDim.x * gridDim.y * blockDim.x);
  const int flat = static_cast<int>((blockIdx.y * gridDim.x + blockIdx.x) * blockDim.x +
                                    threadIdx.x);
  if (unit.window != nullptr) {
    float* head = unit.window + (block_input ? unit.channels : 0);
    for (int e = flat; e < unit.head; e += grid_threads)
      head[e] = unit.state[e];
  }
  const float* x_all = x;  // before this workgroup's row offset
  const int all_rows = t;
  if constexpr (kDw) {
    // The window's last 6 d rows: window element t k + e.
    const int last = t * k;
    for (int e = flat; e < halo * k; e += grid_threads)
      dw.state[e] = dw.head == nullptr ? x[last + e]
                    : last + e < halo * k ? dw.head[last + e]
                                          : x[last + e - halo * k];
    for (int e = flat; e < dw.copy_count; e += grid_threads)
      dw.copy_to[e] = dw.copy_from[e];
  }
  float* window = unit.window != nullptr && !block_input
                      ? unit.window + unit.head + static_cast<std::size_t>(row0) * n
                      : nullptr;
  x += static_cast<std::size_t>(row0) * k;
  y += static_cast<std::size_t>(row0) * n;
  t = min(t - row0, 16 * MT);
  // Buffer loads: masked lanes read zero without a branch, so a wave's
  // loads stay in flight together.
  const __amdgpu_buffer_rsrc_t w_buffer =
      vx::q8::BufferOf(w, 4U * static_cast<std::uint32_t>(n) * static_cast<std::uint32_t>(k));
  const __amdgpu_buffer_rsrc_t x_buffer = vx::q8::BufferOf(
      x, 4U * static_cast<std::uint32_t>(t + halo) * static_cast<std::uint32_t>(k));
  const std::uint32_t w_at = 4U * static_cast<std::uint32_t>((n0 + r) * k + 4 * g);
  std::uint32_t x_at[MT];
  bool row_ok[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    row_ok[m] = 16 * m + r < t;
    x_at[m] = 4U * static_cast<std::uint32_t>((16 * m + r) * k + 4 * g);
  }
  // Output element e = (m, i, lane): row 16 m + 4 (lane / 16) + i, column
  // n0 + lane % 16; thread j-th element e = threadIdx.x + j W 64. With
  // accumulate, y's current values are loaded here beside the operands, not
  // after the products.
  constexpr int kOut = (MT * 4 + W - 1) / W;
  const __amdgpu_buffer_rsrc_t y_buffer =
      vx::q8::BufferOf(y, 4U * static_cast<std::uint32_t>(t) * static_cast<std::uint32_t>(n));
  const bool windowed = unit.window != nullptr;
  const std::uint32_t channel_bytes = 4U * static_cast<std::uint32_t>(unit.channels);
  const __amdgpu_buffer_rsrc_t bias_buffer =
      vx::q8::BufferOf(unit.bias, windowed && unit.bias != nullptr ? channel_bytes : 0U);
  const __amdgpu_buffer_rsrc_t alpha_buffer =
      vx::q8::BufferOf(unit.alpha, windowed ? channel_bytes : 0U);
  const __amdgpu_buffer_rsrc_t scale_buffer =
      vx::q8::BufferOf(unit.scale, windowed && block_input ? channel_bytes : 0U);
  const __amdgpu_buffer_rsrc_t shift_buffer =
      vx::q8::BufferOf(unit.shift, windowed && block_input ? channel_bytes : 0U);
  int out_row[kOut];
  int out_column[kOut];
  float prior[kOut];
  float bias[kOut];
  float alpha[kOut];
  float scale[kOut];
  float shift[kOut];
  const auto load_epilogue = [&]() {  // beside the operands' loads
#pragma unroll
    for (int j = 0; j < kOut; ++j) {
      const int e = static_cast<int>(threadIdx.x) + j * W * kWave;
      const int l = e % kWave;
      out_row[j] =
          e < MT * 4 * kWave ? 16 * (e / (4 * kWave)) + 4 * (l / 16) + (e / kWave) % 4 : t;
      out_column[j] = n0 + l % 16;
      const bool live = out_row[j] < t && out_column[j] < n;
      prior[j] = __builtin_bit_cast(
          float, vx::q8::BufferLoad4(
                     y_buffer, 4U * static_cast<std::uint32_t>(out_row[j] * n + out_column[j]),
                     live && accumulate != 0));
      const std::uint32_t at = 4U * static_cast<std::uint32_t>(out_column[j] % unit.channels);
      bias[j] = __builtin_bit_cast(
          float, vx::q8::BufferLoad4(bias_buffer, at, live && windowed && unit.bias != nullptr));
      alpha[j] =
          __builtin_bit_cast(float, vx::q8::BufferLoad4(alpha_buffer, at, live && windowed));
      const bool block_live = live && windowed && block_input;
      scale[j] = __builtin_bit_cast(float, vx::q8::BufferLoad4(scale_buffer, at, block_live));
      shift[j] = __builtin_bit_cast(float, vx::q8::BufferLoad4(shift_buffer, at, block_live));
    }
  };
  load_epilogue();
  F32x4 acc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m)
    acc[m] = F32x4{0.0F, 0.0F, 0.0F, 0.0F};
  const int groups = k / 16;
  const auto multiply = [&](const float4& wv, const float4 (&xv)[MT]) {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      acc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[m].x, wv.x, acc[m], 0, 0, 0);
      acc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[m].y, wv.y, acc[m], 0, 0, 0);
      acc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[m].z, wv.z, acc[m], 0, 0, 0);
      acc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[m].w, wv.w, acc[m], 0, 0, 0);
    }
  };
  if constexpr (kDw) {
    // One pass: the launch gives every wave at most KA groups of k. The
    // weights' loads go out first, then the window's, then the operand is
    // made into LDS while they arrive.
    float4 wv[KA];
#pragma unroll
    for (int a = 0; a < KA; ++a) {
      const int group = wave + a * W;
      wv[a] = __builtin_bit_cast(
          float4, vx::q8::BufferLoad16(w_buffer, w_at + 64U * static_cast<std::uint32_t>(group),
                                       group < groups && column_ok));
    }
    // [10][k]: w_j for j < 7, then bias, alpha and Snake's 1 / (alpha + 1e-9)
    float* taps = staged;
    float* rows = staged + 10 * k;      // [16 MT][k + 4]
    const int stride = k + 4;
    const int tid = static_cast<int>(threadIdx.x);
    constexpr int kThreadsW = W * kWave;
    // Items: a quad of channels and up to four operand rows d apart
    // (residue class rho of the rows mod d, run it), which read ten window
    // rows d apart: (4 + 6) loads for four rows instead of 28. One item per
    // thread in flight; the window's loads of the first go out before the
    // tap table's barrier.
    const int quads = k / 4;
    const int runs = (16 * MT + 4 * d - 1) / (4 * d);
    const int items = quads * d * runs;
    const __amdgpu_buffer_rsrc_t head_buffer = vx::q8::BufferOf(
        dw.head, dw.head != nullptr ? 4U * static_cast<std::uint32_t>(halo * k) : 0U);
    const __amdgpu_buffer_rsrc_t x_all_buffer = vx::q8::BufferOf(
        x_all, dw.head != nullptr ? 4U * static_cast<std::uint32_t>(all_rows * k) : 0U);
    float4 win[10];
    int item_q = 0;
    int item_row = 0;  // rho + 4 it d
    const auto load_item = [&](int item) {
      const bool live = item < items;
      item_q = live ? item % quads : 0;
      const int task = live ? item / quads : 0;
      item_row = live ? task % d + 4 * (task / d) * d : 16 * MT;
      if (dw.head == nullptr) {
#pragma unroll
        for (int l = 0; l < 10; ++l) {
          const int row = item_row + l * d;
          win[l] = __builtin_bit_cast(
              float4, vx::q8::BufferLoad16(
                          x_buffer, 4U * static_cast<std::uint32_t>(row * k + 4 * item_q),
                          live && row < t + halo));
        }
      } else {
        // Window row w (of the whole window) from the head below 6 d, else
        // row w - 6 d of x: one of the two loads is masked to zero and the
        // row is their sum (a select kept the pair in scratch memory).
#pragma unroll
        for (int l = 0; l < 10; ++l) {
          const int w = row0 + item_row + l * d;
          const float4 from_head = __builtin_bit_cast(
              float4, vx::q8::BufferLoad16(
                          head_buffer, 4U * static_cast<std::uint32_t>(w * k + 4 * item_q),
                          live && w < halo));
          const float4 from_x = __builtin_bit_cast(
              float4,
              vx::q8::BufferLoad16(
                  x_all_buffer, 4U * static_cast<std::uint32_t>((w - halo) * k + 4 * item_q),
                  live && w >= halo && w - halo < all_rows));
          win[l] = float4{from_head.x + from_x.x, from_head.y + from_x.y,
                          from_head.z + from_x.z, from_head.w + from_x.w};
        }
      }
    };
    const auto make_item = [&]() {
      if (item_row >= 16 * MT)
        return;
      const int c = 4 * item_q;
      float4 sum[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sum[i] = *reinterpret_cast<const float4*>(&taps[7 * k + c]);
      // Tap by tap (each row's sum in tap order), one tap's weights live.
#pragma unroll
      for (int j = 0; j < kTaps; ++j) {
        const float4 wj = *reinterpret_cast<const float4*>(&taps[j * k + c]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sum[i].x += wj.x * win[i + j].x;
          sum[i].y += wj.y * win[i + j].y;
          sum[i].z += wj.z * win[i + j].z;
          sum[i].w += wj.w * win[i + j].w;
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = item_row + i * d;
        if (row >= 16 * MT)
          break;
        *reinterpret_cast<float4*>(&rows[row * stride + c]) =
            row < t ? sum[i] : float4{0.0F, 0.0F, 0.0F, 0.0F};
      }
    };
    load_item(tid);
    // The tap table: [c][7] in memory, tap-major in LDS.
    const __amdgpu_buffer_rsrc_t taps_buffer =
        vx::q8::BufferOf(dw.weights, 4U * kTaps * static_cast<std::uint32_t>(k));
    const __amdgpu_buffer_rsrc_t dw_bias_buffer =
        vx::q8::BufferOf(dw.bias, 4U * static_cast<std::uint32_t>(k));
    const __amdgpu_buffer_rsrc_t dw_alpha_buffer =
        vx::q8::BufferOf(dw.alpha, dw.alpha != nullptr ? 4U * static_cast<std::uint32_t>(k) : 0U);
    for (int e = tid; e < kTaps * quads; e += kThreadsW) {
      const float4 v = __builtin_bit_cast(
          float4, vx::q8::BufferLoad16(taps_buffer, 16U * static_cast<std::uint32_t>(e), true));
      const float parts[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int flat_tap = 4 * e + s;  // channel flat_tap / 7, tap flat_tap % 7
        taps[(flat_tap % kTaps) * k + flat_tap / kTaps] = parts[s];
      }
    }
    for (int e = tid; e < quads; e += kThreadsW) {
      const std::uint32_t at = 16U * static_cast<std::uint32_t>(e);
      *reinterpret_cast<uint4*>(&taps[7 * k + 4 * e]) =
          vx::q8::BufferLoad16(dw_bias_buffer, at, true);
      const float4 a = __builtin_bit_cast(
          float4, vx::q8::BufferLoad16(dw_alpha_buffer, at, dw.alpha != nullptr));
      *reinterpret_cast<float4*>(&taps[8 * k + 4 * e]) = a;
      *reinterpret_cast<float4*>(&taps[9 * k + 4 * e]) =
          float4{SnakeScale(a.x), SnakeScale(a.y), SnakeScale(a.z), SnakeScale(a.w)};
    }
    __syncthreads();
    make_item();
    for (int item = tid + kThreadsW; item < items; item += kThreadsW) {
      load_item(item);
      make_item();
    }
    __syncthreads();
#pragma unroll
    for (int a = 0; a < KA; ++a) {
      const int group = wave + a * W;
      if (group >= groups)
        break;
      // The second Snake as the operand is read: each element of the rows
      // is read by one lane of one wave. Rows past t hold zero, and
      // Snake(0) = 0.
      const int c = 16 * group + 4 * g;
      const float4 alpha4 = *reinterpret_cast<const float4*>(&taps[8 * k + c]);
      const float4 inverse4 = *reinterpret_cast<const float4*>(&taps[9 * k + c]);
      float4 xv[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        xv[m] = *reinterpret_cast<const float4*>(&rows[(16 * m + r) * stride + c]);
        if (dw.alpha != nullptr)
          xv[m] = float4{Snake(xv[m].x, alpha4.x, inverse4.x),
                         Snake(xv[m].y, alpha4.y, inverse4.y),
                         Snake(xv[m].z, alpha4.z, inverse4.z),
                         Snake(xv[m].w, alpha4.w, inverse4.w)};
      }
      multiply(wv[a], xv);
    }
    __syncthreads();  // the operand rows become the partial sums' LDS
  } else {
    for (int base = wave; base < groups; base += W * KA) {
      float4 wv[KA];
      float4 xv[KA][MT];
#pragma unroll
      for (int a = 0; a < KA; ++a) {
        const int group = base + a * W;
        const bool ok = group < groups;
        wv[a] = __builtin_bit_cast(
            float4, vx::q8::BufferLoad16(w_buffer, w_at + 64U * static_cast<std::uint32_t>(group),
                                         ok && column_ok));
#pragma unroll
        for (int m = 0; m < MT; ++m)
          xv[a][m] = __builtin_bit_cast(
              float4, vx::q8::BufferLoad16(x_buffer,
                                           x_at[m] + 64U * static_cast<std::uint32_t>(group),
                                           ok && row_ok[m]));
      }
#pragma unroll
      for (int a = 0; a < KA; ++a)
        multiply(wv[a], xv[a]);
    }
  }
  float* reduce = kDw ? staged : &reduce_static[0][0][0][0];  // [W][MT][4][64]
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      reduce[((wave * MT + m) * 4 + i) * kWave + lane] = acc[m][i];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kOut; ++j) {
    if (out_row[j] >= t || out_column[j] >= n)
      continue;
    const int e = static_cast<int>(threadIdx.x) + j * W * kWave;
    const int m = e / (4 * kWave);
    const int i = (e / kWave) % 4;
    const int l = e % kWave;
    float total = reduce[((0 * MT + m) * 4 + i) * kWave + l];
#pragma unroll
    for (int v = 1; v < W; ++v)
      total += reduce[((v * MT + m) * 4 + i) * kWave + l];
    float v = accumulate != 0 ? prior[j] + total : total;
    const std::size_t at = static_cast<std::size_t>(out_row[j]) * n + out_column[j];
    if (windowed) {
      if (unit.bias != nullptr)
        v += bias[j];
      if (block_input) {
        // The output is [frames][channels]: frame row0 + row, channel column.
        const float u = Snake(v * scale[j] + shift[j], alpha[j]);
        const int frame = row0 + out_row[j];
        const std::size_t c = static_cast<std::size_t>(unit.channels);
        unit.window[static_cast<std::size_t>(frame) * 2 * c + out_column[j]] = u;
        if (frame + 1 < unit.frames)
          unit.window[static_cast<std::size_t>(frame + 1) * 2 * c + c + out_column[j]] = u;
      } else {
        window[at] = Snake(v, alpha[j]);
      }
    }
    y[at] = v;
  }
}

// ---- float32 products of many rows --------------------------------------------
//
// y[t][n] (+)= x[t][k] W[n][k]^T on v_mfma_f32_16x16x4_f32 over 32 x 32
// output tiles (grid: column tiles x row tiles), for products whose
// column tiles would each re-read many rows of x. Eight waves, two per
// SIMD: wave w owns the 16 x 16 quadrant w % 4 and, of each stage's 64
// columns of k, the half w / 4; the halves' sums meet once, at the end, in
// LDS. Per stage the workgroup's 512 threads bring both 32 x 64 operand
// tiles into LDS with one 16-byte load each (the loads of the four stages
// after it are in flight while one is multiplied; two LDS buffers, one
// barrier per stage); a wave then reads its rows and columns back as 16-byte chunks,
// lane (r = L % 16, g = L / 16) the k-slots 16 j + 4 g .. + 3 of row r,
// and step s of four multiplies slot 16 j + 4 g + s. Rows are 68 floats
// apart in LDS: the 16 rows of a read fall on two passes of the 32 banks.
// The epilogue is F32SkinnyKernel's (bias, unit window or block input).
//
// With a grid of S > 1 along z, workgroup z takes the z-th of S runs of
// k (whole stages) and stores its sums into y + z t n, with no epilogue;
// SplitSumKernel adds the S partial products in split order and applies
// the epilogue.

constexpr int kTileRows = 32;
constexpr int kTileK = 128;
constexpr int kTileStride = kTileK + 4;
constexpr int kTileThreads = 512;
constexpr int kTileDepth = 2;
// k splits of a few-row tile product: two (four measured 0.6 us slower per
// patch, eight 3 us).
constexpr std::size_t kMaxSplits = 2;
constexpr std::size_t kSplitK = 2048;  // least k that splits

__global__ __launch_bounds__(kTileThreads) void F32TileKernel(const float* x, const float* w, float* y,
                                                     int t, int k, int n, int accumulate,
                                                     UnitWindow unit) {
  __shared__ float xs[2][kTileRows][kTileStride];
  __shared__ float ws[2][kTileRows][kTileStride];
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  const int quadrant = wave % 4;
  const int half = wave / 4;      // the wave's half of each stage's k
  const int wm = quadrant / 2;    // the quadrant's 16-row half of the tile
  const int wn = quadrant % 2;    // its 16-column half
  const int r = lane % 16;
  const int g = lane / 16;
  const int n0 = kTileRows * static_cast<int>(blockIdx.x);
  const int row0 = kTileRows * static_cast<int>(blockIdx.y);
  // This workgroup's run of k: all of it, or split z of gridDim.z.
  const int splits = static_cast<int>(gridDim.z);
  const int run = ((k + splits - 1) / splits + kTileK - 1) / kTileK * kTileK;
  const int k_begin = static_cast<int>(blockIdx.z) * run;
  const int k_end = min(k, k_begin + run);
  y += static_cast<std::size_t>(blockIdx.z) * t * n;
  const bool block_input = unit.scale != nullptr;
  if (unit.window != nullptr) {  // spread over every workgroup of the grid
    float* head = unit.window + (block_input ? unit.channels : 0);
    for (int e = static_cast<int>((blockIdx.y * gridDim.x + blockIdx.x) * blockDim.x) + tid;
         e < unit.head; e += static_cast<int>(gridDim.x * gridDim.y * blockDim.x))
      head[e] = unit.state[e];
  }
  const __amdgpu_buffer_rsrc_t w_buffer =
      vx::q8::BufferOf(w, 4U * static_cast<std::uint32_t>(n) * static_cast<std::uint32_t>(k));
  const __amdgpu_buffer_rsrc_t x_buffer =
      vx::q8::BufferOf(x, 4U * static_cast<std::uint32_t>(t) * static_cast<std::uint32_t>(k));
  // Thread tid's 16-byte chunks of each operand tile: chunk q = tid + 512 h
  // is row q / 32, columns 4 (q % 32) .. + 3 of the stage.
  struct StageRegs {
    float4 x[2];
    float4 w[2];
  };
  const auto load_stage = [&](int k0, StageRegs& v) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int q = tid + kTileThreads * h;
      const int row = q / 32;
      const int column = k_begin + k0 + 4 * (q % 32);
      const bool k_ok = column < k_end;
      v.x[h] = __builtin_bit_cast(
          float4, vx::q8::BufferLoad16(
                      x_buffer, 4U * static_cast<std::uint32_t>((row0 + row) * k + column),
                      k_ok && row0 + row < t));
      v.w[h] = __builtin_bit_cast(
          float4, vx::q8::BufferLoad16(
                      w_buffer, 4U * static_cast<std::uint32_t>((n0 + row) * k + column),
                      k_ok && n0 + row < n));
    }
  };
  const auto store_stage = [&](int buffer, const StageRegs& v) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int q = tid + kTileThreads * h;
      *reinterpret_cast<float4*>(&xs[buffer][q / 32][4 * (q % 32)]) = v.x[h];
      *reinterpret_cast<float4*>(&ws[buffer][q / 32][4 * (q % 32)]) = v.w[h];
    }
  };

  // The epilogue's operands, loaded beside the first stage.
  const int out_column = n0 + 16 * wn + r;
  const bool windowed = unit.window != nullptr;
  const std::uint32_t channel_bytes = 4U * static_cast<std::uint32_t>(unit.channels);
  const __amdgpu_buffer_rsrc_t y_buffer =
      vx::q8::BufferOf(y, 4U * static_cast<std::uint32_t>(t) * static_cast<std::uint32_t>(n));
  const __amdgpu_buffer_rsrc_t bias_buffer =
      vx::q8::BufferOf(unit.bias, windowed && unit.bias != nullptr ? channel_bytes : 0U);
  const __amdgpu_buffer_rsrc_t alpha_buffer =
      vx::q8::BufferOf(unit.alpha, windowed ? channel_bytes : 0U);
  const __amdgpu_buffer_rsrc_t scale_buffer =
      vx::q8::BufferOf(unit.scale, windowed && block_input ? channel_bytes : 0U);
  const __amdgpu_buffer_rsrc_t shift_buffer =
      vx::q8::BufferOf(unit.shift, windowed && block_input ? channel_bytes : 0U);
  const bool column_ok = out_column < n;
  const std::uint32_t channel_at =
      4U * static_cast<std::uint32_t>(column_ok ? out_column % unit.channels : 0);
  const float bias = __builtin_bit_cast(
      float, vx::q8::BufferLoad4(bias_buffer, channel_at,
                                 column_ok && windowed && unit.bias != nullptr));
  const float alpha =
      __builtin_bit_cast(float, vx::q8::BufferLoad4(alpha_buffer, channel_at, column_ok && windowed));
  const bool block_live = column_ok && windowed && block_input;
  const float scale =
      __builtin_bit_cast(float, vx::q8::BufferLoad4(scale_buffer, channel_at, block_live));
  const float shift =
      __builtin_bit_cast(float, vx::q8::BufferLoad4(shift_buffer, channel_at, block_live));
  float prior[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = row0 + 16 * wm + 4 * g + i;
    prior[i] = __builtin_bit_cast(
        float, vx::q8::BufferLoad4(y_buffer, 4U * static_cast<std::uint32_t>(row * n + out_column),
                                   row < t && column_ok && accumulate != 0));
  }

  F32x4 acc = F32x4{0.0F, 0.0F, 0.0F, 0.0F};
  const int stages = k_end > k_begin ? (k_end - k_begin + kTileK - 1) / kTileK : 0;
  // kTileDepth stages' loads in flight: a stage's products take far less
  // time than a load's round trip.
  StageRegs regs[kTileDepth];
#pragma unroll
  for (int p = 0; p < kTileDepth; ++p)
    load_stage(p * kTileK, regs[p]);  // stages past k load zeros
  for (int s0 = 0; s0 < stages; s0 += kTileDepth) {
#pragma unroll
    for (int p = 0; p < kTileDepth; ++p) {
      const int s = s0 + p;
      if (s >= stages)
        break;
      const int buffer = s % 2;
      store_stage(buffer, regs[p]);
      __syncthreads();
      if (s + kTileDepth < stages)
        load_stage((s + kTileDepth) * kTileK, regs[p]);
      // The wave's half of the stage: its operand chunks read at once,
      // then the products.
      constexpr int kChunks = kTileK / 32;
      float4 a[kChunks], b[kChunks];
#pragma unroll
      for (int jj = 0; jj < kChunks; ++jj) {
        const int j = kChunks * half + jj;
        a[jj] = *reinterpret_cast<const float4*>(&xs[buffer][16 * wm + r][16 * j + 4 * g]);
        b[jj] = *reinterpret_cast<const float4*>(&ws[buffer][16 * wn + r][16 * j + 4 * g]);
      }
#pragma unroll
      for (int jj = 0; jj < kChunks; ++jj) {
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[jj].x, b[jj].x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[jj].y, b[jj].y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[jj].z, b[jj].z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[jj].w, b[jj].w, acc, 0, 0, 0);
      }
    }
  }
  // The second halves' sums join the first halves' (through the first LDS
  // operand buffer, which the last stage no longer reads once every wave
  // has passed this barrier).
  __syncthreads();
  float* meet = &xs[0][0][0];
  if (half == 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      meet[(quadrant * 4 + i) * kWave + lane] = acc[i];
  }
  __syncthreads();
  if (half == 1 || !column_ok)
    return;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    acc[i] += meet[(quadrant * 4 + i) * kWave + lane];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = row0 + 16 * wm + 4 * g + i;
    if (row >= t)
      continue;
    float v = accumulate != 0 ? prior[i] + acc[i] : acc[i];
    const std::size_t at = static_cast<std::size_t>(row) * n + out_column;
    if (windowed) {
      if (unit.bias != nullptr)
        v += bias;
      if (block_input) {
        // The output is [frames][channels]: frame `row`, channel out_column.
        const float u = Snake(v * scale + shift, alpha);
        const std::size_t c = static_cast<std::size_t>(unit.channels);
        unit.window[static_cast<std::size_t>(row) * 2 * c + out_column] = u;
        if (row + 1 < unit.frames)
          unit.window[static_cast<std::size_t>(row + 1) * 2 * c + c + out_column] = u;
      } else {
        unit.window[static_cast<std::size_t>(unit.head) + at] = Snake(v, alpha);
      }
    }
    y[at] = v;
  }
}

/// W2[(r out + o)][k]: k < in the tap r of input channel k, k >= in the tap
/// r + s of channel k - in, from ConvTranspose1d's [in][out][2 s].
__global__ void RepackUpKernel(const float* up, float* w2, std::size_t in, std::size_t out,
                               std::size_t s) {
  const std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= s * out * 2 * in)
    return;
  const std::size_t row = i / (2 * in);
  const std::size_t k = i % (2 * in);
  const std::size_t r = row / out;
  const std::size_t o = row % out;
  const std::size_t channel = k < in ? k : k - in;
  const std::size_t tap = k < in ? r : r + s;
  w2[i] = up[(channel * out + o) * 2 * s + tap];
}

/// y[i] = sum over s < splits of partials[s][i], s in order, for the t x n
/// output of a product into a residual unit's window, then that epilogue
/// (UnitWindow: bias, y, and Snake into the window after its history,
/// which is copied here too), a thread per element.
__global__ void SplitSumKernel(const float* partials, int splits, float* y, int t, int n,
                               UnitWindow unit) {
  const int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
  for (int e = i; e < unit.head; e += static_cast<int>(gridDim.x * blockDim.x))
    unit.window[e] = unit.state[e];
  if (i >= t * n)
    return;
  const std::size_t count = static_cast<std::size_t>(t) * n;
  float v = partials[i];
  for (int s = 1; s < splits; ++s)
    v += partials[s * count + i];
  const int channel = (i % n) % unit.channels;
  if (unit.bias != nullptr)
    v += unit.bias[channel];
  unit.window[unit.head + i] = Snake(v, unit.alpha[channel]);
  y[i] = v;
}

/// One F32SkinnyKernel launch's grid and arguments.
struct SkinnyLaunch {
  dim3 grid;
  std::size_t lds = 0;  // dynamic LDS bytes: the fused operand's
  hipStream_t stream = nullptr;
  const float* x = nullptr;
  const float* w = nullptr;
  float* y = nullptr;
  int t = 0;
  int k = 0;
  int n = 0;
  int accumulate = 0;
  UnitWindow unit;
  DwOperand dw;
};

/// F32SkinnyKernel<MT, W, KA, fused> for `ka` groups per wave pass, fused
/// when the launch carries a depthwise operand.
template<int MT, int W>
void LaunchSkinny(const SkinnyLaunch& l, int ka) {
  const auto launch = [&](auto kernel) {
    kernel<<<l.grid, W * kWave, l.lds, l.stream>>>(l.x, l.w, l.y, l.t, l.k, l.n, l.accumulate,
                                                   l.unit, l.dw);
  };
  if (l.dw.weights != nullptr) {
    if (ka == 2)
      launch(F32SkinnyKernel<MT, W, 2, true>);
    else
      launch(F32SkinnyKernel<MT, W, 4, true>);
  } else if (ka == 2) {
    launch(F32SkinnyKernel<MT, W, 2, false>);
  } else {
    launch(F32SkinnyKernel<MT, W, 4, false>);
  }
}

template<typename T>
int Allocate(T** pointer, std::size_t count, const char* what) {
  if (hipMalloc(reinterpret_cast<void**>(pointer), std::max<std::size_t>(count, 1) * sizeof(T)) !=
      hipSuccess)
    return vx::Fail(VX_HIP_ERROR, what);
  return VX_OK;
}

struct Block {
  std::size_t in = 0;
  std::size_t out = 0;
  std::size_t stride = 0;
  vx_vae_block w{};
  float* up2 = nullptr;       // [s out][2 in]
  float* state = nullptr;     // [in]: the last frame's Snake output
  float* unit_state[3] = {};  // [6 d][out]
};

struct GraphKey {
  const float* latents = nullptr;
  float* samples = nullptr;
  std::size_t frames = 0;
  hipStream_t stream = nullptr;
  bool operator==(const GraphKey& o) const {
    return latents == o.latents && samples == o.samples && frames == o.frames &&
           stream == o.stream;
  }
};

}  // namespace

struct vx_vae {
  vx_vae_shape shape{};
  vx_vae_weights weights{};
  std::vector<Block> blocks;
  std::size_t out_channels = 0;
  std::size_t hop = 1;
  float* in_state = nullptr;   // [6][latent]
  float* in_state_next = nullptr;  // [6][latent]: the next chunk's, copied in at the end
  float* out_state = nullptr;  // [6][out_channels]
  float* hidden = nullptr;
  float* next = nullptr;
  float* work = nullptr;
  float* scratch = nullptr;
  float* scratch2 = nullptr;
  float* partials = nullptr;  // [kMaxSplits][t][n] of split products
  std::size_t capacity_frames = 0;
  GraphKey graph_key;
  hipGraphExec_t graph = nullptr;
  bool seen = false;  // the key has run once eagerly before its capture

  ~vx_vae() {
    if (graph != nullptr)
      (void)hipGraphExecDestroy(graph);
    for (Block& b : blocks) {
      (void)hipFree(b.up2);
      (void)hipFree(b.state);
      for (float* s : b.unit_state)
        (void)hipFree(s);
    }
    for (void* p : {static_cast<void*>(in_state), static_cast<void*>(in_state_next),
                    static_cast<void*>(out_state),
                    static_cast<void*>(hidden), static_cast<void*>(next),
                    static_cast<void*>(work), static_cast<void*>(scratch),
                    static_cast<void*>(scratch2), static_cast<void*>(partials)})
      (void)hipFree(p);
  }

  /// y[t][n] (+)= x[t][k] W[n][k]^T. F32SkinnyKernel can take it where k
  /// is whole groups of 16 and its workgroups re-read at most 32 MiB of x
  /// between them (one x read per 16 columns): every product of VoxCPM2's
  /// decoder but block 2's transposed convolution (192 rows x 2048 over
  /// 1280 columns), which F32TileKernel tiles in both dimensions (Gemm
  /// also gives the tile kernel the unfused products it fills the compute
  /// units with).
  static bool Skinny(std::size_t t, std::size_t k, std::size_t n) {
    const std::size_t x_reads = t * k * sizeof(float) * ((n + 15) / 16);
    return k % 16 == 0 && n * k * sizeof(float) < (std::size_t{1} << 32) &&
           (t <= 32 || x_reads <= (std::size_t{32} << 20));
  }

  /// A residual unit's depthwise convolution is made in its pointwise
  /// product's operand loads (DwOperand) when the product takes
  /// F32SkinnyKernel over at most 256 channels. Every 16-column workgroup
  /// makes its row block's operand: at 512 channels (32 workgroups per row
  /// block) that measured slower than the separate depthwise launch, at
  /// 32-256 channels faster (one patch of VoxCPM2's decoder 284 -> 268 us
  /// up to 128 channels with the library sine in Snake, 251 -> 249 us
  /// adding 256 with the hardware sine).
  static bool Fusable(std::size_t t, std::size_t k, std::size_t n) {
    return k <= 256 && Skinny(t, k, n) && DwLdsFloats(k, 1) * sizeof(float) <= kDwLdsBytes &&
           (t + (kTaps - 1) * kDilations[2]) * k * sizeof(float) < (std::size_t{1} << 32);
  }

  /// With `unit.window` set, the product's epilogue also makes its
  /// consumer's input. With `dw` (Fusable shapes only), x is a window
  /// [6 d rows | t rows] and the operand is made from it. k a multiple of
  /// 4 (checked at create).
  int Gemm(const float* x, const float* w, float* y, std::size_t t, std::size_t k, std::size_t n,
           bool accumulate, hipStream_t stream, const UnitWindow& unit = UnitWindow{},
           const DwOperand* dw = nullptr) {
    if (dw != nullptr && !Fusable(t, k, n))
      return vx::Fail(VX_UNSUPPORTED, "vx_vae_decode: fused operand shape");
    // Over 32 rows an unfused product whose 32 x 32 tiles fill three
    // quarters of the 256 compute units takes F32TileKernel, which reads x
    // once per 32 columns instead of once per 16: blocks 3-5's transposed
    // convolutions (240 tiles) 9.16 / 6.68 / 5.92 -> 7.68 / 6.34 / 5.60 us,
    // where block 1's units (96 tiles) measured 5.6-5.8 -> 6.2-6.4 us.
    const std::size_t tiles = ((n + kTileRows - 1) / kTileRows) * ((t + kTileRows - 1) / kTileRows);
    const bool tiled = dw == nullptr && t > 32 && tiles >= 192;
    // A product of at most 32 rows into a residual unit's window (no
    // accumulation) whose 16-column workgroups would not fill the compute
    // units, over k of at least kSplitK, splits k over the tile kernel's
    // 32 x 32 tiles instead (each split reading x once per 32 columns), up
    // to kMaxSplits and 384 workgroups, and a second launch adds the
    // splits and applies the epilogue.
    const std::size_t column_tiles16 = (n + 15) / 16;
    std::size_t splits = 1;
    const bool window_only = unit.window != nullptr && unit.scale == nullptr && !accumulate;
    if (dw == nullptr && window_only && t <= 32 && column_tiles16 < 256 && k >= kSplitK)
      while (splits < kMaxSplits && tiles * 2 * splits <= 384 && k / (2 * splits) >= 256)
        splits *= 2;
    if (Skinny(t, k, n) && !tiled && splits == 1) {
      // One 16-row tile per workgroup up to 16 rows, and up to 32 while
      // the tiles still take one workgroup per compute unit (twice the
      // workgroups of 32-row tiles, each with half the operand loads:
      // block 0's units 8.2 -> 6.2-7.2 us; where the second round of
      // workgroups would load more per compute unit than 32-row tiles, as
      // block 1's transposed convolution, 14.0 -> 17.7 us); 32-row tiles
      // beyond.
      const std::size_t column_tiles = (n + 15) / 16;
      int mt = t <= 16 || (t <= 32 && 2 * column_tiles <= 256) ? 1 : 2;
      // A fused operand of at most 32 channels takes 16-row tiles too, while
      // their row blocks fit the grid's rows: block 5's units (32 channels,
      // 7680 rows) 7.1-7.6 -> 6.6-6.8 us, where block 4's (64 channels)
      // measured 6.6-7.8 -> 7.2-8.2 us.
      if (dw != nullptr && ((k <= 32 && (t + 15) / 16 <= 65535) ||
                            DwLdsFloats(k, mt) * sizeof(float) > kDwLdsBytes))
        mt = 1;
      const std::size_t groups = k / 16;
      // At least two groups of k per wave; with a fused operand one group
      // per wave from 4 up to 8 waves, whose threads then make it in about
      // one round and whose workgroups fit two to a compute unit (waves
      // past the groups make operand rows and outputs only: block 5's
      // units, two groups of k, 7.8-8.3 -> 7.1-7.6 us with four waves
      // instead of two; eight measured slower).
      const std::size_t per_wave = dw != nullptr ? 1 : 2;
      int waves = dw != nullptr ? kF32Waves / 2 : kF32Waves;
      const int fewest_waves = dw != nullptr ? 4 : 1;
      while (waves > fewest_waves && groups < per_wave * static_cast<std::size_t>(waves))
        waves /= 2;
      // Groups per wave pass: two where that covers k in one pass.
      const int ka = groups <= 2 * static_cast<std::size_t>(waves) ? 2 : 4;
      if (dw != nullptr && groups > static_cast<std::size_t>(waves) * ka)
        return vx::Fail(VX_UNSUPPORTED, "vx_vae_decode: fused operand over one pass of k");
      // The waves' partial sums reuse the fused operand's LDS.
      const std::size_t lds =
          dw != nullptr ? std::max(DwLdsFloats(k, mt),
                                   static_cast<std::size_t>(waves * mt * 4 * kWave)) *
                              sizeof(float)
                        : 0;
      const dim3 grid(static_cast<unsigned>((n + 15) / 16),
                      static_cast<unsigned>((t + 16 * mt - 1) / (16 * mt)));
      if ((t + 16 * mt - 1) / (16 * mt) > 65535)
        return vx::Fail(VX_UNSUPPORTED, "vx_vae_decode: more row blocks than grid rows");
      const DwOperand none;
      const SkinnyLaunch launch{grid,
                                lds,
                                stream,
                                x,
                                w,
                                y,
                                static_cast<int>(t),
                                static_cast<int>(k),
                                static_cast<int>(n),
                                accumulate ? 1 : 0,
                                unit,
                                dw != nullptr ? *dw : none};
      switch (mt * 100 + waves) {
        case 101: LaunchSkinny<1, 1>(launch, ka); break;
        case 102: LaunchSkinny<1, 2>(launch, ka); break;
        case 104: LaunchSkinny<1, 4>(launch, ka); break;
        case 108: LaunchSkinny<1, 8>(launch, ka); break;
        case 116: LaunchSkinny<1, 16>(launch, ka); break;
        case 201: LaunchSkinny<2, 1>(launch, ka); break;
        case 202: LaunchSkinny<2, 2>(launch, ka); break;
        case 204: LaunchSkinny<2, 4>(launch, ka); break;
        case 208: LaunchSkinny<2, 8>(launch, ka); break;
        default: LaunchSkinny<2, 16>(launch, ka); break;
      }
      return VX_OK;
    }
    if (k % 4 != 0 || std::max(n, t) * k * sizeof(float) >= (std::size_t{1} << 32) ||
        t * n * sizeof(float) >= (std::size_t{1} << 32))
      return vx::Fail(VX_UNSUPPORTED, "vx_vae_decode: product shape");
    const dim3 grid(static_cast<unsigned>((n + kTileRows - 1) / kTileRows),
                    static_cast<unsigned>((t + kTileRows - 1) / kTileRows),
                    static_cast<unsigned>(splits));
    if (splits == 1) {
      F32TileKernel<<<grid, kTileThreads, 0, stream>>>(x, w, y, static_cast<int>(t),
                                                       static_cast<int>(k), static_cast<int>(n),
                                                       accumulate ? 1 : 0, unit);
      return VX_OK;
    }
    F32TileKernel<<<grid, kTileThreads, 0, stream>>>(x, w, partials, static_cast<int>(t),
                                                     static_cast<int>(k), static_cast<int>(n), 0,
                                                     UnitWindow{});
    SplitSumKernel<<<Blocks(std::max(t * n, static_cast<std::size_t>(unit.head))), kThreads, 0,
                     stream>>>(partials, static_cast<int>(splits), y, static_cast<int>(t),
                               static_cast<int>(n), unit);
    return VX_OK;
  }

  /// Buffers for chunks of `frames` latent frames.
  int Reserve(std::size_t frames) {
    if (frames <= capacity_frames)
      return VX_OK;
    std::size_t widest = frames * std::max(shape.latent_dim, shape.decoder_dim);
    std::size_t t = frames;
    for (const Block& b : blocks) {
      widest = std::max(widest, t * 2 * b.in);
      t *= b.stride;
      widest = std::max(widest, t * b.out + 54 * b.out);
    }
    widest = std::max(widest, (t + kTaps) * out_channels);
    for (float** p : {&hidden, &next, &work, &scratch, &scratch2, &partials}) {
      if (*p != nullptr)
        (void)hipFree(*p);
      *p = nullptr;
      const std::size_t copies = p == &partials ? kMaxSplits : 1;
      VX_TRY(Allocate(p, copies * (widest + (kTaps - 1) * shape.latent_dim),
                      "vx_vae: hipMalloc"));
    }
    capacity_frames = frames;
    if (graph != nullptr) {
      (void)hipGraphExecDestroy(graph);
      graph = nullptr;
      seen = false;
    }
    return VX_OK;
  }

  int Launch(const float* latents, std::size_t frames, float* samples, hipStream_t stream) {
    const std::size_t latent = shape.latent_dim;
    // The residual stream and the transposed convolutions' outputs trade
    // buffers block by block (locals: every call starts from the same two).
    float* stream_rows = hidden;
    float* next_rows = next;
    // The windows alternate between two buffers: a product whose operand
    // is made from one window writes the next window into the other.
    float* windows[2] = {scratch, scratch2};
    std::size_t t = frames;
    // Each product's epilogue makes its consumer's input: a block's input
    // x2 (in work; unit 0 then refreshes the block's state from x2's last
    // frame), a unit's window or the output window. Where a unit's
    // depthwise convolution is not made in its product's operand loads, it
    // writes into the stream buffer the block's transposed convolution
    // left behind.
    const auto block_input_of = [&](const Block& b, const float* bias) {
      UnitWindow unit;
      unit.bias = bias;
      unit.alpha = b.w.alpha;
      unit.window = work;
      unit.state = b.state;
      unit.head = static_cast<int>(b.in);
      unit.channels = static_cast<int>(b.in);
      unit.scale = b.w.scale;
      unit.shift = b.w.bias;
      unit.frames = static_cast<int>(t);
      return unit;
    };
    const auto window_of = [&](float* into, const float* alpha, float* state, int head_rows,
                               std::size_t c, const float* bias) {
      UnitWindow unit;
      unit.bias = bias;
      unit.alpha = alpha;
      unit.window = into;
      unit.state = state;
      unit.head = head_rows * static_cast<int>(c);
      unit.channels = static_cast<int>(c);
      return unit;
    };
    // A depthwise convolution (with Snake when alpha is set) of `window`
    // feeding a product: in its operand loads where Fusable, else its own
    // launch into next_rows.
    const auto depthwise_product = [&](const float* window, const float* dw_w, const float* dw_b,
                                       const float* dw_alpha, float* state, int d,
                                       const float* copy_from, float* copy_to,
                                       std::size_t copy_count, const float* w, float* y,
                                       std::size_t k, std::size_t n, bool accumulate,
                                       const UnitWindow& next) {
      if (Fusable(t, k, n)) {
        DwOperand op;
        op.weights = dw_w;
        op.bias = dw_b;
        op.alpha = dw_alpha;
        op.dilation = d;
        op.state = state;
        op.copy_from = copy_from;
        op.copy_to = copy_to;
        op.copy_count = static_cast<int>(copy_count);
        return Gemm(window, w, y, t, k, n, accumulate, stream, next, &op);
      }
      const std::size_t rows = static_cast<std::size_t>(kTaps - 1) * d;
      DepthwiseKernel<<<WaveBlocks(std::max({t * k, rows * k, copy_count})), kWaveThreads, 0,
                        stream>>>(
          window, dw_w, dw_b, dw_alpha, next_rows, state, t, k, d, copy_from, copy_to,
          copy_count);
      return Gemm(next_rows, w, y, t, k, n, accumulate, stream, next);
    };
    // The latents' depthwise (no Snake) and pointwise convolutions. Where
    // Fusable the product reads its window from the latents' history and
    // the latents themselves, and leaves the next chunk's history in
    // in_state_next, which the last launch copies into in_state; else the
    // latents are staged after their history in the second window buffer.
    const bool input_fused = Fusable(t, latent, shape.decoder_dim);
    if (input_fused) {
      DwOperand op;
      op.weights = weights.in_depthwise;
      op.bias = weights.in_depthwise_bias;
      op.dilation = 1;
      op.state = in_state_next;
      op.head = in_state;
      VX_TRY(Gemm(latents, weights.in_pointwise, stream_rows, t, latent, shape.decoder_dim, false,
                  stream, block_input_of(blocks.front(), weights.in_pointwise_bias), &op));
    } else {
      StageKernel<<<Blocks((kTaps - 1 + t) * latent), kThreads, 0, stream>>>(
          in_state, latents, windows[1], t, latent);
      VX_TRY(depthwise_product(windows[1], weights.in_depthwise, weights.in_depthwise_bias,
                               nullptr, in_state, 1, nullptr, nullptr, 0, weights.in_pointwise,
                               stream_rows, latent, shape.decoder_dim, false,
                               block_input_of(blocks.front(), weights.in_pointwise_bias)));
    }
    for (std::size_t bi = 0; bi < blocks.size(); ++bi) {
      Block& b = blocks[bi];
      const std::size_t t_in = t;
      const std::size_t c = b.out;
      VX_TRY(Gemm(work, b.up2, next_rows, t, 2 * b.in, b.stride * c, false, stream,
                  window_of(windows[0], b.w.units[0].alpha_in, b.unit_state[0], kTaps - 1, c,
                            b.w.up_bias)));
      std::swap(stream_rows, next_rows);
      t *= b.stride;
      for (int u = 0; u < 3; ++u) {
        const vx_vae_unit& unit = b.w.units[u];
        const bool refresh = u == 0;
        // The next consumer: unit u + 1, the next block's input or the output.
        float* into = windows[(u + 1) % 2];
        UnitWindow next;
        if (u < 2) {
          const int dn = kDilations[u + 1];
          next = window_of(into, b.w.units[u + 1].alpha_in, b.unit_state[u + 1],
                           (kTaps - 1) * dn, c, unit.pointwise_bias);
        } else if (bi + 1 < blocks.size()) {
          next = block_input_of(blocks[bi + 1], unit.pointwise_bias);
        } else {
          next = window_of(into, weights.out_alpha, out_state, kTaps - 1, c,
                           unit.pointwise_bias);
        }
        VX_TRY(depthwise_product(windows[u % 2], unit.depthwise, unit.depthwise_bias,
                                 unit.alpha_out, b.unit_state[u], kDilations[u],
                                 refresh ? work + (t_in - 1) * 2 * b.in : nullptr,
                                 refresh ? b.state : nullptr, refresh ? b.in : 0, unit.pointwise,
                                 stream_rows, c, c, true, next));
      }
    }
    const std::size_t c = out_channels;
    float* out_window = windows[1];  // the last unit's (u = 2) next window
    int lanes = 1;
    while (lanes < kWave && 4 * static_cast<std::size_t>(lanes) < c)
      lanes *= 2;
    const std::size_t copy_floats = input_fused ? (kTaps - 1) * latent : 0;
    ToMonoKernel<<<Blocks(std::max({t * lanes, (kTaps - 1) * c, copy_floats})), kThreads, 0,
                   stream>>>(out_window, weights.out_conv, weights.out_bias, samples, out_state,
                             t, c, lanes, input_fused ? in_state_next : nullptr,
                             input_fused ? in_state : nullptr, static_cast<int>(copy_floats));
    return vx::LaunchStatus("vx_vae_decode");
  }
};

namespace {

int CheckUnit(const vx_vae_unit& u) {
  return u.alpha_in && u.depthwise && u.depthwise_bias && u.alpha_out && u.pointwise &&
                 u.pointwise_bias
             ? VX_OK
             : vx::Fail(VX_BAD_ARG, "vx_vae_create: null unit weights");
}

}  // namespace

extern "C" {

int vx_vae_create(vx_vae** vae, const vx_vae_shape* shape, const vx_vae_weights* weights) {
  if (vae == nullptr || shape == nullptr || weights == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_vae_create: null argument");
  *vae = nullptr;
  if (shape->latent_dim == 0 || shape->decoder_dim == 0 || shape->rate_count == 0 ||
      shape->rate_count > 8 || (shape->decoder_dim >> shape->rate_count) == 0 ||
      shape->decoder_dim % (std::size_t{1} << shape->rate_count) != 0)
    return vx::Fail(VX_BAD_ARG, "vx_vae_create: bad shape");
  // The products read x and the weights 16 bytes at a time along k.
  if (shape->latent_dim % 4 != 0 || (shape->decoder_dim >> shape->rate_count) % 4 != 0)
    return vx::Fail(VX_UNSUPPORTED,
                    "vx_vae_create: latent and channel counts must be multiples of 4");
  if (weights->blocks == nullptr || weights->in_depthwise == nullptr ||
      weights->in_depthwise_bias == nullptr || weights->in_pointwise == nullptr ||
      weights->in_pointwise_bias == nullptr || weights->out_alpha == nullptr ||
      weights->out_conv == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_vae_create: null weights");
  std::size_t hop = 1;
  for (std::size_t b = 0; b < shape->rate_count; ++b) {
    const vx_vae_block& block = weights->blocks[b];
    hop *= shape->rates[b];
    if (shape->rates[b] == 0 || hop > kMaxSamples)
      return vx::Fail(VX_BAD_ARG, "vx_vae_create: a zero rate, or over 2096640 samples per frame");
    if (!block.scale || !block.bias || !block.alpha || !block.up ||
        !block.up_bias)
      return vx::Fail(VX_BAD_ARG, "vx_vae_create: null block weights");
    for (const vx_vae_unit& u : block.units)
      VX_TRY(CheckUnit(u));
  }
  auto* created = new vx_vae();
  created->shape = *shape;
  created->weights = *weights;
  created->weights.blocks = nullptr;
  int status = VX_OK;
  std::size_t c = shape->decoder_dim;
  for (std::size_t b = 0; b < shape->rate_count && status == VX_OK; ++b) {
    Block block;
    block.in = c;
    block.out = c / 2;
    block.stride = shape->rates[b];
    block.w = weights->blocks[b];
    created->hop *= block.stride;
    status = Allocate(&block.up2, block.stride * block.out * 2 * block.in, "vx_vae: hipMalloc");
    if (status == VX_OK)
      status = Allocate(&block.state, block.in, "vx_vae: hipMalloc");
    for (int u = 0; u < 3 && status == VX_OK; ++u)
      status = Allocate(&block.unit_state[u],
                        static_cast<std::size_t>(kTaps - 1) * kDilations[u] * block.out,
                        "vx_vae: hipMalloc");
    if (status == VX_OK) {
      const std::size_t count = block.stride * block.out * 2 * block.in;
      RepackUpKernel<<<Blocks(count), kThreads>>>(block.w.up, block.up2, block.in, block.out,
                                                  block.stride);
      status = vx::LaunchStatus("vx_vae_create");
    }
    created->blocks.push_back(block);
    c /= 2;
  }
  created->out_channels = c;
  if (status == VX_OK)
    status = Allocate(&created->in_state, (kTaps - 1) * shape->latent_dim, "vx_vae: hipMalloc");
  if (status == VX_OK)
    status = Allocate(&created->in_state_next, (kTaps - 1) * shape->latent_dim,
                      "vx_vae: hipMalloc");
  if (status == VX_OK)
    status = Allocate(&created->out_state, (kTaps - 1) * c, "vx_vae: hipMalloc");
  if (status == VX_OK && hipDeviceSynchronize() != hipSuccess)
    status = vx::Fail(VX_HIP_ERROR, "vx_vae_create: repack");
  if (status != VX_OK) {
    delete created;
    return status;
  }
  *vae = created;
  return vx_vae_reset(created, nullptr);
}

void vx_vae_destroy(vx_vae* vae) { delete vae; }

int vx_vae_reset(vx_vae* vae, void* stream) {
  if (vae == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_vae_reset: null handle");
  hipStream_t s = vx::Stream(stream);
  const auto clear = [&](float* p, std::size_t count) {
    ZeroKernel<<<Blocks(count), kThreads, 0, s>>>(p, count);
    return hipGetLastError() == hipSuccess;
  };
  bool ok = clear(vae->in_state, (kTaps - 1) * vae->shape.latent_dim) &&
            clear(vae->out_state, (kTaps - 1) * vae->out_channels);
  for (Block& b : vae->blocks) {
    ok = ok && clear(b.state, b.in);
    for (int u = 0; u < 3; ++u)
      ok = ok && clear(b.unit_state[u], static_cast<std::size_t>(kTaps - 1) * kDilations[u] * b.out);
  }
  if (!ok)
    return vx::Fail(VX_HIP_ERROR, "vx_vae_reset: launch");
  return vx::Succeed();
}

size_t vx_vae_hop(const vx_vae* vae) { return vae == nullptr ? 0 : vae->hop; }

// Products take one 32-row block per grid row, at most 65535 of them.
size_t vx_vae_max_frames(const vx_vae* vae) {
  return vae == nullptr ? 0 : kMaxSamples / vae->hop;
}

int vx_vae_decode(vx_vae* vae, const float* latents, size_t frames, float* samples,
                  void* stream) {
  if (vae == nullptr || latents == nullptr || samples == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_vae_decode: null argument");
  if (frames == 0)
    return VX_OK;
  if (frames > vx_vae_max_frames(vae))
    return vx::Fail(VX_BAD_ARG, "vx_vae_decode: too many frames in one chunk "
                                "(vx_vae_max_frames)");
  hipStream_t s = vx::Stream(stream);
  VX_TRY(vae->Reserve(frames));
  GraphKey key{latents, samples, frames, s};
  hipStreamCaptureStatus capturing = hipStreamCaptureStatusNone;
  if (s != nullptr)
    VX_HIP(hipStreamIsCapturing(s, &capturing), "vx_vae_decode: capture status");
  if (s == nullptr || capturing != hipStreamCaptureStatusNone || frames > kMaxGraphFrames)
    return vae->Launch(latents, frames, samples, s);
  if (!(vae->graph_key == key)) {
    if (vae->graph != nullptr)
      (void)hipGraphExecDestroy(vae->graph);
    vae->graph = nullptr;
    vae->graph_key = key;
    vae->seen = false;
  }
  if (vae->graph == nullptr) {
    if (!vae->seen) {  // the first call of a key runs eagerly
      vae->seen = true;
      return vae->Launch(latents, frames, samples, s);
    }
    VX_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal),
           "vx_vae_decode: begin capture");
    const int status = vae->Launch(latents, frames, samples, s);
    hipGraph_t captured = nullptr;
    const hipError_t ended = hipStreamEndCapture(s, &captured);
    if (status != VX_OK) {
      if (captured != nullptr)
        (void)hipGraphDestroy(captured);
      return status;
    }
    if (ended != hipSuccess)
      return vx::FailHip(ended, "vx_vae_decode: end capture");
    const hipError_t made = hipGraphInstantiate(&vae->graph, captured, nullptr, nullptr, 0);
    (void)hipGraphDestroy(captured);
    if (made != hipSuccess) {
      vae->graph = nullptr;
      return vx::FailHip(made, "vx_vae_decode: instantiate");
    }
  }
  VX_HIP(hipGraphLaunch(vae->graph, s), "vx_vae_decode: graph launch");
  return vx::Succeed();
}

}  // extern "C"
