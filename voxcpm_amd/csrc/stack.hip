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
#include <utility>
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
constexpr int kMaxNormRows = 8;  // rows of the one-tile row-major path
// The split attention spreads a chunk's query heads over workgroups while
// its grid stays within this many (one per compute unit).
constexpr int kSpreadWorkgroups = 256;

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
  // When non-null, `past` is read here instead (a captured graph replays
  // with the value of each call; the grid then covers the cache).
  const int* past_device;
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

/// Maximum over the wave: rows of 16 by DPP, then the rows by permlane
/// swaps (every lane receives it).
__device__ inline float WaveMax64(float x) {
  x = RowMax16(x);
  auto swapped = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  x = fmaxf(__uint_as_float(swapped[0]), __uint_as_float(swapped[1]));
  swapped = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(swapped[0]), __uint_as_float(swapped[1]));
}

/// Sum over the wave in a fixed order (every lane receives the same bits).
__device__ inline float WaveSum64(float x) { return AddXor32(AddXor16(RowSum16(x))); }

/// Keys of a row: past + its position in the sequence (causal) or the
/// whole sequence.
__device__ inline int KeyCount(const AttentionArgs& a, int row) {
  const int past = a.past_device != nullptr ? *a.past_device : a.past;
  return past + (a.causal != 0 ? row % a.rows_per_sequence + 1 : a.rows_per_sequence);
}

/// One chunk of keys of one (row, KV head) for the KV head's `group` query
/// heads (kernels/generator_kernels.hip:160-241 in the chunk). Every load
/// is issued at the start -- the chunk's keys (lanes over key and quarter
/// of the dimensions), each wave's 16 value rows (lanes over dimensions)
/// and the queries -- so that one memory round trip serves the chunk.
/// Scores q . k scale meet over the quarters by permlane swaps; the
/// chunk's maximum and sum per head; the values weighted by exp(score -
/// max), the four waves' sums added in wave order. One chunk writes the
/// output itself; several leave (max, sum, values) for MergeKernel.
/// Chunks past a row's keys do nothing (the merge reads the row's chunks
/// only). A workgroup takes G of the KV head's query heads (blockIdx.z:
/// the KV head, then which G of its group): a short cache spreads its few
/// chunks' heads over more compute units, each with a G-th of the scoring.
template<int D, int G>
__global__ __launch_bounds__(kThreads) void SplitAttentionKernel(AttentionArgs a) {
  constexpr int kQuarter = D / 4;
  constexpr int kPerLane = D / kWave;
  extern __shared__ float lds[];
  float* qs = lds;                 // [G][D]
  float* ps = qs + G * D;          // [G][kChunk]
  float* stats = ps + G * kChunk;  // [G][2]
  float* parts = stats + 2 * G;    // [waves][G][D]
  const int split = static_cast<int>(blockIdx.x);
  const int row = static_cast<int>(blockIdx.y);
  const int parts_per_kv = a.heads / a.kv_heads / G;
  const int g = static_cast<int>(blockIdx.z) / parts_per_kv;  // the KV head
  const int head0 =
      g * (a.heads / a.kv_heads) + (static_cast<int>(blockIdx.z) % parts_per_kv) * G;
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int first = (row / a.rows_per_sequence) * a.keys_per_sequence;
  const int key0 = split * kChunk;
  // Keys and values are loaded before past is known (a chunk's first key
  // lies in the cache for every past the grid covers); keys past the cache
  // re-read the chunk's first.
  const int limit = a.capacity - first;
  const std::size_t base = static_cast<std::size_t>(g) * a.capacity + first;

  // Keys: lane (key 16 wave + lane % 16, quarter lane / 16).
  const int key_local = 16 * wave + lane % 16;
  const int quarter = lane / 16;
  float4 kv[kQuarter / 4];
  {
    const int key = key0 + key_local;
    const float4* krow = reinterpret_cast<const float4*>(
        a.k + (base + (key < limit ? key : key0)) * D + quarter * kQuarter);
#pragma unroll
    for (int i = 0; i < kQuarter / 4; ++i)
      kv[i] = krow[i];
  }
  // Values: wave w's keys 16 w .. 16 w + 15, lanes over dimensions.
  float vv[16][kPerLane];
#pragma unroll
  for (int kk = 0; kk < 16; ++kk) {
    const int key = key0 + 16 * wave + kk;
    const float* vrow = a.v + (base + (key < limit ? key : key0)) * D + lane * kPerLane;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j)
      vv[kk][j] = vrow[j];
  }
  // The group's queries, four floats per thread per step.
  constexpr int kQueryLoads = (G * D / 4 + kThreads - 1) / kThreads;
  float4 qv4[kQueryLoads];
  const float4* qsrc = reinterpret_cast<const float4*>(
      a.q + (static_cast<std::size_t>(row) * a.heads + head0) * D);
#pragma unroll
  for (int i = 0; i < kQueryLoads; ++i) {
    const int e4 = static_cast<int>(threadIdx.x) + i * kThreads;
    if (e4 < G * D / 4)
      qv4[i] = qsrc[e4];
  }
  const int count = KeyCount(a, row);
  const int key1 = min(count, key0 + kChunk);
  if (key0 >= key1)
    return;  // past this row's keys: the merge reads the row's chunks only
  const bool valid = key0 + key_local < key1;
  // Rows past the row's keys may hold anything (the cache beyond what was
  // written): their values are dropped, not weighted by 0.
#pragma unroll
  for (int kk = 0; kk < 16; ++kk)
#pragma unroll
    for (int j = 0; j < kPerLane; ++j)
      vv[kk][j] = key0 + 16 * wave + kk < key1 ? vv[kk][j] : 0.0F;
#pragma unroll
  for (int i = 0; i < kQueryLoads; ++i) {
    const int e4 = static_cast<int>(threadIdx.x) + i * kThreads;
    if (e4 < G * D / 4) {
      const float4 v = qv4[i];
      reinterpret_cast<float4*>(qs)[e4] =
          make_float4(v.x * a.scale, v.y * a.scale, v.z * a.scale, v.w * a.scale);
    }
  }
  __syncthreads();

  // Scores of up to kHeadBlock heads at once: each step reads the heads'
  // next four query dimensions (one LDS broadcast per head) into
  // independent sums, so the reads are in flight together and no sum waits
  // on another's latency; each sum still adds its terms in dimension order.
  constexpr int kHeadBlock = G < 8 ? G : 8;
  for (int h0 = 0; h0 < G; h0 += kHeadBlock) {
    float s[kHeadBlock];
#pragma unroll
    for (int hh = 0; hh < kHeadBlock; ++hh)
      s[hh] = 0.0F;
#pragma unroll
    for (int i = 0; i < kQuarter / 4; ++i) {
      float4 q[kHeadBlock];
#pragma unroll
      for (int hh = 0; hh < kHeadBlock; ++hh)
        q[hh] = reinterpret_cast<const float4*>(qs + (h0 + hh) * D + quarter * kQuarter)[i];
#pragma unroll
      for (int hh = 0; hh < kHeadBlock; ++hh)
        s[hh] += q[hh].x * kv[i].x + q[hh].y * kv[i].y + q[hh].z * kv[i].z + q[hh].w * kv[i].w;
    }
#pragma unroll
    for (int hh = 0; hh < kHeadBlock; ++hh) {
      const float total = AddXor32(AddXor16(s[hh]));
      if (quarter == 0)
        ps[(h0 + hh) * kChunk + key_local] = valid ? total : -INFINITY;
    }
  }
  __syncthreads();

  // The chunk's softmax statistics per head (wave w: heads w, w + 4, ...).
  for (int hh = wave; hh < G; hh += kWaves) {
    const float s = ps[hh * kChunk + lane];
    const float m = WaveMax64(s);
    const float p = s == -INFINITY ? 0.0F : expf(s - m);
    const float l = WaveSum64(p);
    ps[hh * kChunk + lane] = p;
    if (lane == 0) {
      stats[2 * hh] = m;
      stats[2 * hh + 1] = l;
    }
  }
  __syncthreads();

  // Each head's weighted values over the wave's 16 keys into LDS, four
  // keys per step for a block of heads at once (independent sums, each
  // adding its keys in order).
  for (int h0 = 0; h0 < G; h0 += kHeadBlock) {
    float o[kHeadBlock][kPerLane];
#pragma unroll
    for (int hh = 0; hh < kHeadBlock; ++hh)
#pragma unroll
      for (int j = 0; j < kPerLane; ++j)
        o[hh][j] = 0.0F;
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      float4 p[kHeadBlock];
#pragma unroll
      for (int hh = 0; hh < kHeadBlock; ++hh)
        p[hh] = reinterpret_cast<const float4*>(ps + (h0 + hh) * kChunk + 16 * wave)[k4];
#pragma unroll
      for (int hh = 0; hh < kHeadBlock; ++hh)
#pragma unroll
        for (int j = 0; j < kPerLane; ++j) {
          o[hh][j] += p[hh].x * vv[4 * k4][j];
          o[hh][j] += p[hh].y * vv[4 * k4 + 1][j];
          o[hh][j] += p[hh].z * vv[4 * k4 + 2][j];
          o[hh][j] += p[hh].w * vv[4 * k4 + 3][j];
        }
    }
#pragma unroll
    for (int hh = 0; hh < kHeadBlock; ++hh)
#pragma unroll
      for (int j = 0; j < kPerLane; ++j)
        parts[(wave * G + h0 + hh) * D + lane * kPerLane + j] = o[hh][j];
  }
  __syncthreads();
  const int width = a.heads * D;
  const std::size_t stride = static_cast<std::size_t>(D) + 2;
  for (int e = static_cast<int>(threadIdx.x); e < G * D; e += kThreads) {
    float total = parts[e];
#pragma unroll
    for (int w = 1; w < kWaves; ++w)
      total += parts[w * G * D + e];
    const int hh = e / D;
    const int d = e % D;
    if (a.splits == 1) {
      a.out[OutIndex(a, row, (head0 + hh) * D + d, width)] =
          Bf16Bits(total * (1.0F / stats[2 * hh + 1]));
    } else {
      float* target =
          a.partials +
          ((static_cast<std::size_t>(row) * a.heads + head0 + hh) * a.splits + split) * stride;
      target[2 + d] = total;
      if (d == 0) {
        target[0] = stats[2 * hh];
        target[1] = stats[2 * hh + 1];
      }
    }
  }
}

/// The chunks of one (row, head) met in chunk order: M = max m_c,
/// L = sum l_c exp(m_c - M), out = bf16(sum o_c exp(m_c - M) / L), over the
/// row's chunks only. Lane c takes chunk c's statistics (chunks 64 apart in
/// turn). The first kPreload chunks' values are loaded at the start with
/// the statistics and the row's key count (which may come from the
/// device), so that a cache of up to 2048 keys takes one memory round
/// trip; later chunks are loaded eight at a time.
template<int D>
__global__ __launch_bounds__(kWave) void MergeKernel(AttentionArgs a) {
  constexpr int kPerLane = D / kWave;
  constexpr int kPreload = 32;
  constexpr int kBatch = 8;
  const int row = static_cast<int>(blockIdx.x);
  const int head = static_cast<int>(blockIdx.y);
  const int lane = static_cast<int>(threadIdx.x);
  const std::size_t stride = static_cast<std::size_t>(D) + 2;
  const float* base =
      a.partials + (static_cast<std::size_t>(row) * a.heads + head) * a.splits * stride;
  // Every slot below `splits` lies inside the partials; slots past the
  // row's chunks hold stale values and are masked below.
  const int slots = min(a.splits, kWave);
  const float* mine = base + static_cast<std::size_t>(min(lane, slots - 1)) * stride;
  const float first_m = mine[0];
  const float first_l = mine[1];
  float first[kPreload][kPerLane];
#pragma unroll
  for (int b = 0; b < kPreload; ++b) {
    const float* part = base + static_cast<std::size_t>(min(b, a.splits - 1)) * stride + 2 +
                        lane * kPerLane;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j)
      first[b][j] = part[j];
  }
  const int chunks = (KeyCount(a, row) + kChunk - 1) / kChunk;
  float m = lane < chunks ? first_m : -INFINITY;
  for (int c = lane + kWave; c < chunks; c += kWave)
    m = fmaxf(m, base[c * stride]);
  m = WaveMax64(m);
  float o[kPerLane];
#pragma unroll
  for (int j = 0; j < kPerLane; ++j)
    o[j] = 0.0F;
  float l = 0.0F;
  // Chunks i0 .. i0 + kBatch - 1 of the pass at c0, loaded together.
  const auto add_batch = [&](int c0, int i0, int count, float factor) {
    float values[kBatch][kPerLane];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const float* part = base + (c0 + min(i0 + b, count - 1)) * stride + 2 + lane * kPerLane;
#pragma unroll
      for (int j = 0; j < kPerLane; ++j)
        values[b][j] = part[j];
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const float f = __shfl(factor, i0 + b, kWave);
      if (i0 + b < count) {
#pragma unroll
        for (int j = 0; j < kPerLane; ++j)
          o[j] += values[b][j] * f;
      }
    }
  };
  for (int c0 = 0; c0 < chunks; c0 += kWave) {
    const int c = c0 + lane;
    float factor = 0.0F;
    if (c < chunks) {
      const float* part = base + c * stride;
      const float cm = c0 == 0 ? first_m : part[0];
      const float cl = c0 == 0 ? first_l : part[1];
      factor = expf(cm - m);
      l += cl * factor;
    }
    const int count = min(kWave, chunks - c0);
    int i0 = 0;
    if (c0 == 0) {
#pragma unroll
      for (int b = 0; b < kPreload; ++b) {
        const float f = __shfl(factor, b, kWave);
        if (b < count) {
#pragma unroll
          for (int j = 0; j < kPerLane; ++j)
            o[j] += first[b][j] * f;
        }
      }
      i0 = kPreload;
    }
    for (; i0 < count; i0 += kBatch)
      add_batch(c0, i0, count, factor);
  }
  // Lane c's chunks' sums, then the lanes by a fixed tree.
  l = WaveSum64(l);
  const float inverse = 1.0F / l;
  const int width = a.heads * D;
#pragma unroll
  for (int j = 0; j < kPerLane; ++j)
    a.out[OutIndex(a, row, head * D + lane * kPerLane + j, width)] = Bf16Bits(o[j] * inverse);
}

template<int D, int G>
void LaunchSplit(const AttentionArgs& a, int rows, hipStream_t stream) {
  const std::size_t shared = SharedFloats(G, D) * sizeof(float);
  const int parts_per_kv = a.heads / a.kv_heads / G;
  SplitAttentionKernel<D, G><<<dim3(static_cast<unsigned>(a.splits), static_cast<unsigned>(rows),
                                    static_cast<unsigned>(a.kv_heads * parts_per_kv)),
                               kThreads, shared, stream>>>(a);
}

/// Query heads per workgroup: the KV head's whole group once the chunks
/// alone fill the compute units, fewer (down to one) while they do not.
int HeadsPerWorkgroup(int group, int chunks) {
  int heads = group;
  while (heads > 1 && chunks * (group / heads) * 2 <= kSpreadWorkgroups)
    heads /= 2;
  return heads;
}

template<int D>
void LaunchAttention(const AttentionArgs& a, int rows, hipStream_t stream) {
  switch (HeadsPerWorkgroup(a.heads / a.kv_heads, a.splits * rows * a.kv_heads)) {
    case 1: LaunchSplit<D, 1>(a, rows, stream); break;
    case 2: LaunchSplit<D, 2>(a, rows, stream); break;
    case 4: LaunchSplit<D, 4>(a, rows, stream); break;
    case 8: LaunchSplit<D, 8>(a, rows, stream); break;
    default: LaunchSplit<D, 16>(a, rows, stream); break;
  }
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

/// Writes `past` for the attention launches of a replayed graph.
__global__ void SetPastKernel(int* past_device, int past) { *past_device = past; }

void SetPast(int* past_device, std::size_t past, hipStream_t stream) {
  SetPastKernel<<<1, 1, 0, stream>>>(past_device, static_cast<int>(past));
}

/// Floats of the chunks' partial results of `rows` rows.
std::size_t AttentionPartialFloats(std::size_t rows, std::size_t heads, std::size_t head_dim,
                                   int splits) {
  return splits > 1 ? rows * heads * static_cast<std::size_t>(splits) * (head_dim + 2) : 0;
}

/// Checks the shape the split attention takes: head_dim 64 or 128 (VoxCPM2's
/// stacks take 128), 1, 2, 4, 8 or 16 query heads per KV head, its LDS within
/// 64 KB.
bool AttentionSupported(std::size_t heads, std::size_t kv_heads, std::size_t head_dim) {
  if (kv_heads == 0 || heads % kv_heads != 0)
    return false;
  const std::size_t group = heads / kv_heads;
  if (group != 1 && group != 2 && group != 4 && group != 8 && group != 16)
    return false;
  if (head_dim != 64 && head_dim != 128)
    return false;
  return SharedFloats(static_cast<int>(heads / kv_heads), static_cast<int>(head_dim)) *
             sizeof(float) <=
         65536;
}

/// The split attention over one layer's cache (the caller has checked the
/// shape, the bounds and the partials' size). `splits` chunks per (row, KV
/// head); with `past_device` non-null the kernels read past there.
void Attention(const float* q, const float* k_cache, const float* v_cache, Bf16* out,
               bool fragment, float* partials, std::size_t rows,
               std::size_t rows_per_sequence, std::size_t keys_per_sequence, std::size_t past,
               bool causal, std::size_t heads, std::size_t kv_heads, std::size_t head_dim,
               std::size_t capacity, int splits, const int* past_device, hipStream_t stream) {
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
  a.splits = splits;
  a.scale = 1.0F / std::sqrt(static_cast<float>(head_dim));
  a.fragment = fragment ? 1 : 0;
  a.past_device = past_device;
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

namespace {

template<q8::ASource SRC, q8::Output OUT, int RG, int PW>
void LaunchRowEngine(const q8::TileArgs& args, int tiles, q8::Weights kind, hipStream_t stream) {
  constexpr int kEngineThreads = q8::EngineThreads(1, RG);
  const std::size_t shared = q8::NormRowsShared(1, RG, args.m, args.k);
  if (kind == q8::Weights::kQ8)
    q8::EngineKernel<1, RG, SRC, OUT, PW, 2, q8::Weights::kQ8>
        <<<tiles, kEngineThreads, shared, stream>>>(args);
  else
    q8::EngineKernel<1, RG, SRC, OUT, PW, 2, q8::Weights::kBf16>
        <<<tiles, kEngineThreads, shared, stream>>>(args);
}

q8::TileArgs RowArgs(const void* weight, int m, int k, int n) {
  q8::TileArgs args{};
  args.w = static_cast<const std::uint8_t*>(weight);
  args.m = m;
  args.k = k;
  args.n = n;
  args.pairs = static_cast<int>(q8::Pairs(static_cast<std::size_t>(k)));
  args.groups = (n + 15) / 16;
  args.group_stride = 1;
  args.row_blocks = 1;
  args.rows_per_block = m;
  args.tile_blocks = 1;
  return args;
}

}  // namespace

bool RowsSupported(std::size_t hidden, std::size_t ffn) {
  return hidden % 64 == 0 && hidden <= 2 * 64 * 16 && ffn % 16 == 0 &&
         q8::NormRowsShared(1, 2, kMaxNormRows, static_cast<int>(hidden)) <= 65536;
}

void NormQkvRows(const float* h, const Bf16* gamma, float eps, const void* weight, float* qkv,
                 int rows, int hidden, int n, q8::Weights kind, hipStream_t stream) {
  q8::TileArgs args = RowArgs(weight, rows, hidden, n);
  args.h = h;
  args.gamma = gamma;
  args.eps = eps;
  args.y = qkv;
  if (args.pairs <= 16)
    LaunchRowEngine<q8::ASource::kNormRows, q8::Output::kStore, 1, 1>(args, args.groups, kind,
                                                                       stream);
  else
    LaunchRowEngine<q8::ASource::kNormRows, q8::Output::kStore, 1, 2>(args, args.groups, kind,
                                                                       stream);
}

/// rmsnorm(h) Wqkv^T with the rotary embedding and the cache writes in the
/// epilogue (QkvRope's work): each workgroup owns 8 rows of a rotary
/// dimension's two row groups, head_dim / 2 columns apart (the halves of
/// a pair in two workgroups: twice the workgroups of one pair each, which
/// left most compute units idle: base LM step 1004 -> 980 us at 1024
/// cached positions on MI355X). head_dim a multiple of 32.
void NormQkvCacheRows(const float* h, const Bf16* gamma, float eps, const void* weight,
                      const float* rope, const std::int32_t* positions,
                      const std::int32_t* cache_rows, float* q, float* k_cache, float* v_cache,
                      int rows, int hidden, int heads, int kv_heads, int head_dim, int capacity,
                      q8::Weights kind, hipStream_t stream) {
  const int n = (heads + 2 * kv_heads) * head_dim;
  q8::TileArgs args = RowArgs(weight, rows, hidden, n);
  args.h = h;
  args.gamma = gamma;
  args.eps = eps;
  args.group_stride = head_dim / 32;
  args.q_out = q;
  args.k_cache = k_cache;
  args.v_cache = v_cache;
  args.rope = rope;
  args.positions = positions;
  args.cache_rows = cache_rows;
  args.heads = heads;
  args.kv_heads = kv_heads;
  args.head_dim = head_dim;
  args.capacity = capacity;
  const int tiles = args.groups;  // half pairs
  if (args.pairs <= 16)
    LaunchRowEngine<q8::ASource::kNormRows, q8::Output::kQkvCache, 1, 1>(args, tiles, kind,
                                                                         stream);
  else
    LaunchRowEngine<q8::ASource::kNormRows, q8::Output::kQkvCache, 1, 2>(args, tiles, kind,
                                                                         stream);
}

void NormGateUpRows(const float* h, const Bf16* gamma, float eps, const void* weight, Bf16* act,
                    int rows, int hidden, int ffn, q8::Weights kind, hipStream_t stream) {
  q8::TileArgs args = RowArgs(weight, rows, hidden, 2 * ffn);
  args.h = h;
  args.gamma = gamma;
  args.eps = eps;
  args.y_bf16 = act;
  args.group_stride = ffn / 16;
  // Whole pairs (gate and up groups in one workgroup): half pairs measured
  // slower here, one per 16-wave workgroup (base LM step +16 us: three
  // workgroups per compute unit take two rounds), one per 8-wave workgroup
  // (the same step time, the 5-row encoder 279 -> 286 us) and three per
  // 16-wave workgroup (256 workgroups, each a third of the weights of
  // three pair halves: +9 us).
  const int tiles = ffn / 16;
  if (args.pairs <= 16)
    LaunchRowEngine<q8::ASource::kNormRows, q8::Output::kSwiGluRows, 2, 1>(args, tiles, kind,
                                                                           stream);
  else
    LaunchRowEngine<q8::ASource::kNormRows, q8::Output::kSwiGluRows, 2, 2>(args, tiles, kind,
                                                                           stream);
}

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

/// What a captured forward depends on besides `past`.
struct ForwardKey {
  float* hidden = nullptr;
  float* output = nullptr;
  std::size_t rows = 0;
  const std::int32_t* positions = nullptr;
  const std::int32_t* cache_rows = nullptr;
  std::size_t rows_per_sequence = 0;
  std::size_t keys_per_sequence = 0;
  bool causal = false;
  float* k_cache = nullptr;
  float* v_cache = nullptr;
  std::size_t capacity = 0;
  int path = 0;
  hipStream_t stream = nullptr;

  bool operator==(const ForwardKey& o) const {
    return hidden == o.hidden && output == o.output && rows == o.rows &&
           positions == o.positions && cache_rows == o.cache_rows &&
           rows_per_sequence == o.rows_per_sequence &&
           keys_per_sequence == o.keys_per_sequence && causal == o.causal &&
           k_cache == o.k_cache && v_cache == o.v_cache && capacity == o.capacity &&
           path == o.path && stream == o.stream;
  }
};

struct vx_stack {
  vx_stack_shape shape{};
  vx_stack_weights weights{};
  std::vector<vx_dit_layer> layers;
  std::size_t q_width = 0;
  std::size_t kv_width = 0;
  std::size_t qkv_width = 0;
  bool fused = false;       // the fragment-order kernels take the shape
  bool rows_fused = false;  // the one-tile row-major kernels take it
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

  // The replayed forwards of up to 32 rows and the past they read: one
  // graph per band of kBandKeys attended keys, whose attention grid covers
  // that band's chunks only (a short cache launches no workgroups for the
  // chunks it does not hold yet).
  static constexpr std::size_t kBandKeys = 256;
  int* past_device = nullptr;
  ForwardKey graph_key;
  std::vector<std::pair<int, hipGraphExec_t>> graphs;  // (attention splits, graph)

  void DropGraphs() {
    for (auto& entry : graphs)
      (void)hipGraphExecDestroy(entry.second);
    graphs.clear();
  }

  ~vx_stack() {
    DropGraphs();
    if (past_device != nullptr)
      (void)hipFree(past_device);
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
    const vx::ProductPlan plan = vx::PlanSkinny(m, k, n, 0, 0, 0, 0, 0, Kind());
    return vx::RunSkinny(x, w, y, nullptr, m, k, n, accumulate, plan, nullptr, nullptr,
                         stream, Kind());
  }

  int Resolved(std::size_t rows) const {
    const bool rows_ok = rows_fused && rows <= vx::stack::kMaxNormRows;
    const bool fragments_ok = fused && rows <= vx::q8::kFragRows;
    switch (path) {
      case VX_STACK_PATH_ROWS: return rows_ok ? VX_STACK_PATH_ROWS : VX_STACK_PATH_UNFUSED;
      case VX_STACK_PATH_FUSED: return fragments_ok ? VX_STACK_PATH_FUSED : VX_STACK_PATH_UNFUSED;
      case VX_STACK_PATH_UNFUSED: return VX_STACK_PATH_UNFUSED;
      default:
        return rows_ok ? VX_STACK_PATH_ROWS
                       : fragments_ok ? VX_STACK_PATH_FUSED : VX_STACK_PATH_UNFUSED;
    }
  }

  /// The launches of one forward; `splits` chunks per (row, KV head) of the
  /// attention, past read from `past_device` when it is non-null.
  int Launch(const ForwardKey& f, std::size_t past, int splits, const int* past_device,
             hipStream_t stream) {
    const std::size_t rows = f.rows;
    const std::size_t width = shape.hidden;
    const std::size_t ffn = shape.ffn;
    const std::size_t layer_stride = shape.kv_heads * f.capacity * shape.head_dim;
    const float* rope = shape.rope != 0 ? weights.rope : nullptr;
    if (f.path == VX_STACK_PATH_ROWS) {
      const int m = static_cast<int>(rows);
      for (std::size_t l = 0; l < layers.size(); ++l) {
        const vx_dit_layer& layer = layers[l];
        float* keys = f.k_cache + l * layer_stride;
        float* values = f.v_cache + l * layer_stride;
        if (shape.head_dim % 32 == 0) {
          vx::stack::NormQkvCacheRows(
              f.hidden, layer.input_norm, shape.eps, layer.qkv, rope, f.positions, f.cache_rows,
              q, keys, values, m, static_cast<int>(width), static_cast<int>(shape.heads),
              static_cast<int>(shape.kv_heads), static_cast<int>(shape.head_dim),
              static_cast<int>(f.capacity), Kind(), stream);
        } else {
          vx::stack::NormQkvRows(f.hidden, layer.input_norm, shape.eps, layer.qkv, qkv, m,
                                 static_cast<int>(width), static_cast<int>(qkv_width), Kind(),
                                 stream);
          vx::kernels::QkvRope(qkv, rope, f.positions, f.cache_rows, q, keys, values, rows,
                               shape.heads, shape.kv_heads, shape.head_dim, f.capacity, stream);
        }
        vx::stack::Attention(q, keys, values, bf16, false, attention_partials, rows,
                             f.rows_per_sequence, f.keys_per_sequence, past, f.causal,
                             shape.heads, shape.kv_heads, shape.head_dim, f.capacity, splits,
                             past_device, stream);
        VX_TRY(Linear(bf16, layer.o, f.hidden, rows, q_width, width, true, stream));
        vx::stack::NormGateUpRows(f.hidden, layer.post_norm, shape.eps, layer.gate_up, bf16, m,
                                  static_cast<int>(width), static_cast<int>(ffn), Kind(),
                                  stream);
        VX_TRY(Linear(bf16, layer.down, f.hidden, rows, ffn, width, true, stream));
      }
      vx::kernels::RmsNorm(f.hidden, weights.norm, bf16, f.output, rows, width, shape.eps,
                           stream);
      return vx::LaunchStatus("vx_stack_forward");
    }
    if (f.path == VX_STACK_PATH_FUSED) {
      vx::fused::Shape s = fs;
      s.rows = static_cast<int>(rows);
      vx::stack::ToFragments(f.hidden, h_frag, s.rows, s.hidden, stream);
      for (std::size_t l = 0; l < layers.size(); ++l) {
        const vx_dit_layer& layer = layers[l];
        float* keys = f.k_cache + l * layer_stride;
        float* values = f.v_cache + l * layer_stride;
        vx::fused::Qkv(h_frag, layer.input_norm, layer.qkv, qkv, s, stream);
        vx::kernels::QkvRope(qkv, rope, f.positions, f.cache_rows, q, keys, values, rows,
                             shape.heads, shape.kv_heads, shape.head_dim, f.capacity, stream);
        vx::stack::Attention(q, keys, values, attention_frag, true, attention_partials, rows,
                             f.rows_per_sequence, f.keys_per_sequence, past, f.causal,
                             shape.heads, shape.kv_heads, shape.head_dim, f.capacity, splits,
                             past_device, stream);
        vx::fused::Residual(attention_frag, layer.o, static_cast<int>(q_width), s.hidden,
                            h_frag, s, stream);
        vx::fused::GateUp(h_frag, layer.post_norm, layer.gate_up, swiglu_frag, s, stream);
        vx::fused::Residual(swiglu_frag, layer.down, s.ffn, s.hidden, h_frag, s, stream);
      }
      vx::stack::FromFragments(h_frag, f.hidden, s.rows, s.hidden, stream);
      vx::kernels::RmsNorm(f.hidden, weights.norm, bf16, f.output, rows, width, shape.eps,
                           stream);
      return vx::LaunchStatus("vx_stack_forward");
    }
    for (std::size_t l = 0; l < layers.size(); ++l) {
      const vx_dit_layer& layer = layers[l];
      float* keys = f.k_cache + l * layer_stride;
      float* values = f.v_cache + l * layer_stride;
      vx::kernels::RmsNorm(f.hidden, layer.input_norm, bf16, nullptr, rows, width, shape.eps,
                           stream);
      VX_TRY(Linear(bf16, layer.qkv, qkv, rows, width, qkv_width, false, stream));
      vx::kernels::QkvRope(qkv, rope, f.positions, f.cache_rows, q, keys, values, rows,
                           shape.heads, shape.kv_heads, shape.head_dim, f.capacity, stream);
      vx::stack::Attention(q, keys, values, bf16, false, attention_partials, rows,
                           f.rows_per_sequence, f.keys_per_sequence, past, f.causal,
                           shape.heads, shape.kv_heads, shape.head_dim, f.capacity, splits,
                           past_device, stream);
      VX_TRY(Linear(bf16, layer.o, f.hidden, rows, q_width, width, true, stream));
      vx::kernels::RmsNorm(f.hidden, layer.post_norm, bf16, nullptr, rows, width, shape.eps,
                           stream);
      VX_TRY(Linear(bf16, layer.gate_up, gate_up, rows, width, 2 * ffn, false, stream));
      vx::kernels::SwiGlu(gate_up, bf16, rows, ffn, stream);
      VX_TRY(Linear(bf16, layer.down, f.hidden, rows, ffn, width, true, stream));
    }
    vx::kernels::RmsNorm(f.hidden, weights.norm, bf16, f.output, rows, width, shape.eps,
                         stream);
    return vx::LaunchStatus("vx_stack_forward");
  }

  int Forward(const ForwardKey& f, std::size_t past) {
    const std::size_t rows = f.rows;
    const std::size_t sequences = rows / f.rows_per_sequence;
    // Up to 32 rows (decode steps, encoder patches: the same buffers call
    // after call) the launches replay as a graph captured on first use, one
    // per band of attended keys: its attention grid covers the band's
    // chunks and reads past from the device.
    hipStreamCaptureStatus capturing = hipStreamCaptureStatusNone;
    if (f.stream != nullptr)
      VX_HIP(hipStreamIsCapturing(f.stream, &capturing), "vx_stack_forward: capture status");
    const bool graphed = f.stream != nullptr && capturing == hipStreamCaptureStatusNone &&
                         rows <= vx::q8::kFragRows;
    // The keys the cache holds for the last sequence bound every band; the
    // partials are sized for them, so a new band never moves a buffer.
    const std::size_t most =
        f.capacity - (sequences - 1) * f.keys_per_sequence - f.rows_per_sequence;
    const std::size_t need = past + f.rows_per_sequence;
    const std::size_t banded =
        std::min(most, (need + kBandKeys - 1) / kBandKeys * kBandKeys - f.rows_per_sequence);
    const int splits = graphed ? vx::stack::AttentionSplits(banded, f.rows_per_sequence)
                               : vx::stack::AttentionSplits(past, f.rows_per_sequence);
    const std::size_t partials = vx::stack::AttentionPartialFloats(
        rows, shape.heads, shape.head_dim,
        graphed ? vx::stack::AttentionSplits(most, f.rows_per_sequence) : splits);
    const std::size_t wide = std::max({shape.hidden, qkv_width, shape.ffn});
    const char* what = "vx_stack_forward: hipMalloc";
    // Growing a buffer moves it: a graph that holds the old one is dropped.
    // (Products beyond 128 rows grow their own partials; those rows are
    // never replayed.)
    const void* before[] = {attention_partials, q, qkv, bf16, gate_up};
    VX_TRY(Grow(&attention_partials, &attention_partial_floats, partials, what));
    VX_TRY(Grow(&q, &q_floats, rows * q_width, what));
    VX_TRY(Grow(&qkv, &qkv_floats, rows * qkv_width, what));
    VX_TRY(Grow(&bf16, &bf16_count, rows * wide, what));
    VX_TRY(Grow(&gate_up, &gate_up_floats, rows * 2 * shape.ffn, what));
    const void* after[] = {attention_partials, q, qkv, bf16, gate_up};
    const bool moved = !std::equal(std::begin(before), std::end(before), std::begin(after));
    if (!graphed)
      return Launch(f, past, splits, nullptr, f.stream);

    vx::stack::SetPast(past_device, past, f.stream);
    if (moved || !(graph_key == f))
      DropGraphs();
    hipGraphExec_t graph = nullptr;
    for (const auto& entry : graphs)
      if (entry.first == splits)
        graph = entry.second;
    if (graph == nullptr) {
      VX_HIP(hipStreamBeginCapture(f.stream, hipStreamCaptureModeThreadLocal),
             "vx_stack_forward: begin capture");
      const int status = Launch(f, past, splits, past_device, f.stream);
      hipGraph_t captured = nullptr;
      const hipError_t ended = hipStreamEndCapture(f.stream, &captured);
      if (status != VX_OK) {
        if (captured != nullptr)
          (void)hipGraphDestroy(captured);
        return status;
      }
      if (ended != hipSuccess)
        return vx::FailHip(ended, "vx_stack_forward: end capture");
      const hipError_t instantiated = hipGraphInstantiate(&graph, captured, nullptr, nullptr, 0);
      (void)hipGraphDestroy(captured);
      if (instantiated != hipSuccess)
        return vx::FailHip(instantiated, "vx_stack_forward: instantiate");
      graph_key = f;
      graphs.emplace_back(splits, graph);
    }
    VX_HIP(hipGraphLaunch(graph, f.stream), "vx_stack_forward: graph launch");
    return vx::Succeed();
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
                    "vx_stack_create: attention takes head_dim 64 or 128 and 1, 2, 4, 8 "
                    "or 16 query heads per KV head");
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
  created->rows_fused = vx::stack::RowsSupported(shape->hidden, shape->ffn);
  int status = Allocate(&created->past_device, 1);
  if (status == VX_OK && created->fused) {
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
  ForwardKey f;
  f.hidden = hidden;
  f.output = output;
  f.rows = rows;
  f.positions = positions;
  f.cache_rows = cache_rows;
  f.rows_per_sequence = rows_per_sequence;
  f.keys_per_sequence = keys_per_sequence;
  f.causal = causal != 0;
  f.k_cache = k_cache;
  f.v_cache = v_cache;
  f.capacity = capacity;
  f.path = stack->Resolved(rows);
  f.stream = vx::Stream(stream);
  return stack->Forward(f, past);
}

void vx_stack_destroy(vx_stack* stack) { delete stack; }

int vx_stack_set_path(vx_stack* stack, int path) {
  if (stack == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_stack_set_path: null handle");
  if (path != VX_STACK_PATH_AUTO && path != VX_STACK_PATH_FUSED &&
      path != VX_STACK_PATH_UNFUSED && path != VX_STACK_PATH_ROWS)
    return vx::Fail(VX_BAD_ARG, "vx_stack_set_path: unknown path");
  if ((path == VX_STACK_PATH_FUSED && !stack->fused) ||
      (path == VX_STACK_PATH_ROWS && !stack->rows_fused))
    return vx::Fail(VX_UNSUPPORTED, "vx_stack_set_path: no such kernels for this shape");
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
                       capacity, splits, nullptr, vx::Stream(stream));
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
