// The MiniCPM4 stack of the reference (transformer.hpp:17-76) with its
// configuration and weight types (config.hpp:15-51, weights.hpp:20-41),
// the subset the local DiT needs, over the voxcpm_amd C ABI.
#ifndef VOXCPM_AMD_HOST_TRANSFORMER_HPP_
#define VOXCPM_AMD_HOST_TRANSFORMER_HPP_

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <vector>

#include "device.hpp"
#include "gemm.hpp"
#include "matrix.hpp"

namespace gufo::models::voxcpm {

/// Raw bfloat16 bits.
using Bf16 = std::uint16_t;

/// One MiniCPM4 stack (config.hpp:15-31).
struct TransformerConfig {
  std::size_t hidden = 0;
  std::size_t intermediate = 0;
  std::size_t layers = 0;
  std::size_t heads = 0;
  std::size_t kv_heads = 0;
  std::size_t head_dim = 0;
  float rms_eps = 0.0F;
  bool rope = true;
};

/// MiniCPM's LongRoPE (config.hpp:37-51): the factors the reference applies
/// and the magnitude scale of the table.
struct RopeConfig {
  double theta = 10000.0;
  std::size_t dim = 0;
  std::vector<double> factors;  // dim / 2 values; empty = all 1
  double scaling = 1.0;
};

/// A linear layer y = x W^T (+ b) (weights.hpp:20-26).
struct Projection {
  Matrix weight;
  const Bf16* bias = nullptr;
  std::size_t in = 0;
  std::size_t out = 0;
};

struct LayerWeights {
  const Bf16* input_norm = nullptr;
  Projection qkv;  // [q heads | k heads | v heads]
  Projection o;
  const Bf16* post_norm = nullptr;
  Projection gate_up;  // [gate | up]
  Projection down;
};

struct StackWeights {
  TransformerConfig config;
  std::vector<LayerWeights> layers;
  const Bf16* norm = nullptr;
};

/// Keys and values of one stack: [layer][kv_head][capacity][head_dim] each
/// (transformer.hpp:18-36).
class KvCache {
public:
  KvCache() = default;
  KvCache(const TransformerConfig& config, std::size_t capacity);

  [[nodiscard]] std::size_t capacity() const { return capacity_; }
  [[nodiscard]] float* keys(std::size_t layer) const {
    return keys_.get() + layer * layer_stride_;
  }
  [[nodiscard]] float* values(std::size_t layer) const {
    return values_.get() + layer * layer_stride_;
  }

private:
  DeviceBuffer<float> keys_;
  DeviceBuffer<float> values_;
  std::size_t capacity_ = 0;
  std::size_t layer_stride_ = 0;
};

/// Which keys each row attends to (transformer.hpp:41-48).
struct AttentionLayout {
  const std::int32_t* positions = nullptr;
  const std::int32_t* cache_rows = nullptr;
  std::size_t rows_per_sequence = 0;
  std::size_t keys_per_sequence = 0;
  std::size_t past = 0;
  bool causal = true;
};

/// The vx_stack handles ForwardStack runs, one per stack (by its first
/// layer's qkv weights) and rotary table; destroyed with the scratch.
class NativeStacks {
public:
  NativeStacks() = default;
  NativeStacks(const NativeStacks&) = delete;
  NativeStacks& operator=(const NativeStacks&) = delete;
  ~NativeStacks();

  /// The handle of `stack` with `rope` (created on first use), or null when
  /// its weights are in a format vx_stack does not take (rows, tiles,
  /// biases): ForwardStack then runs its kernels one by one.
  vx_stack* Get(const StackWeights& stack, const float* rope);

private:
  struct Entry {
    const void* key = nullptr;
    const float* rope = nullptr;
    vx_stack* handle = nullptr;
  };
  std::vector<Entry> entries_;
};

/// Scratch shared by the stacks (transformer.hpp:51-58).
struct StackScratch {
  DeviceBuffer<Bf16> normed;
  DeviceBuffer<float> qkv;
  DeviceBuffer<float> q;
  DeviceBuffer<Bf16> attention;
  DeviceBuffer<float> gate_up;
  DeviceBuffer<Bf16> activation;
  NativeStacks native;
};

/// The rotary table [position][cos (dim / 2) | sin (dim / 2)] in float32
/// (transformer.hpp:62-63).
[[nodiscard]] std::vector<float> RopeTable(const RopeConfig& rope,
                                           std::size_t positions);

/// One stack over `rows` rows of the float32 residual `hidden` (updated in
/// place); the final norm's float32 output goes to `output`
/// (transformer.hpp:69-72). Stacks of Q8_0 or bf16 panels without biases
/// run as one vx_stack_forward call (fused launches, one HIP graph up to 32
/// rows); others run the reference's launch sequence.
void ForwardStack(const StackWeights& stack, const float* rope,
                  const AttentionLayout& layout, KvCache& cache, float* hidden,
                  float* output, std::size_t rows, StackScratch& scratch,
                  Bf16Gemm& gemm, hipStream_t stream);

/// y[rows][out] = x[rows][in] W^T + b with bf16 x (transformer.hpp:75-76).
void Project(const Projection& projection, const Bf16* x, float* y,
             std::size_t rows, Bf16Gemm& gemm, hipStream_t stream);

}  // namespace gufo::models::voxcpm

#endif  // VOXCPM_AMD_HOST_TRANSFORMER_HPP_
