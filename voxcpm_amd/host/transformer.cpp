#include "transformer.hpp"

#include "voxcpm_amd.h"

namespace gufo::models::voxcpm {

KvCache::KvCache(const TransformerConfig& config, std::size_t capacity)
    : capacity_(capacity),
      layer_stride_(config.kv_heads * capacity * config.head_dim) {
  keys_ = DeviceBuffer<float>(config.layers * layer_stride_);
  values_ = DeviceBuffer<float>(config.layers * layer_stride_);
}

std::vector<float> RopeTable(const RopeConfig& rope, std::size_t positions) {
  std::vector<float> table(positions * rope.dim);
  CheckVx(vx_rope_table(rope.theta, rope.dim,
                        rope.factors.empty() ? nullptr : rope.factors.data(),
                        static_cast<float>(rope.scaling), positions,
                        table.data()),
          "RopeTable");
  return table;
}

void Project(const Projection& projection, const Bf16* x, float* y,
             std::size_t rows, Bf16Gemm& gemm, hipStream_t stream) {
  gemm.Linear(x, projection.weight, y, rows, projection.in, projection.out,
              false);
  if (projection.bias != nullptr)
    CheckVx(vx_add_bias(y, projection.bias, rows, projection.out, stream),
            "Project bias");
}

NativeStacks::~NativeStacks() {
  for (const Entry& entry : entries_)
    vx_stack_destroy(entry.handle);
}

vx_stack* NativeStacks::Get(const StackWeights& stack, const float* rope) {
  if (stack.layers.empty())
    return nullptr;
  const void* key = stack.layers.front().qkv.weight.data;
  for (const Entry& entry : entries_)
    if (entry.key == key && entry.rope == rope)
      return entry.handle;
  const WeightFormat format = stack.layers.front().qkv.weight.format;
  if (format != WeightFormat::kQ8Panels && format != WeightFormat::kBf16Panels)
    return nullptr;
  std::vector<vx_dit_layer> layers;
  for (const LayerWeights& layer : stack.layers) {
    for (const Projection* p : {&layer.qkv, &layer.o, &layer.gate_up, &layer.down})
      if (p->weight.format != format || p->bias != nullptr)
        return nullptr;
    layers.push_back({layer.input_norm, layer.qkv.weight.data, layer.o.weight.data,
                      layer.post_norm, layer.gate_up.weight.data, layer.down.weight.data});
  }
  const TransformerConfig& c = stack.config;
  const bool rotary = c.rope && rope != nullptr;
  const vx_stack_shape shape{c.hidden, c.heads, c.kv_heads, c.head_dim, c.intermediate,
                             stack.layers.size(), c.rms_eps, rotary ? 1 : 0};
  const vx_stack_weights weights{
      layers.data(), stack.norm, rotary ? rope : nullptr,
      format == WeightFormat::kQ8Panels ? static_cast<std::uint32_t>(VX_WEIGHTS_Q8_0)
                                        : static_cast<std::uint32_t>(VX_WEIGHTS_BF16)};
  vx_stack* handle = nullptr;
  if (vx_stack_create(&handle, &shape, &weights) != VX_OK)
    return nullptr;  // a shape the native stack does not take
  entries_.push_back({key, rope, handle});
  return handle;
}

void ForwardStack(const StackWeights& stack, const float* rope,
                  const AttentionLayout& layout, KvCache& cache, float* hidden,
                  float* output, std::size_t rows, StackScratch& scratch,
                  Bf16Gemm& gemm, hipStream_t stream) {
  if (vx_stack* native = scratch.native.Get(stack, rope)) {
    CheckVx(vx_stack_forward(native, hidden, output, rows, layout.positions,
                             layout.cache_rows, layout.rows_per_sequence,
                             layout.keys_per_sequence, layout.past, layout.causal ? 1 : 0,
                             cache.keys(0), cache.values(0), cache.capacity(), stream),
            "ForwardStack");
    return;
  }
  // transformer.cpp:55-100: 12x [RMSNorm, qkv, RoPE + cache, attention,
  // o (+residual), RMSNorm, gate_up, SwiGLU, down (+residual)], final norm.
  const TransformerConfig& config = stack.config;
  const std::size_t width = config.hidden;
  const std::size_t q_width = config.heads * config.head_dim;
  const std::size_t qkv_width =
      (config.heads + 2 * config.kv_heads) * config.head_dim;
  scratch.normed.Reserve(rows * width);
  scratch.qkv.Reserve(rows * qkv_width);
  scratch.q.Reserve(rows * q_width);
  scratch.attention.Reserve(rows * q_width);
  scratch.gate_up.Reserve(rows * 2 * config.intermediate);
  scratch.activation.Reserve(rows * config.intermediate);
  for (std::size_t index = 0; index < stack.layers.size(); ++index) {
    const LayerWeights& layer = stack.layers[index];
    CheckVx(vx_rms_norm(hidden, layer.input_norm, scratch.normed.get(),
                        nullptr, rows, width, config.rms_eps, stream),
            "RmsNorm");
    gemm.Linear(scratch.normed.get(), layer.qkv.weight, scratch.qkv.get(),
                rows, width, qkv_width, false);
    CheckVx(vx_qkv_rope(scratch.qkv.get(), config.rope ? rope : nullptr,
                        layout.positions, layout.cache_rows, scratch.q.get(),
                        cache.keys(index), cache.values(index), rows,
                        config.heads, config.kv_heads, config.head_dim,
                        cache.capacity(), stream),
            "QkvRope");
    CheckVx(vx_attention(scratch.q.get(), cache.keys(index),
                         cache.values(index), scratch.attention.get(), rows,
                         layout.rows_per_sequence, layout.keys_per_sequence,
                         layout.past, layout.causal ? 1 : 0, config.heads,
                         config.kv_heads, config.head_dim, cache.capacity(),
                         stream),
            "Attention");
    gemm.Linear(scratch.attention.get(), layer.o.weight, hidden, rows, q_width,
                width, true);
    CheckVx(vx_rms_norm(hidden, layer.post_norm, scratch.normed.get(), nullptr,
                        rows, width, config.rms_eps, stream),
            "RmsNorm");
    gemm.Linear(scratch.normed.get(), layer.gate_up.weight,
                scratch.gate_up.get(), rows, width, 2 * config.intermediate,
                false);
    CheckVx(vx_swiglu(scratch.gate_up.get(), scratch.activation.get(), rows,
                      config.intermediate, stream),
            "SwiGlu");
    gemm.Linear(scratch.activation.get(), layer.down.weight, hidden, rows,
                config.intermediate, width, true);
  }
  CheckVx(vx_rms_norm(hidden, stack.norm, scratch.normed.get(), output, rows,
                      width, config.rms_eps, stream),
          "RmsNorm");
}

}  // namespace gufo::models::voxcpm
