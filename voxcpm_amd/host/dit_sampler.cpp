#include "dit_sampler.hpp"

#include <cstdint>
#include <exception>
#include <utility>

#include "voxcpm_amd.h"

namespace gufo::models::voxcpm {
namespace {

vx_dit_projection Panels(const Projection& projection, const char* name) {
  if (projection.weight.format != WeightFormat::kQ8Panels)
    throw GpuError(std::string(name) + " is not in Q8_0 panels");
  return vx_dit_projection{projection.weight.data, projection.bias};
}

}  // namespace

std::vector<EulerStep> EulerSchedule(std::size_t timesteps, float sway) {
  std::vector<float> t(timesteps), dt(timesteps);
  std::vector<std::int32_t> evaluate(timesteps);
  CheckVx(vx_euler_schedule(timesteps, sway, 1, t.data(), dt.data(),
                            evaluate.data()),
          "EulerSchedule");
  std::vector<EulerStep> steps(timesteps);
  for (std::size_t i = 0; i < timesteps; ++i)
    steps[i] = {t[i], dt[i], evaluate[i] != 0};
  return steps;
}

std::unique_ptr<DitSampler> DitSampler::Create(const DitConfig& config,
                                               const DitWeights& weights,
                                               std::string* error) {
  std::unique_ptr<DitSampler> sampler(new DitSampler());
  try {
    sampler->config_ = config;
    Check(hipStreamCreateWithFlags(&sampler->stream_, hipStreamNonBlocking),
          "hipStreamCreate");
    const TransformerConfig& stack = config.dit;
    if (weights.dit.layers.size() != stack.layers)
      throw GpuError("the DiT weights do not match its layer count");
    const std::size_t length = 3 + 2 * config.patch_size;
    const std::vector<float> rope = RopeTable(config.rope, length);
    sampler->rope_ = DeviceBuffer<float>(rope.size());
    Check(hipMemcpy(sampler->rope_.get(), rope.data(),
                    rope.size() * sizeof(float), hipMemcpyHostToDevice),
          "hipMemcpy rope");
    std::vector<vx_dit_layer> layers;
    for (const LayerWeights& layer : weights.dit.layers) {
      layers.push_back({layer.input_norm, Panels(layer.qkv, "qkv").weight,
                        Panels(layer.o, "o").weight, layer.post_norm,
                        Panels(layer.gate_up, "gate_up").weight,
                        Panels(layer.down, "down").weight});
    }
    vx_dit_shape shape{};
    shape.hidden = static_cast<std::uint32_t>(stack.hidden);
    shape.heads = static_cast<std::uint32_t>(stack.heads);
    shape.kv_heads = static_cast<std::uint32_t>(stack.kv_heads);
    shape.head_dim = static_cast<std::uint32_t>(stack.head_dim);
    shape.ffn = static_cast<std::uint32_t>(stack.intermediate);
    shape.layers = static_cast<std::uint32_t>(stack.layers);
    shape.patch = static_cast<std::uint32_t>(config.patch_size);
    shape.feat = static_cast<std::uint32_t>(config.feat_dim);
    shape.time_in = static_cast<std::uint32_t>(
        config.time_in != 0 ? config.time_in : stack.hidden);
    shape.has_delta = config.delta_time ? 1U : 0U;
    shape.eps = stack.rms_eps;
    vx_dit_weights device{};
    device.layers = layers.data();
    device.norm = weights.dit.norm;
    device.rope = stack.rope ? sampler->rope_.get() : nullptr;
    device.in_proj = Panels(weights.dit_in, "dit_in");
    device.cond_proj = Panels(weights.dit_cond, "dit_cond");
    device.out_proj = Panels(weights.dit_out, "dit_out");
    device.time_1 = Panels(weights.time_1, "time_1");
    device.time_2 = Panels(weights.time_2, "time_2");
    if (config.delta_time) {
      device.delta_1 = Panels(weights.delta_time_1, "delta_time_1");
      device.delta_2 = Panels(weights.delta_time_2, "delta_time_2");
    }
    CheckVx(vx_dit_create(&sampler->dit_, &shape, &device), "vx_dit_create");
    const std::size_t values = config.patch_size * config.feat_dim;
    sampler->mu_ = DeviceBuffer<float>(2 * stack.hidden);
    sampler->prefix_cond_ = DeviceBuffer<float>(values);
    sampler->x_ = DeviceBuffer<float>(values);
    sampler->velocity_ = DeviceBuffer<float>(2 * values);
    sampler->latent_ring_ = DeviceBuffer<float>(2 * values);
    Check(hipEventCreateWithFlags(&sampler->latent_event_,
                                  hipEventDisableTiming),
          "hipEventCreate");
  } catch (const std::exception& failure) {
    if (error != nullptr)
      *error = failure.what();
    return nullptr;
  }
  return sampler;
}

DitSampler::~DitSampler() {
  if (stream_ != nullptr)
    (void)hipStreamSynchronize(stream_);
  vx_dit_destroy(dit_);
  if (latent_event_ != nullptr)
    (void)hipEventDestroy(latent_event_);
  if (stream_ != nullptr)
    (void)hipStreamDestroy(stream_);
}

void DitSampler::Velocity(const float* mu, const float* cond, const float* x,
                          float t, float* velocity) {
  const std::size_t values = config_.patch_size * config_.feat_dim;
  Check(hipMemcpyAsync(mu_.get(), mu, 2 * config_.dit.hidden * sizeof(float),
                       hipMemcpyHostToDevice, stream_),
        "hipMemcpy mu");
  Check(hipMemcpyAsync(prefix_cond_.get(), cond, values * sizeof(float),
                       hipMemcpyHostToDevice, stream_),
        "hipMemcpy cond");
  Check(hipMemcpyAsync(x_.get(), x, values * sizeof(float),
                       hipMemcpyHostToDevice, stream_),
        "hipMemcpy x");
  CheckVx(vx_dit_velocity(dit_, mu_.get(), prefix_cond_.get(), x_.get(), t,
                          velocity_.get(), stream_),
          "vx_dit_velocity");
  Check(hipMemcpyAsync(velocity, velocity_.get(), 2 * values * sizeof(float),
                       hipMemcpyDeviceToHost, stream_),
        "hipMemcpy velocity");
  Check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
}

void DitSampler::Sample(const float* mu, const float* prefix_cond,
                        const float* noise, std::size_t timesteps, float cfg,
                        float* latent, const SamplerOptions& options) {
  const std::size_t values = config_.patch_size * config_.feat_dim;
  std::vector<float> t(timesteps), dt(timesteps);
  std::vector<std::int32_t> evaluate(timesteps);
  CheckVx(vx_euler_schedule(timesteps, options.sway,
                            options.skip_first ? 1 : 0, t.data(), dt.data(),
                            evaluate.data()),
          "EulerSchedule");
  Check(hipMemcpyAsync(mu_.get(), mu, 2 * config_.dit.hidden * sizeof(float),
                       hipMemcpyHostToDevice, stream_),
        "hipMemcpy mu");
  Check(hipMemcpyAsync(prefix_cond_.get(), prefix_cond, values * sizeof(float),
                       hipMemcpyHostToDevice, stream_),
        "hipMemcpy prefix");
  Check(hipMemcpyAsync(x_.get(), noise, values * sizeof(float),
                       hipMemcpyHostToDevice, stream_),
        "hipMemcpy noise");
  CheckVx(vx_dit_patch(dit_, mu_.get(), prefix_cond_.get(), x_.get(), t.data(),
                       dt.data(), evaluate.data(), timesteps, cfg,
                       options.cfg_zero_star ? 1 : 0, stream_),
          "vx_dit_patch");
  float* slot = latent_ring_.get() + (steps_taken_ % 2) * values;
  Check(hipMemcpyAsync(slot, x_.get(), values * sizeof(float),
                       hipMemcpyDeviceToDevice, stream_),
        "hipMemcpy latent");
  Check(hipEventRecord(latent_event_, stream_), "hipEventRecord");
  latent_slot_ = slot;
  if (latent != nullptr)
    Check(hipMemcpyAsync(latent, x_.get(), values * sizeof(float),
                         hipMemcpyDeviceToHost, stream_),
          "hipMemcpy latent");
  if (trace_ != nullptr) {
    std::vector<float> used(2 * config_.dit.hidden);
    Check(hipMemcpyAsync(used.data(), mu_.get(), used.size() * sizeof(float),
                         hipMemcpyDeviceToHost, stream_),
          "hipMemcpy trace");
    trace_->mu.push_back(std::move(used));
  }
  Check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
  ++steps_taken_;
}

}  // namespace gufo::models::voxcpm
