// The local-DiT half of VoxCPM2's Generator (generator.hpp:34-179 of the
// reference) as its own class, DitSampler, over the voxcpm_amd C ABI. It is
// not the reference's Generator: that class also owns the text-semantic and
// residual LMs, the local encoder, FSQ and the stop head, which produce the
// DiT's condition `mu` and consume its latent; those stay in the reference.
// What matches the reference exactly: EulerSchedule (generator.hpp:34-44),
// EulerStep, Velocity's signature (generator.hpp:90-91), latent() and
// latent_event() (generator.hpp:85-86). What differs: Create takes the DiT's
// shape and device weights instead of Config and ModelFiles, and Sample
// takes mu and the previous patch as arguments where the reference's
// Step(noise, timesteps, cfg, latent, stop_logits) reads them from its LM
// state and also writes the stop logits.
#ifndef VOXCPM_AMD_HOST_DIT_SAMPLER_HPP_
#define VOXCPM_AMD_HOST_DIT_SAMPLER_HPP_

#include <hip/hip_runtime.h>

#include <cstddef>
#include <memory>
#include <string>
#include <vector>

#include "device.hpp"
#include "transformer.hpp"

struct vx_dit;

namespace gufo::models::voxcpm {

/// The Euler steps of UnifiedCFM.solve_euler with the sway-sampled
/// schedule in float32; CFG-Zero* leaves the first
/// max(1, int(0.04 (n + 1))) steps at zero velocity (generator.hpp:34-44).
struct EulerStep {
  float t = 0.0F;
  float dt = 0.0F;
  bool evaluate = true;
};
[[nodiscard]] std::vector<EulerStep> EulerSchedule(std::size_t timesteps,
                                                   float sway = 1.0F);

/// The DiT's shape: its stack, RoPE and the patch it samples.
struct DitConfig {
  TransformerConfig dit;
  RopeConfig rope;
  std::size_t patch_size = 4;
  std::size_t feat_dim = 64;
  std::size_t time_in = 0;  // sinusoid width (the reference: dit.hidden)
  bool delta_time = true;   // add delta_time_mlp(sinusoid(0))
};

/// The DiT's weights on the device (the reference's GeneratorWeights
/// subset, weights.hpp:48-71); every matrix in Q8_0 panels.
struct DitWeights {
  StackWeights dit;
  Projection dit_in;
  Projection dit_cond;
  Projection dit_out;
  Projection time_1;
  Projection time_2;
  Projection delta_time_1;
  Projection delta_time_2;
};

/// How the sampler guides: the reference's sway schedule with CFG-Zero*
/// (the defaults), or a uniform schedule with plain CFG (sway 0, no skip,
/// cfg_zero_star false).
struct SamplerOptions {
  float sway = 1.0F;
  bool skip_first = true;
  bool cfg_zero_star = true;
};

/// Intermediate tensors for tests, copied to the host while tracing: the
/// DiT's part of the reference's Trace (generator.hpp:47-53), the condition
/// mu [2 hidden] of every Sample call as the device held it when the patch
/// ran (the reference records it per Step).
struct SamplerTrace {
  std::vector<std::vector<float>> mu;
};

/// The local DiT with its CFM sampler on one non-blocking stream. One
/// sequence at a time; not thread-safe (the reference's Generator,
/// generator.hpp:55-58, has the same rule).
class DitSampler {
public:
  /// nullptr and the message in `error` on failure, as the reference's
  /// Generator::Create reports (generator.cpp:168-172).
  [[nodiscard]] static std::unique_ptr<DitSampler> Create(
      const DitConfig& config, const DitWeights& weights,
      std::string* error = nullptr);
  ~DitSampler();
  DitSampler(const DitSampler&) = delete;
  DitSampler& operator=(const DitSampler&) = delete;

  [[nodiscard]] const DitConfig& config() const { return config_; }
  [[nodiscard]] hipStream_t stream() const { return stream_; }

  /// The CFG pair of velocities [2][patch_size][feat_dim] of one evaluation
  /// at time t; host arrays mu [2 hidden], cond and x [patch][feat]
  /// (generator.hpp:87-91).
  void Velocity(const float* mu, const float* cond, const float* x, float t,
                float* velocity);

  /// The sampler inside the reference's Generator::Step
  /// (generator.cpp:448-469): the patch from `noise` with `timesteps` Euler
  /// steps and guidance `cfg`, conditioned on `mu` and the previous patch
  /// `prefix_cond` (host arrays). Writes the latent [patch][feat] to
  /// `latent` when not null; it also stays on the device: latent() until
  /// the call after next, ready once latent_event() completes.
  void Sample(const float* mu, const float* prefix_cond, const float* noise,
              std::size_t timesteps, float cfg, float* latent,
              const SamplerOptions& options = SamplerOptions());

  [[nodiscard]] const float* latent() const { return latent_slot_; }
  [[nodiscard]] hipEvent_t latent_event() const { return latent_event_; }

  /// Copies intermediate tensors into `trace` while set, null to stop
  /// (tests; generator.hpp:93-94).
  void set_trace(SamplerTrace* trace) { trace_ = trace; }

private:
  DitSampler() = default;

  DitConfig config_;
  hipStream_t stream_ = nullptr;
  ::vx_dit* dit_ = nullptr;
  DeviceBuffer<float> rope_;
  DeviceBuffer<float> mu_;
  DeviceBuffer<float> prefix_cond_;
  DeviceBuffer<float> x_;
  DeviceBuffer<float> velocity_;
  DeviceBuffer<float> latent_ring_;
  const float* latent_slot_ = nullptr;
  std::size_t steps_taken_ = 0;
  hipEvent_t latent_event_ = nullptr;
  SamplerTrace* trace_ = nullptr;
};

}  // namespace gufo::models::voxcpm

#endif  // VOXCPM_AMD_HOST_DIT_SAMPLER_HPP_
