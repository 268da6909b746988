// The C++ host surface (Bf16Gemm::Linear, DitSampler::Velocity,
// DitSampler::Sample and ForwardStack over the voxcpm_amd C ABI) against the
// CPU oracle, in the
// style of the reference's tests/products_test.cpp and
// tests/generator_test.cpp: random GGML Q8_0 weights, products compared with
// a double-precision sum relative to sum |x w| (limit 1e-5; 1e-4 for the
// expanded path beyond 128 rows), one DiT evaluation and one sampled patch
// against the oracle (max |d| / max |ref| <= 1e-2). Exit 77 without a GPU.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <iostream>
#include <sstream>
#include <string>
#include <vector>

#include "../../oracle/oracle.h"
#include "../../voxcpm_amd/host/dit_sampler.hpp"
#include "voxcpm_amd.h"
#include "voxcpm_amd_internal.h"

namespace vc = gufo::models::voxcpm;

namespace {

constexpr int kSkip = 77;
int failures = 0;

/// splitmix64 with Box-Muller (the tests' own generator).
class Random {
public:
  explicit Random(std::uint64_t seed) : state_(seed) {}
  std::uint64_t Bits() {
    std::uint64_t z = (state_ += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
  }
  double Uniform() { return static_cast<double>(Bits() >> 11) * 0x1.0p-53; }
  double Normal() {
    const double u1 = Uniform();
    const double u2 = Uniform();
    return std::sqrt(-2.0 * std::log1p(-u1)) * std::cos(2.0 * M_PI * u2);
  }

private:
  std::uint64_t state_;
};

/// GGML Q8_0 blocks as in products_test.cpp:65-86 (q in [-128, 127], scale
/// bits in [0x1000, 0x1C00]).
std::vector<std::uint8_t> Weights(std::size_t out, std::size_t in,
                                  Random& rng) {
  std::vector<std::uint8_t> blocks(out * in / 32 * 34);
  for (std::size_t b = 0; b < out * in / 32; ++b) {
    const auto bits = static_cast<std::uint16_t>(0x1000 + rng.Bits() % 0xC01);
    blocks[b * 34] = static_cast<std::uint8_t>(bits & 0xFF);
    blocks[b * 34 + 1] = static_cast<std::uint8_t>(bits >> 8);
    for (int i = 0; i < 32; ++i)
      blocks[b * 34 + 2 + i] = static_cast<std::uint8_t>(rng.Bits() & 0xFF);
  }
  return blocks;
}

/// GGML Q8_0 blocks with the DiT workload's law: q uniform in [-127, 127],
/// scale fp16(|N(0, 0.02)| / 127), subnormals kept.
std::vector<std::uint8_t> ModelWeights(std::size_t out, std::size_t in,
                                       Random& rng) {
  std::vector<std::uint8_t> blocks(out * in / 32 * 34);
  for (std::size_t b = 0; b < out * in / 32; ++b) {
    const std::uint16_t bits = vo_half_bits(
        static_cast<float>(std::fabs(rng.Normal() * 0.02) / 127.0));
    blocks[b * 34] = static_cast<std::uint8_t>(bits & 0xFF);
    blocks[b * 34 + 1] = static_cast<std::uint8_t>(bits >> 8);
    for (int i = 0; i < 32; ++i)
      blocks[b * 34 + 2 + i] = static_cast<std::uint8_t>(
          static_cast<std::int8_t>(static_cast<int>(rng.Bits() % 255) - 127));
  }
  return blocks;
}

std::vector<std::uint16_t> Activations(std::size_t rows, std::size_t in,
                                       Random& rng, double std) {
  std::vector<std::uint16_t> x(rows * in);
  for (auto& v : x)
    v = vo_bf16_bits(static_cast<float>(rng.Normal() * std));
  return x;
}

template<typename T>
vc::DeviceBuffer<T> Upload(const std::vector<T>& host) {
  vc::DeviceBuffer<T> device(host.size());
  vc::Check(hipMemcpy(device.get(), host.data(), host.size() * sizeof(T),
                      hipMemcpyHostToDevice),
            "upload");
  return device;
}

template<typename T>
std::vector<T> Download(const T* device, std::size_t count) {
  std::vector<T> host(count);
  vc::Check(hipMemcpy(host.data(), device, count * sizeof(T),
                      hipMemcpyDeviceToHost),
            "download");
  return host;
}

vc::DeviceBuffer<std::uint8_t> Pack(const std::vector<std::uint8_t>& blocks,
                                    std::size_t out, std::size_t in) {
  auto raw = Upload(blocks);
  vc::DeviceBuffer<std::uint8_t> packed(vx_q8_packed_bytes(out, in));
  vc::CheckVx(vx_q8_pack(raw.get(), out, in, packed.get(), nullptr), "pack");
  vc::Check(hipDeviceSynchronize(), "sync");
  return packed;
}

std::string Scientific(double value) {
  std::ostringstream out;
  out << std::scientific << value;
  return out.str();
}

void Report(bool ok, const std::string& line) {
  std::cout << (ok ? "ok   " : "FAIL ") << line << "\n";
  if (!ok)
    ++failures;
}

/// Error of y against x . bf16(scale q) in double, relative to sum |x w|
/// (the expansion of more than 128 rows, products_test.cpp:301-309).
double ExpandedError(const std::vector<float>& y,
                     const std::vector<std::uint16_t>& x,
                     const std::vector<std::uint8_t>& blocks,
                     const std::vector<float>* before, std::size_t rows,
                     std::size_t in, std::size_t out) {
  std::vector<std::uint16_t> w(out * in);
  vo_q8_dequant_bf16(blocks.data(), out, in, w.data());
  double worst = 0.0;
  for (std::size_t m = 0; m < rows; ++m)
    for (std::size_t n = 0; n < out; ++n) {
      double exact = before != nullptr ? (*before)[m * out + n] : 0.0;
      double magnitude = 0.0;
      for (std::size_t k = 0; k < in; ++k) {
        const double p = static_cast<double>(vo_bf16_value(x[m * in + k])) *
                         vo_bf16_value(w[n * in + k]);
        exact += p;
        magnitude += std::fabs(p);
      }
      worst = std::max(worst, std::fabs(y[m * out + n] - exact) /
                                  std::max(magnitude, 1e-30));
    }
  return worst;
}

/// Bf16Gemm::Linear on panels at rows 1, 22, 40 and 130, with and without
/// accumulation (products_test.cpp:256-313).
void TestLinear(std::size_t in, std::size_t out, Random& rng,
                hipStream_t stream) {
  const auto blocks = Weights(out, in, rng);
  const auto packed = Pack(blocks, out, in);
  vc::Bf16Gemm gemm(nullptr, stream);
  vc::Matrix matrix{vc::WeightFormat::kQ8Panels, packed.get()};
  for (const std::size_t rows : {1, 22, 40, 130}) {
    const auto x = Activations(rows, in, rng, 2.0);
    const auto x_device = Upload(x);
    std::vector<float> before(rows * out);
    for (auto& v : before)
      v = static_cast<float>(rng.Normal());
    vc::DeviceBuffer<float> y(rows * out);
    for (const bool accumulate : {false, true}) {
      vc::Check(hipMemcpy(y.get(), before.data(), before.size() * sizeof(float),
                          hipMemcpyHostToDevice),
                "upload");
      gemm.Linear(x_device.get(), matrix, y.get(), rows, in, out, accumulate);
      vc::Check(hipStreamSynchronize(stream), "sync");
      const auto result = Download(y.get(), y.size());
      const double worst =
          rows > 128
              ? ExpandedError(result, x, blocks, accumulate ? &before : nullptr,
                              rows, in, out)
              : vo_q8_check(result.data(), x.data(), blocks.data(),
                            accumulate ? before.data() : nullptr, rows, in,
                            out);
      const double limit = rows > 128 ? 1e-4 : 1e-5;
      Report(worst <= limit,
             "linear q8 panels rows " + std::to_string(rows) + " in " +
                 std::to_string(in) + " out " + std::to_string(out) +
                 (accumulate ? " (accumulate)" : "") + ": worst " +
                 Scientific(worst));
    }
  }
  // A format this build does not serve throws GpuError.
  bool threw = false;
  try {
    gemm.Linear(nullptr, vc::Matrix{vc::WeightFormat::kBf16Tiles, packed.get()},
                nullptr, 1, in, out, false);
  } catch (const vc::GpuError&) {
    threw = true;
  }
  Report(threw, "unsupported weight format throws GpuError");
}

/// Bf16Gemm::Linear of 320 x 6144 x 2048 takes the expanded path's plan
/// that splits k (its grid has few tiles): the operator's scratch holds the
/// split's partial sums, as the reference's State owns its partials
/// (gemm.cpp:95-98). The result is bit for bit vx_q8_linear's with a
/// scratch that size, whose plan splits (and without one would not), and
/// within 1e-4 of the expanded arithmetic (products_test.cpp:301-309).
void TestPrefillSplit(Random& rng, hipStream_t stream) {
  const std::size_t rows = 320, in = 6144, out = 2048;
  const auto blocks = Weights(out, in, rng);
  const auto packed = Pack(blocks, out, in);
  const auto x = Activations(rows, in, rng, 2.0);
  const auto x_device = Upload(x);
  vx_scratch* scratch = nullptr;
  vc::CheckVx(vx_scratch_create(&scratch, 128, VX_PREFILL_SPLIT_FLOATS / (16 * 128)),
              "scratch");
  std::int32_t plan[4] = {0, 0, 0, 0};
  std::int32_t bare[4] = {0, 0, 0, 0};
  vc::CheckVx(vx_q8_prefill_plan(rows, in, out, scratch, plan), "plan");
  vc::CheckVx(vx_q8_prefill_plan(rows, in, out, nullptr, bare), "plan");
  Report(plan[3] > 1 && bare[3] == 1,
         "prefill 320 x 6144 x 2048 plan: " + std::to_string(plan[3]) +
             " splits with the scratch, " + std::to_string(bare[3]) + " without");
  vc::DeviceBuffer<float> y(rows * out);
  vc::DeviceBuffer<float> reference(rows * out);
  vc::Bf16Gemm gemm(nullptr, stream);
  gemm.Linear(x_device.get(), vc::Matrix{vc::WeightFormat::kQ8Panels, packed.get()}, y.get(),
              rows, in, out, false);
  vc::CheckVx(vx_q8_linear(x_device.get(), packed.get(), reference.get(), rows, in, out, 0,
                           scratch, stream),
              "vx_q8_linear");
  vc::Check(hipStreamSynchronize(stream), "sync");
  vx_scratch_destroy(scratch);
  const auto result = Download(y.get(), y.size());
  const auto expected = Download(reference.get(), reference.size());
  Report(std::memcmp(result.data(), expected.data(), result.size() * sizeof(float)) == 0,
         "Bf16Gemm::Linear 320 x 6144 x 2048 equals the split plan's product bit for bit");
  const double worst = ExpandedError(result, x, blocks, nullptr, rows, in, out);
  Report(worst <= 1e-4, "Bf16Gemm::Linear 320 x 6144 x 2048 (split k): worst " +
                            Scientific(worst));
}

/// Bf16Gemm::Linear on bf16 weights, as panels and as rows, at rows 1, 22,
/// 40 and 130 (products_test.cpp:256-313 with kBf16Tiles): the bf16
/// expansion of Q8_0 weights, error relative to sum |x w| <= 1e-5.
void TestLinearBf16(std::size_t in, std::size_t out, Random& rng,
                    hipStream_t stream) {
  const auto blocks = Weights(out, in, rng);
  std::vector<std::uint16_t> w(out * in);
  vo_q8_dequant_bf16(blocks.data(), out, in, w.data());
  const auto rows_w = Upload(w);
  vc::DeviceBuffer<std::uint8_t> panels(vx_bf16_packed_bytes(out, in));
  vc::CheckVx(vx_bf16_pack(rows_w.get(), out, in, panels.get(), nullptr), "pack");
  vc::Check(hipDeviceSynchronize(), "sync");
  vc::Bf16Gemm gemm(nullptr, stream);
  for (const vc::WeightFormat format : {vc::WeightFormat::kBf16Panels, vc::WeightFormat::kBf16}) {
    const vc::Matrix matrix{format, format == vc::WeightFormat::kBf16
                                        ? static_cast<const void*>(rows_w.get())
                                        : static_cast<const void*>(panels.get())};
    for (const std::size_t rows : {1, 22, 40, 130}) {
      const auto x = Activations(rows, in, rng, 2.0);
      const auto x_device = Upload(x);
      std::vector<float> before(rows * out);
      for (auto& v : before)
        v = static_cast<float>(rng.Normal());
      vc::DeviceBuffer<float> y(rows * out);
      for (const bool accumulate : {false, true}) {
        vc::Check(hipMemcpy(y.get(), before.data(), before.size() * sizeof(float),
                            hipMemcpyHostToDevice),
                  "upload");
        gemm.Linear(x_device.get(), matrix, y.get(), rows, in, out, accumulate);
        vc::Check(hipStreamSynchronize(stream), "sync");
        const auto result = Download(y.get(), y.size());
        const double worst = vo_bf16_check(result.data(), x.data(), w.data(),
                                           accumulate ? before.data() : nullptr, rows, in, out);
        Report(worst <= 1e-5,
               std::string("linear bf16 ") +
                   (format == vc::WeightFormat::kBf16 ? "rows" : "panels") + " rows " +
                   std::to_string(rows) + " in " + std::to_string(in) + " out " +
                   std::to_string(out) + (accumulate ? " (accumulate)" : "") + ": worst " +
                   Scientific(worst));
      }
    }
  }
}

/// A small DiT of the released model's shape (GQA, head_dim 128, LongRoPE
/// off for brevity: factors 1) with two layers.
struct SmallDit {
  vc::DitConfig config;
  std::vector<std::vector<std::uint8_t>> matrices;  // host GGML blocks
  std::vector<std::vector<std::uint16_t>> vectors;  // host bf16
  std::vector<vc::DeviceBuffer<std::uint8_t>> packed;
  std::vector<vc::DeviceBuffer<std::uint16_t>> device_vectors;
  vc::DitWeights weights;
  std::vector<vo_layer> oracle_layers;
  vo_dit oracle{};
  std::vector<float> rope;

  explicit SmallDit(Random& rng) {
    vc::TransformerConfig& s = config.dit;
    s.hidden = 256;
    s.intermediate = 512;
    s.layers = 2;
    s.heads = 4;
    s.kv_heads = 2;
    s.head_dim = 128;
    s.rms_eps = 1e-5F;
    config.rope.dim = 128;
    config.patch_size = 4;
    config.feat_dim = 64;
    config.time_in = 256;
    config.delta_time = true;
    matrices.reserve(64);
    vectors.reserve(64);
    packed.reserve(64);
    device_vectors.reserve(64);
    const auto matrix = [&](std::size_t out, std::size_t in) {
      matrices.push_back(ModelWeights(out, in, rng));
      packed.push_back(Pack(matrices.back(), out, in));
      return vc::Matrix{vc::WeightFormat::kQ8Panels, packed.back().get()};
    };
    const auto vector = [&](std::size_t count, double mean, double std) {
      std::vector<std::uint16_t> v(count);
      for (auto& x : v)
        x = vo_bf16_bits(static_cast<float>(mean + std * rng.Normal()));
      vectors.push_back(v);
      device_vectors.push_back(Upload(v));
      return static_cast<const vc::Bf16*>(device_vectors.back().get());
    };
    const auto projection = [&](std::size_t out, std::size_t in) {
      vc::Projection p;
      p.weight = matrix(out, in);
      p.bias = vector(out, 0.0, 0.02);
      p.in = in;
      p.out = out;
      return p;
    };
    const std::size_t h = s.hidden;
    const std::size_t qkv = (s.heads + 2 * s.kv_heads) * s.head_dim;
    weights.dit.config = s;
    for (std::size_t l = 0; l < s.layers; ++l) {
      vc::LayerWeights layer;
      layer.input_norm = vector(h, 1.0, 0.02);
      layer.qkv.weight = matrix(qkv, h);
      layer.o.weight = matrix(h, s.heads * s.head_dim);
      layer.post_norm = vector(h, 1.0, 0.02);
      layer.gate_up.weight = matrix(2 * s.intermediate, h);
      layer.down.weight = matrix(h, s.intermediate);
      weights.dit.layers.push_back(layer);
      const std::size_t base = matrices.size() - 4;
      const std::size_t vbase = vectors.size() - 2;
      oracle_layers.push_back(
          vo_layer{vectors[vbase].data(), matrices[base].data(),
                   matrices[base + 1].data(), vectors[vbase + 1].data(),
                   matrices[base + 2].data(), matrices[base + 3].data()});
    }
    weights.dit.norm = vector(h, 1.0, 0.02);
    const std::uint16_t* norm = vectors.back().data();
    weights.dit_in = projection(h, 64);
    weights.dit_cond = projection(h, 64);
    weights.dit_out = projection(64, h);
    weights.time_1 = projection(h, 256);
    weights.time_2 = projection(h, h);
    weights.delta_time_1 = projection(h, 256);
    weights.delta_time_2 = projection(h, h);
    const std::size_t first = matrices.size() - 7;
    const std::size_t vfirst = vectors.size() - 7;
    const auto op = [&](std::size_t i) {
      return vo_projection{matrices[first + i].data(),
                           vectors[vfirst + i].data()};
    };
    rope = vc::RopeTable(config.rope, 11);
    oracle.hidden = h;
    oracle.heads = s.heads;
    oracle.kv_heads = s.kv_heads;
    oracle.head_dim = s.head_dim;
    oracle.ffn = s.intermediate;
    oracle.layers = s.layers;
    oracle.patch = 4;
    oracle.feat = 64;
    oracle.time_in = 256;
    oracle.eps = s.rms_eps;
    oracle.has_delta = 1;
    oracle.rope = rope.data();
    oracle.layer = oracle_layers.data();
    oracle.norm = norm;
    oracle.in_proj = op(0);
    oracle.cond_proj = op(1);
    oracle.out_proj = op(2);
    oracle.time_1 = op(3);
    oracle.time_2 = op(4);
    oracle.delta_1 = op(5);
    oracle.delta_2 = op(6);
    oracle.threads = 8;
  }
};

double RelativeMax(const std::vector<float>& a, const std::vector<float>& b) {
  double diff = 0.0, scale = 0.0;
  for (std::size_t i = 0; i < a.size(); ++i) {
    diff = std::max(diff, static_cast<double>(std::fabs(a[i] - b[i])));
    scale = std::max(scale, static_cast<double>(std::fabs(b[i])));
  }
  return diff / std::max(scale, 1e-30);
}

void TestDitSampler(Random& rng) {
  SmallDit dit(rng);
  std::string error;
  auto sampler = vc::DitSampler::Create(dit.config, dit.weights, &error);
  if (sampler == nullptr) {
    Report(false, "DitSampler::Create: " + error);
    return;
  }
  std::vector<float> mu(2 * 256), cond(4 * 64), x(4 * 64);
  for (auto& v : mu)
    v = vo_bf16_value(vo_bf16_bits(static_cast<float>(rng.Normal())));
  for (auto& v : cond)
    v = static_cast<float>(rng.Normal());
  for (auto& v : x)
    v = static_cast<float>(rng.Normal());
  std::vector<float> velocity(2 * 4 * 64), expected(2 * 4 * 64);
  sampler->Velocity(mu.data(), cond.data(), x.data(), 0.63F,
                    velocity.data());
  vo_dit_velocity(&dit.oracle, mu.data(), cond.data(), x.data(), 0.63F,
                  expected.data());
  const double v_error = RelativeMax(velocity, expected);
  Report(v_error <= 1e-2,
         "DitSampler::Velocity against the oracle: " + Scientific(v_error));

  std::vector<float> latent(4 * 64);
  sampler->Sample(mu.data(), cond.data(), x.data(), 10, 2.0F, latent.data());
  const std::vector<vc::EulerStep> schedule = vc::EulerSchedule(10);
  std::vector<float> t, dt;
  std::vector<std::int32_t> evaluate;
  for (const auto& step : schedule) {
    t.push_back(step.t);
    dt.push_back(step.dt);
    evaluate.push_back(step.evaluate ? 1 : 0);
  }
  std::vector<float> sampled = x;
  vo_dit_patch(&dit.oracle, mu.data(), cond.data(), sampled.data(), t.data(),
               dt.data(), evaluate.data(), t.size(), 2.0F, 1);
  // The sampler's own sensitivity: the oracle from noise moved by 1e-4.
  std::vector<float> moved = x;
  for (auto& v : moved)
    v *= 1.0F + 1e-4F;
  vo_dit_patch(&dit.oracle, mu.data(), cond.data(), moved.data(), t.data(),
               dt.data(), evaluate.data(), t.size(), 2.0F, 1);
  std::cout << "info oracle sensitivity to a 1e-4 noise change: "
            << RelativeMax(moved, sampled) << "\n";
  const double p_error = RelativeMax(latent, sampled);
  Report(p_error <= 1e-2,
         "DitSampler::Sample latent against the oracle: " + Scientific(p_error));
  Report(!schedule.front().evaluate && schedule.back().evaluate,
         "EulerSchedule skips the first step only");
  vc::Check(hipEventSynchronize(sampler->latent_event()), "latent event");
  const auto on_device = Download(sampler->latent(), latent.size());
  Report(on_device == latent, "latent() holds the returned latent");
  // set_trace (generator.hpp:93-94): each traced Sample records the mu it
  // ran with; none after the trace is cleared.
  vc::SamplerTrace trace;
  sampler->set_trace(&trace);
  std::vector<float> mu2 = mu;
  for (auto& v : mu2)
    v = -v;
  sampler->Sample(mu.data(), cond.data(), x.data(), 10, 2.0F, nullptr);
  sampler->Sample(mu2.data(), cond.data(), x.data(), 10, 2.0F, nullptr);
  sampler->set_trace(nullptr);
  sampler->Sample(mu.data(), cond.data(), x.data(), 10, 2.0F, nullptr);
  Report(trace.mu.size() == 2 && trace.mu[0] == mu && trace.mu[1] == mu2,
         "set_trace records the mu of each traced Sample");
}

/// ForwardStack (transformer.cpp:55-100) on a small GQA stack with a key/
/// value cache: a causal 6-row prefill, then one-row decode steps (the
/// LM's layout, generator.cpp:482-510) against the oracle's stack, on Q8_0
/// panels (one vx_stack_forward call) and on bf16 rows of the same weights
/// (the reference's launch sequence).
void TestForwardStack(Random& rng, hipStream_t stream) {
  vc::TransformerConfig config;
  config.hidden = 256;
  config.intermediate = 512;
  config.layers = 2;
  config.heads = 4;
  config.kv_heads = 2;
  config.head_dim = 64;
  config.rms_eps = 1e-5F;
  const std::size_t h = config.hidden;
  const std::size_t qkv = (config.heads + 2 * config.kv_heads) * config.head_dim;
  const std::size_t q_width = config.heads * config.head_dim;
  const std::size_t capacity = 16;
  std::vector<std::vector<std::uint8_t>> blocks;
  std::vector<std::vector<std::uint16_t>> vectors;
  std::vector<vc::DeviceBuffer<std::uint8_t>> panels;
  std::vector<vc::DeviceBuffer<std::uint16_t>> rows_bf16;
  std::vector<vc::DeviceBuffer<std::uint16_t>> device_vectors;
  blocks.reserve(16);
  vectors.reserve(16);
  panels.reserve(16);
  rows_bf16.reserve(16);
  device_vectors.reserve(16);
  vc::StackWeights q8_stack, bf16_stack;
  q8_stack.config = bf16_stack.config = config;
  std::vector<vo_layer> q8_layers, bf16_layers;
  std::vector<std::vector<std::uint16_t>> dequantized;
  dequantized.reserve(16);
  const auto vector = [&](std::size_t count) {
    std::vector<std::uint16_t> v(count);
    for (auto& x : v)
      x = vo_bf16_bits(static_cast<float>(1.0 + 0.02 * rng.Normal()));
    vectors.push_back(v);
    device_vectors.push_back(Upload(v));
    return static_cast<const vc::Bf16*>(device_vectors.back().get());
  };
  // One matrix: Q8_0 panels for the first stack, bf16 rows of bf16(scale q)
  // for the second; the oracle's copies of both.
  const auto matrix = [&](std::size_t out, std::size_t in, vc::Projection& q8,
                          vc::Projection& bf16, const std::uint8_t** q8_host,
                          const std::uint8_t** bf16_host) {
    blocks.push_back(ModelWeights(out, in, rng));
    panels.push_back(Pack(blocks.back(), out, in));
    std::vector<std::uint16_t> w(out * in);
    vo_q8_dequant_bf16(blocks.back().data(), out, in, w.data());
    dequantized.push_back(w);
    rows_bf16.push_back(Upload(w));
    q8 = {vc::Matrix{vc::WeightFormat::kQ8Panels, panels.back().get()}, nullptr, in, out};
    bf16 = {vc::Matrix{vc::WeightFormat::kBf16, rows_bf16.back().get()}, nullptr, in, out};
    *q8_host = blocks.back().data();
    *bf16_host = reinterpret_cast<const std::uint8_t*>(dequantized.back().data());
  };
  for (std::size_t l = 0; l < config.layers; ++l) {
    vc::LayerWeights a, b;
    vo_layer oa{}, ob{};
    a.input_norm = b.input_norm = vector(h);
    oa.input_norm = ob.input_norm = vectors.back().data();
    matrix(qkv, h, a.qkv, b.qkv, &oa.qkv, &ob.qkv);
    matrix(h, q_width, a.o, b.o, &oa.o, &ob.o);
    a.post_norm = b.post_norm = vector(h);
    oa.post_norm = ob.post_norm = vectors.back().data();
    matrix(2 * config.intermediate, h, a.gate_up, b.gate_up, &oa.gate_up, &ob.gate_up);
    matrix(h, config.intermediate, a.down, b.down, &oa.down, &ob.down);
    q8_stack.layers.push_back(a);
    bf16_stack.layers.push_back(b);
    q8_layers.push_back(oa);
    bf16_layers.push_back(ob);
  }
  q8_stack.norm = bf16_stack.norm = vector(h);
  vc::RopeConfig rope_config;
  rope_config.dim = config.head_dim;
  const std::vector<float> rope = vc::RopeTable(rope_config, 64);
  const auto rope_device = Upload(rope);

  for (const bool native : {true, false}) {
    const vc::StackWeights& stack = native ? q8_stack : bf16_stack;
    vo_stack oracle{};
    oracle.hidden = h;
    oracle.heads = config.heads;
    oracle.kv_heads = config.kv_heads;
    oracle.head_dim = config.head_dim;
    oracle.ffn = config.intermediate;
    oracle.layers = config.layers;
    oracle.eps = config.rms_eps;
    oracle.rope = rope.data();
    oracle.layer = native ? q8_layers.data() : bf16_layers.data();
    oracle.norm = vectors.back().data();
    oracle.threads = 4;
    oracle.bf16_weights = native ? 0 : 1;
    vc::KvCache cache(config, capacity);
    vc::StackScratch scratch;
    vc::Bf16Gemm gemm(nullptr, stream);
    const std::size_t cache_floats = config.layers * config.kv_heads * capacity * config.head_dim;
    std::vector<float> k_host(cache_floats, 0.0F), v_host(cache_floats, 0.0F);
    vc::Check(hipMemset(cache.keys(0), 0, cache_floats * sizeof(float)), "clear");
    vc::Check(hipMemset(cache.values(0), 0, cache_floats * sizeof(float)), "clear");
    double worst = 0.0;
    for (const std::size_t position : {0, 6, 7}) {
      const std::size_t rows = position == 0 ? 6 : 1;
      std::vector<std::int32_t> at(rows);
      for (std::size_t r = 0; r < rows; ++r)
        at[r] = static_cast<std::int32_t>(position + r);
      const auto at_device = Upload(at);
      vc::AttentionLayout layout;
      layout.positions = at_device.get();
      layout.cache_rows = at_device.get();
      layout.rows_per_sequence = rows;
      layout.keys_per_sequence = rows;
      layout.past = position;
      layout.causal = true;
      std::vector<float> hidden(rows * h);
      for (auto& v : hidden)
        v = static_cast<float>(rng.Normal());
      auto hidden_device = Upload(hidden);
      vc::DeviceBuffer<float> output(rows * h);
      vc::ForwardStack(stack, rope_device.get(), layout, cache, hidden_device.get(),
                       output.get(), rows, scratch, gemm, stream);
      vc::Check(hipStreamSynchronize(stream), "sync");
      std::vector<float> expected(rows * h);
      vo_stack_forward(&oracle, hidden.data(), expected.data(), rows, at.data(), at.data(),
                       rows, rows, position, 1, k_host.data(), v_host.data(), capacity);
      worst = std::max(worst, RelativeMax(Download(output.get(), rows * h), expected));
      worst = std::max(worst, RelativeMax(Download(hidden_device.get(), rows * h), hidden));
    }
    worst = std::max(worst, RelativeMax(Download(cache.keys(0), cache_floats), k_host));
    Report(worst <= 1e-2, std::string("ForwardStack on ") +
                              (native ? "Q8_0 panels (vx_stack)" : "bf16 rows (per kernel)") +
                              " against the oracle: " + Scientific(worst));
  }
}

}  // namespace

int main() {
  int devices = 0;
  if (hipGetDeviceCount(&devices) != hipSuccess || devices == 0) {
    std::cout << "no GPU; skipped\n";
    return kSkip;
  }
  try {
    hipStream_t stream = nullptr;
    vc::Check(hipStreamCreate(&stream), "stream");
    Random rng(1234);
    TestLinear(1024, 2560, rng, stream);
    TestLinear(4096, 1024, rng, stream);
    TestLinearBf16(1024, 2560, rng, stream);
    TestPrefillSplit(rng, stream);
    TestDitSampler(rng);
    TestForwardStack(rng, stream);
    vc::Check(hipStreamDestroy(stream), "stream");
  } catch (const std::exception& failure) {
    std::cout << "FAIL " << failure.what() << "\n";
    return 1;
  }
  if (failures > 0) {
    std::cout << failures << " failures\n";
    return 1;
  }
  std::cout << "all host-surface checks match\n";
  return 0;
}
