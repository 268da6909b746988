// The local DiT of VoxCPM2 and its sampler on one stream: the CFG pair of
// branches (22 rows) through the stack, the time embedding cached per t,
// and the whole multi-step patch replayed as one HIP graph.
//
// Follows generator.cpp:297-324 (EvaluateDit), 424-463 (Step's sampler),
// 515-538 (Velocity), 212-237 (TimeVector), 63-80 (EulerSchedule) and
// transformer.cpp:20-45 (RopeTable), 55-100 (ForwardStack).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <map>
#include <vector>

#include "common.hpp"
#include "dit_fused.hpp"
#include "dit_kernels.hpp"
#include "dit_persistent.hpp"
#include "products.hpp"
#include "q8.hpp"
#include "q8_tile.hpp"
#include "voxcpm_amd_internal.h"

namespace {

using vx::Bf16;

template<typename T>
int Allocate(T** pointer, std::size_t count) {
  const hipError_t error = hipMalloc(reinterpret_cast<void**>(pointer),
                                     std::max<std::size_t>(count, 1) * sizeof(T));
  if (error != hipSuccess)
    return vx::FailHip(error, "vx_dit_create: hipMalloc");
  return VX_OK;
}

/// The time embedding's input features for time t, already rounded to the
/// bf16 operand of time_mlp: width / 2 sines and then the cosines of the
/// same phases, phase j = (1000 t) * e^(-j d) with d = ln(10000) / (width / 2 - 1)
/// rounded to float32 once. Each step is one float32 operation, so the
/// values are those of the reference's SinusoidalPosEmb (generator.cpp:40-53).
std::vector<Bf16> TimeFeatures(float t, std::size_t width) {
  const std::size_t count = width / 2;
  const float decay = static_cast<float>(std::log(10000.0) / static_cast<double>(count - 1));
  const float time_scaled = t * 1000.0F;
  std::vector<Bf16> features(2 * count);
  for (std::size_t j = 0; j < count; ++j) {
    const float phase = time_scaled * std::exp(-decay * static_cast<float>(j));
    features[j] = vx::Bf16Bits(std::sin(phase));
    features[count + j] = vx::Bf16Bits(std::cos(phase));
  }
  return features;
}

struct GraphKey {
  const float* mu = nullptr;
  const float* cond_latent = nullptr;
  float* x = nullptr;
  std::vector<float> t;
  std::vector<float> dt;
  std::vector<std::int32_t> evaluate;
  float cfg = 0.0F;
  int zero_star = 0;
  int path = 0;
  hipStream_t stream = nullptr;

  bool operator==(const GraphKey& other) const {
    return mu == other.mu && cond_latent == other.cond_latent &&
           x == other.x && t == other.t && dt == other.dt &&
           evaluate == other.evaluate && cfg == other.cfg &&
           zero_star == other.zero_star && path == other.path &&
           stream == other.stream;
  }
};

}  // namespace

struct vx_dit {
  vx_dit_shape shape{};
  vx_dit_weights weights{};
  std::vector<vx_dit_layer> layers;
  std::size_t rows = 0;     // 2 (3 + 2 patch)
  std::size_t length = 0;   // 3 + 2 patch
  std::size_t q_width = 0;
  std::size_t kv_width = 0;
  std::size_t qkv_width = 0;

  // Product split scratch (partials, counters zero between products).
  float* partials = nullptr;
  std::size_t partial_floats = 0;
  unsigned* counters = nullptr;
  std::size_t counter_count = 0;

  std::int32_t* positions = nullptr;
  std::int32_t* cache_rows = nullptr;
  std::int32_t* outputs = nullptr;
  float* hidden = nullptr;
  float* output = nullptr;
  float* qkv = nullptr;
  float* q = nullptr;
  float* k_cache = nullptr;
  float* v_cache = nullptr;
  float* gate_up = nullptr;
  float* x_rows = nullptr;
  float* gathered = nullptr;
  float* cond_rows = nullptr;
  float* velocity = nullptr;
  float* middle = nullptr;
  float* delta = nullptr;
  Bf16* bf16 = nullptr;
  Bf16* time_bf16 = nullptr;
  std::map<std::uint32_t, float*> time_vectors;  // by the bits of t

  // The fused path (up to 32 rows): residual stream and product inputs in
  // fragment order (q8_tile.hpp).
  bool fused = false;
  vx::fused::Shape fused_shape{};
  float* h_frag = nullptr;
  Bf16* attention_frag = nullptr;
  Bf16* swiglu_frag = nullptr;
  // The next norm's operand as its producer leaves it: bf16(h gamma) in
  // fragment order [32][hidden] and the rows' sums of h^2 per 16 columns
  // [32][hidden / 16].
  Bf16* norm_frag = nullptr;
  float* norm_squares = nullptr;

  // The persistent evaluation (one launch per evaluation): its write-once
  // workspace and barrier counters.
  bool persistent = false;
  int grid = 0;
  vx::persistent::Workspace workspace{};

  // Which evaluation runs (vx_dit_set_path): VX_DIT_PATH_AUTO takes the
  // fused kernels where the shape allows, else the per-kernel path. The
  // persistent kernel is selected explicitly: on MI355X it measures about
  // 10 % slower per evaluation than the fused launches (378 vs 335 us for
  // 12 layers), its phases bound by the same memory round trips.
  int path = VX_DIT_PATH_AUTO;
  // vx_dit_set_trace: device buffer of persistent launches' timestamps.
  unsigned long long* trace = nullptr;

  GraphKey graph_key;
  hipGraphExec_t graph = nullptr;

  ~vx_dit() {
    if (graph != nullptr)
      (void)hipGraphExecDestroy(graph);
    for (auto& entry : time_vectors)
      (void)hipFree(entry.second);
    for (void* pointer :
         {static_cast<void*>(partials), static_cast<void*>(counters),
          static_cast<void*>(positions), static_cast<void*>(cache_rows),
          static_cast<void*>(outputs), static_cast<void*>(hidden),
          static_cast<void*>(output), static_cast<void*>(qkv),
          static_cast<void*>(q), static_cast<void*>(k_cache),
          static_cast<void*>(v_cache), static_cast<void*>(gate_up),
          static_cast<void*>(x_rows), static_cast<void*>(gathered),
          static_cast<void*>(cond_rows), static_cast<void*>(velocity),
          static_cast<void*>(middle), static_cast<void*>(delta),
          static_cast<void*>(bf16), static_cast<void*>(time_bf16),
          static_cast<void*>(h_frag), static_cast<void*>(attention_frag),
          static_cast<void*>(swiglu_frag), static_cast<void*>(norm_frag),
          static_cast<void*>(norm_squares), static_cast<void*>(workspace.h),
          static_cast<void*>(workspace.qkv),
          static_cast<void*>(workspace.attention),
          static_cast<void*>(workspace.swiglu),
          static_cast<void*>(workspace.norm),
          static_cast<void*>(workspace.squares),
          static_cast<void*>(workspace.sync)})
      if (pointer != nullptr)
        (void)hipFree(pointer);
  }

  /// The weights' format (every matrix).
  vx::q8::Weights Kind() const {
    return weights.format == VX_WEIGHTS_BF16 ? vx::q8::Weights::kBf16 : vx::q8::Weights::kQ8;
  }

  /// y[m][n] (+)= x W^T on the panels.
  int Linear(const Bf16* x, const void* w, float* y, std::size_t m,
             std::size_t k, std::size_t n, bool accumulate,
             hipStream_t stream) {
    const vx::ProductPlan plan =
        vx::PlanSkinny(m, k, n, partial_floats, counter_count, 0, 0, 0, Kind());
    return vx::RunSkinny(x, w, y, nullptr, m, k, n, accumulate, plan,
                         partials, counters, stream, Kind());
  }

  /// Project (transformer.cpp:47-53): y = x W^T + b.
  int Project(const vx_dit_projection& p, const Bf16* x, float* y,
              std::size_t m, std::size_t k, std::size_t n,
              hipStream_t stream) {
    VX_TRY(Linear(x, p.weight, y, m, k, n, false, stream));
    if (p.bias != nullptr)
      vx::kernels::AddBias(y, p.bias, m, n, stream);
    return VX_OK;
  }

  /// time_mlp(sinusoid(t)) (+ delta) into `vector` (generator.cpp:212-237).
  int TimeVector(float t, float* vector, hipStream_t stream) {
    const std::size_t width = shape.hidden;
    const std::size_t in = shape.time_in;
    const std::vector<Bf16> host = TimeFeatures(t, in);
    VX_HIP(hipMemcpyAsync(time_bf16, host.data(), in * sizeof(Bf16),
                          hipMemcpyHostToDevice, stream),
           "time embedding upload");
    VX_TRY(Project(weights.time_1, time_bf16, middle, 1, in, width, stream));
    vx::kernels::ToBf16(middle, time_bf16, width, true, stream);
    if (shape.has_delta)
      vx::kernels::CopyFloats(delta, vector, width, stream);
    VX_TRY(Linear(time_bf16, weights.time_2.weight, vector, 1, width, width,
                  shape.has_delta != 0, stream));
    if (weights.time_2.bias != nullptr)
      vx::kernels::AddBias(vector, weights.time_2.bias, 1, width, stream);
    // The host staging goes away on return.
    VX_HIP(hipStreamSynchronize(stream), "time embedding");
    return vx::LaunchStatus("time embedding");
  }

  /// The cached time vector of t (computed on first use, like the
  /// reference's per-t cache).
  int CachedTime(float t, const float** vector, hipStream_t stream) {
    std::uint32_t bits;
    std::memcpy(&bits, &t, sizeof bits);
    const auto found = time_vectors.find(bits);
    if (found != time_vectors.end()) {
      *vector = found->second;
      return VX_OK;
    }
    float* created = nullptr;
    VX_TRY(Allocate(&created, shape.hidden));
    const int status = TimeVector(t, created, stream);
    if (status != VX_OK) {
      (void)hipFree(created);
      return status;
    }
    time_vectors.emplace(bits, created);
    *vector = created;
    return VX_OK;
  }

  int CondRows(const float* cond_latent, float* rows_out, hipStream_t stream) {
    const std::size_t values = shape.patch * shape.feat;
    vx::kernels::ToBf16(cond_latent, bf16, values, false, stream);
    return Project(weights.cond_proj, bf16, rows_out, shape.patch, shape.feat,
                   shape.hidden, stream);
  }

  /// The evaluation path that runs: VX_DIT_PATH_PERSISTENT,
  /// VX_DIT_PATH_FUSED, VX_DIT_PATH_FUSED_REFERENCE_ORDER or
  /// VX_DIT_PATH_UNFUSED.
  int Resolved() const {
    if (path == VX_DIT_PATH_AUTO)
      return fused ? VX_DIT_PATH_FUSED : VX_DIT_PATH_UNFUSED;
    return path;
  }

  /// EvaluateDit (generator.cpp:297-324) with ForwardStack
  /// (transformer.cpp:55-100) on the fused kernels: one persistent launch,
  /// or 5 launches per layer plus the input assembly and the output
  /// projection; the last also takes the guided Euler step when `x_update`
  /// is given.
  int EvalFused(const float* mu, const float* cond, const float* x,
                const float* time, float* velocity_out, float* x_update,
                float cfg, float dt, int zero_star, hipStream_t stream) {
    const vx::fused::Shape& fs = fused_shape;
    if (Resolved() == VX_DIT_PATH_PERSISTENT) {
      vx::persistent::Weights w{};
      for (std::size_t l = 0; l < layers.size() && l < vx::persistent::kMaxLayers; ++l)
        w.layers[l] = {layers[l].input_norm, static_cast<const std::uint8_t*>(layers[l].qkv),
                       static_cast<const std::uint8_t*>(layers[l].o), layers[l].post_norm,
                       static_cast<const std::uint8_t*>(layers[l].gate_up),
                       static_cast<const std::uint8_t*>(layers[l].down)};
      w.in_w = static_cast<const std::uint8_t*>(weights.in_proj.weight);
      w.in_b = weights.in_proj.bias;
      w.out_w = static_cast<const std::uint8_t*>(weights.out_proj.weight);
      w.out_b = weights.out_proj.bias;
      w.final_norm = weights.norm;
      w.rope = weights.rope;
      return vx::persistent::Evaluate(fs, static_cast<int>(shape.layers), grid, w,
                                      workspace, mu, time, cond, x, velocity_out,
                                      x_update, cfg, dt, zero_star, trace, stream);
    }
    if (Resolved() == VX_DIT_PATH_FUSED_REFERENCE_ORDER) {
      // The norm products normalise the float32 stream in their prologue
      // (bf16((h r) gamma), the reference's rounding).
      vx::fused::InAssemble(x, weights.in_proj.weight, weights.in_proj.bias, mu,
                            time, cond, h_frag, fs, stream);
      for (const vx_dit_layer& layer : layers) {
        vx::fused::Qkv(h_frag, layer.input_norm, layer.qkv, qkv, fs, stream);
        vx::fused::Attention(qkv, weights.rope, attention_frag, fs, stream);
        vx::fused::Residual(attention_frag, layer.o, static_cast<int>(q_width), fs.hidden,
                            h_frag, fs, stream);
        vx::fused::GateUp(h_frag, layer.post_norm, layer.gate_up, swiglu_frag, fs, stream);
        vx::fused::Residual(swiglu_frag, layer.down, fs.ffn, fs.hidden, h_frag, fs, stream);
      }
      vx::fused::OutEuler(h_frag, weights.norm, weights.out_proj.weight,
                          weights.out_proj.bias, velocity_out, x_update, cfg, dt,
                          zero_star, fs, stream);
      return vx::LaunchStatus("vx_dit_eval");
    }
    // Each residual update also leaves the next RMSNorm's operand
    // bf16(h gamma) and the rows' sums of squares, which the qkv and
    // gate_up products read in place of the float32 stream, applying the
    // rows' rsqrt(mean + eps) to their outputs.
    const auto operand = [&](const Bf16* gamma) {
      return vx::fused::NormOperand{norm_frag, gamma, norm_squares};
    };
    vx::fused::InAssemble(x, weights.in_proj.weight, weights.in_proj.bias, mu,
                          time, cond, h_frag, fs, stream,
                          layers.empty() ? vx::fused::NormOperand{}
                                         : operand(layers[0].input_norm));
    for (std::size_t l = 0; l < layers.size(); ++l) {
      const vx_dit_layer& layer = layers[l];
      vx::fused::QkvScaled(operand(nullptr), layer.qkv, qkv, fs, stream);
      vx::fused::Attention(qkv, weights.rope, attention_frag, fs, stream);
      vx::fused::Residual(attention_frag, layer.o,
                          static_cast<int>(q_width), fs.hidden, h_frag, fs,
                          stream, operand(layer.post_norm));
      vx::fused::GateUpScaled(operand(nullptr), layer.gate_up, swiglu_frag, fs, stream);
      vx::fused::Residual(swiglu_frag, layer.down, fs.ffn, fs.hidden, h_frag,
                          fs, stream,
                          l + 1 < layers.size() ? operand(layers[l + 1].input_norm)
                                                : vx::fused::NormOperand{});
    }
    vx::fused::OutEuler(h_frag, weights.norm, weights.out_proj.weight,
                        weights.out_proj.bias, velocity_out, x_update, cfg, dt,
                        zero_star, fs, stream);
    return vx::LaunchStatus("vx_dit_eval");
  }

  /// EvaluateDit (generator.cpp:297-324) with ForwardStack
  /// (transformer.cpp:55-100).
  int Eval(const float* mu, const float* cond, const float* x,
           const float* time, float* velocity_out, hipStream_t stream) {
    if (Resolved() != VX_DIT_PATH_UNFUSED)
      return EvalFused(mu, cond, x, time, velocity_out, nullptr, 0.0F, 0.0F,
                       0, stream);
    const std::size_t width = shape.hidden;
    const std::size_t patch = shape.patch;
    const std::size_t feat = shape.feat;
    const std::size_t ffn = shape.ffn;
    vx::kernels::ToBf16(x, bf16, patch * feat, false, stream);
    VX_TRY(Project(weights.in_proj, bf16, x_rows, patch, feat, width, stream));
    vx::kernels::AssembleDit(mu, time, cond, x_rows, hidden, patch, width,
                             stream);
    for (const vx_dit_layer& layer : layers) {
      vx::kernels::RmsNorm(hidden, layer.input_norm, bf16, nullptr, rows,
                           width, shape.eps, stream);
      VX_TRY(Linear(bf16, layer.qkv, qkv, rows, width, qkv_width, false,
                    stream));
      vx::kernels::QkvRope(qkv, weights.rope, positions, cache_rows, q,
                           k_cache, v_cache, rows, shape.heads,
                           shape.kv_heads, shape.head_dim, rows, stream);
      vx::kernels::Attention(q, k_cache, v_cache, bf16, rows, length, length,
                             0, false, shape.heads, shape.kv_heads,
                             shape.head_dim, rows, stream);
      VX_TRY(Linear(bf16, layer.o, hidden, rows, q_width, width, true,
                    stream));
      vx::kernels::RmsNorm(hidden, layer.post_norm, bf16, nullptr, rows,
                           width, shape.eps, stream);
      VX_TRY(Linear(bf16, layer.gate_up, gate_up, rows, width, 2 * ffn, false,
                    stream));
      vx::kernels::SwiGlu(gate_up, bf16, rows, ffn, stream);
      VX_TRY(Linear(bf16, layer.down, hidden, rows, ffn, width, true,
                    stream));
    }
    vx::kernels::RmsNorm(hidden, weights.norm, bf16, output, rows, width,
                         shape.eps, stream);
    vx::kernels::GatherRows(output, outputs, gathered, 2 * patch, width,
                            stream);
    vx::kernels::ToBf16(gathered, bf16, 2 * patch * width, false, stream);
    VX_TRY(Project(weights.out_proj, bf16, velocity_out, 2 * patch, width,
                   feat, stream));
    return vx::LaunchStatus("vx_dit_eval");
  }

  /// The sampler loop of Step (generator.cpp:457-463) after the condition.
  int Sample(const float* mu, float* x, const GraphKey& key,
             const std::vector<const float*>& times, hipStream_t stream) {
    const std::size_t values = shape.patch * shape.feat;
    for (std::size_t step = 0; step < key.t.size(); ++step) {
      if (!key.evaluate[step])
        continue;  // zero velocity
      if (Resolved() != VX_DIT_PATH_UNFUSED) {
        VX_TRY(EvalFused(mu, cond_rows, x, times[step], velocity, x, key.cfg,
                         key.dt[step], key.zero_star, stream));
        continue;
      }
      VX_TRY(Eval(mu, cond_rows, x, times[step], velocity, stream));
      vx::kernels::GuidedEuler(velocity, x, values, key.cfg, key.dt[step],
                               key.zero_star != 0, stream);
    }
    return vx::LaunchStatus("vx_dit_patch");
  }
};

namespace {

int CheckShape(const vx_dit_shape& s) {
  if (s.hidden == 0 || s.heads == 0 || s.kv_heads == 0 || s.head_dim == 0 ||
      s.ffn == 0 || s.layers == 0 || s.patch == 0 || s.feat == 0 ||
      s.time_in < 4)
    return vx::Fail(VX_BAD_ARG, "vx_dit_create: zero dimension");
  if (s.heads % s.kv_heads != 0)
    return vx::Fail(VX_BAD_ARG,
                    "vx_dit_create: heads must be a multiple of kv_heads");
  if (s.head_dim % 2 != 0 || s.head_dim > 256)
    return vx::Fail(VX_UNSUPPORTED,
                    "vx_dit_create: head_dim must be even and <= 256");
  if (s.hidden % 32 != 0 || s.ffn % 32 != 0 || s.feat % 32 != 0 ||
      s.time_in % 32 != 0 || (s.heads * s.head_dim) % 32 != 0)
    return vx::Fail(VX_UNSUPPORTED,
                    "vx_dit_create: product inputs must be multiples of 32");
  if (2 * (3 + 2 * s.patch) > vx::kExactRows)
    return vx::Fail(VX_UNSUPPORTED, "vx_dit_create: patch too long");
  return VX_OK;
}

int CheckWeights(const vx_dit_shape& s, const vx_dit_weights& w) {
  if (w.format != VX_WEIGHTS_Q8_0 && w.format != VX_WEIGHTS_BF16)
    return vx::Fail(VX_BAD_ARG, "vx_dit_create: unknown weight format");
  if (w.layers == nullptr || w.norm == nullptr || w.in_proj.weight == nullptr ||
      w.cond_proj.weight == nullptr || w.out_proj.weight == nullptr ||
      w.time_1.weight == nullptr || w.time_2.weight == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_dit_create: missing weights");
  if (s.has_delta &&
      (w.delta_1.weight == nullptr || w.delta_2.weight == nullptr))
    return vx::Fail(VX_BAD_ARG, "vx_dit_create: missing delta_time weights");
  for (std::uint32_t l = 0; l < s.layers; ++l) {
    const vx_dit_layer& layer = w.layers[l];
    if (layer.input_norm == nullptr || layer.qkv == nullptr ||
        layer.o == nullptr || layer.post_norm == nullptr ||
        layer.gate_up == nullptr || layer.down == nullptr)
      return vx::Fail(VX_BAD_ARG, "vx_dit_create: missing layer weights");
  }
  return VX_OK;
}

int Create(vx_dit* dit) {
  const vx_dit_shape& s = dit->shape;
  const std::size_t rows = dit->rows;
  const std::size_t wide = std::max<std::size_t>(
      {s.hidden, dit->q_width, s.ffn, s.time_in, s.patch * s.feat});
  dit->partial_floats = 16 * rows * std::max<std::size_t>(
                                        {dit->qkv_width, 2 * s.ffn, s.hidden});
  dit->counter_count =
      vx::q8::Groups(std::max<std::size_t>({dit->qkv_width, 2 * s.ffn, s.hidden}));
  VX_TRY(Allocate(&dit->partials, dit->partial_floats));
  VX_TRY(Allocate(&dit->counters, dit->counter_count));
  VX_HIP(hipMemset(dit->counters, 0, dit->counter_count * sizeof(unsigned)),
         "vx_dit_create: hipMemset");
  VX_TRY(Allocate(&dit->positions, rows));
  VX_TRY(Allocate(&dit->cache_rows, rows));
  VX_TRY(Allocate(&dit->outputs, 2 * s.patch));
  VX_TRY(Allocate(&dit->hidden, rows * s.hidden));
  VX_TRY(Allocate(&dit->output, rows * s.hidden));
  VX_TRY(Allocate(&dit->qkv, rows * dit->qkv_width));
  VX_TRY(Allocate(&dit->q, rows * dit->q_width));
  VX_TRY(Allocate(&dit->k_cache, rows * dit->kv_width));
  VX_TRY(Allocate(&dit->v_cache, rows * dit->kv_width));
  VX_TRY(Allocate(&dit->gate_up, rows * 2 * s.ffn));
  VX_TRY(Allocate(&dit->x_rows, s.patch * s.hidden));
  VX_TRY(Allocate(&dit->gathered, 2 * s.patch * s.hidden));
  VX_TRY(Allocate(&dit->cond_rows, s.patch * s.hidden));
  VX_TRY(Allocate(&dit->velocity, 2 * s.patch * s.feat));
  VX_TRY(Allocate(&dit->middle, s.hidden));
  VX_TRY(Allocate(&dit->delta, s.hidden));
  VX_TRY(Allocate(&dit->bf16, rows * wide));
  VX_TRY(Allocate(&dit->time_bf16, std::max<std::size_t>(s.hidden, s.time_in)));

  vx::fused::Shape& fs = dit->fused_shape;
  fs.rows = static_cast<int>(rows);
  fs.length = static_cast<int>(dit->length);
  fs.patch = static_cast<int>(s.patch);
  fs.hidden = static_cast<int>(s.hidden);
  fs.heads = static_cast<int>(s.heads);
  fs.kv_heads = static_cast<int>(s.kv_heads);
  fs.head_dim = static_cast<int>(s.head_dim);
  fs.ffn = static_cast<int>(s.ffn);
  fs.feat = static_cast<int>(s.feat);
  fs.eps = s.eps;
  fs.weights = dit->Kind();
  dit->fused = vx::fused::Supported(fs);
  if (dit->fused) {
    const std::size_t h_count = vx::q8::FragElements(s.hidden);
    const std::size_t a_count = vx::q8::FragElements(dit->q_width);
    const std::size_t s_count = vx::q8::FragElements(s.ffn);
    VX_TRY(Allocate(&dit->h_frag, h_count));
    VX_TRY(Allocate(&dit->attention_frag, a_count));
    VX_TRY(Allocate(&dit->swiglu_frag, s_count));
    const std::size_t squares_count = vx::q8::kFragRows * (s.hidden / 16);
    VX_TRY(Allocate(&dit->norm_frag, h_count));
    VX_TRY(Allocate(&dit->norm_squares, squares_count));
    // Rows past the pair stay zero (never written, never read).
    VX_HIP(hipMemset(dit->h_frag, 0, h_count * sizeof(float)),
           "vx_dit_create: hipMemset");
    VX_HIP(hipMemset(dit->attention_frag, 0, a_count * sizeof(Bf16)),
           "vx_dit_create: hipMemset");
    VX_HIP(hipMemset(dit->swiglu_frag, 0, s_count * sizeof(Bf16)),
           "vx_dit_create: hipMemset");
    VX_HIP(hipMemset(dit->norm_frag, 0, h_count * sizeof(Bf16)),
           "vx_dit_create: hipMemset");
    VX_HIP(hipMemset(dit->norm_squares, 0, squares_count * sizeof(float)),
           "vx_dit_create: hipMemset");

    dit->grid = vx::persistent::GridSize();
    const int layers = static_cast<int>(s.layers);
    // The persistent kernel reads Q8_0 panels only.
    dit->persistent = fs.weights == vx::q8::Weights::kQ8 &&
                      vx::persistent::Supported(fs, layers, dit->grid) &&
                      vx::persistent::Prepare(fs);
  }
  if (dit->persistent) {
    vx::persistent::Workspace& ws = dit->workspace;
    const int layers = static_cast<int>(s.layers);
    const std::size_t h_count = vx::persistent::HElements(fs, layers);
    const std::size_t norm_count = vx::persistent::NormElements(fs, layers);
    const std::size_t squares_count = vx::persistent::SquaresElements(fs, layers);
    const std::size_t qkv_count = vx::persistent::QkvElements(fs, layers);
    const std::size_t attention_count = vx::persistent::AttentionElements(fs, layers);
    const std::size_t swiglu_count = vx::persistent::SwigluElements(fs, layers);
    VX_TRY(Allocate(&ws.h, h_count));
    VX_TRY(Allocate(&ws.norm, norm_count));
    VX_TRY(Allocate(&ws.squares, squares_count));
    VX_TRY(Allocate(&ws.qkv, qkv_count));
    VX_TRY(Allocate(&ws.attention, attention_count));
    VX_TRY(Allocate(&ws.swiglu, swiglu_count));
    const std::size_t sync_words = vx::persistent::SyncWords(fs, layers);
    VX_TRY(Allocate(&ws.sync, sync_words));
    // Rows past the pair are never written and read as zeros.
    VX_HIP(hipMemset(ws.h, 0, h_count * sizeof(float)), "vx_dit_create: hipMemset");
    VX_HIP(hipMemset(ws.norm, 0, norm_count * sizeof(Bf16)), "vx_dit_create: hipMemset");
    VX_HIP(hipMemset(ws.squares, 0, squares_count * sizeof(float)),
           "vx_dit_create: hipMemset");
    VX_HIP(hipMemset(ws.qkv, 0, qkv_count * sizeof(float)), "vx_dit_create: hipMemset");
    VX_HIP(hipMemset(ws.attention, 0, attention_count * sizeof(Bf16)),
           "vx_dit_create: hipMemset");
    VX_HIP(hipMemset(ws.swiglu, 0, swiglu_count * sizeof(Bf16)), "vx_dit_create: hipMemset");
    VX_HIP(hipMemset(ws.sync, 0, sync_words * sizeof(unsigned)), "vx_dit_create: hipMemset");
  }

  // The rows: two sequences of 3 + 2P positions; the outputs are the last
  // P rows of each (generator.cpp:108-124).
  std::vector<std::int32_t> positions(rows), cache_rows(rows), outputs;
  for (std::size_t row = 0; row < rows; ++row) {
    positions[row] = static_cast<std::int32_t>(row % dit->length);
    cache_rows[row] = static_cast<std::int32_t>(row);
  }
  for (std::size_t sequence = 0; sequence < 2; ++sequence)
    for (std::size_t i = 0; i < s.patch; ++i)
      outputs.push_back(
          static_cast<std::int32_t>(sequence * dit->length + 3 + s.patch + i));
  VX_HIP(hipMemcpy(dit->positions, positions.data(),
                   rows * sizeof(std::int32_t), hipMemcpyHostToDevice),
         "vx_dit_create: upload");
  VX_HIP(hipMemcpy(dit->cache_rows, cache_rows.data(),
                   rows * sizeof(std::int32_t), hipMemcpyHostToDevice),
         "vx_dit_create: upload");
  VX_HIP(hipMemcpy(dit->outputs, outputs.data(),
                   outputs.size() * sizeof(std::int32_t),
                   hipMemcpyHostToDevice),
         "vx_dit_create: upload");

  // delta_time_mlp(sinusoid(0)) (generator.cpp:150-167).
  if (s.has_delta) {
    hipStream_t stream = nullptr;
    VX_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking),
           "vx_dit_create: stream");
    const std::vector<Bf16> host = TimeFeatures(0.0F, s.time_in);
    int status = VX_OK;
    hipError_t error = hipMemcpyAsync(dit->time_bf16, host.data(),
                                      s.time_in * sizeof(Bf16),
                                      hipMemcpyHostToDevice, stream);
    if (error == hipSuccess) {
      status = dit->Project(dit->weights.delta_1, dit->time_bf16, dit->middle,
                            1, s.time_in, s.hidden, stream);
      if (status == VX_OK) {
        vx::kernels::ToBf16(dit->middle, dit->time_bf16, s.hidden, true,
                            stream);
        status = dit->Project(dit->weights.delta_2, dit->time_bf16, dit->delta,
                              1, s.hidden, s.hidden, stream);
      }
      error = hipStreamSynchronize(stream);
    }
    (void)hipStreamDestroy(stream);
    if (error != hipSuccess)
      return vx::FailHip(error, "vx_dit_create: delta time");
    VX_TRY(status);
  }
  return vx::Succeed();
}

}  // namespace

extern "C" {

int vx_dit_create(vx_dit** dit, const vx_dit_shape* shape,
                  const vx_dit_weights* weights) {
  if (dit == nullptr || shape == nullptr || weights == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_dit_create: null pointer");
  *dit = nullptr;
  VX_TRY(CheckShape(*shape));
  VX_TRY(CheckWeights(*shape, *weights));
  auto* created = new vx_dit();
  created->shape = *shape;
  created->weights = *weights;
  created->layers.assign(weights->layers, weights->layers + shape->layers);
  created->weights.layers = created->layers.data();
  created->length = 3 + 2 * shape->patch;
  created->rows = 2 * created->length;
  created->q_width = static_cast<std::size_t>(shape->heads) * shape->head_dim;
  created->kv_width =
      static_cast<std::size_t>(shape->kv_heads) * shape->head_dim;
  created->qkv_width = created->q_width + 2 * created->kv_width;
  const int status = Create(created);
  if (status != VX_OK) {
    delete created;
    return status;
  }
  *dit = created;
  return VX_OK;
}

void vx_dit_destroy(vx_dit* dit) { delete dit; }

int vx_dit_time_vector(vx_dit* dit, float t, float* vector, void* stream) {
  if (dit == nullptr || vector == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_dit_time_vector: null pointer");
  return dit->TimeVector(t, vector, vx::Stream(stream));
}

int vx_dit_cond_rows(vx_dit* dit, const float* cond_latent, float* cond_rows,
                     void* stream) {
  if (dit == nullptr || cond_latent == nullptr || cond_rows == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_dit_cond_rows: null pointer");
  VX_TRY(dit->CondRows(cond_latent, cond_rows, vx::Stream(stream)));
  return vx::LaunchStatus("vx_dit_cond_rows");
}

int vx_dit_eval(vx_dit* dit, const float* mu, const float* cond_rows,
                const float* x, const float* time_vector, float* velocity,
                void* stream) {
  if (dit == nullptr || mu == nullptr || cond_rows == nullptr ||
      x == nullptr || time_vector == nullptr || velocity == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_dit_eval: null pointer");
  return dit->Eval(mu, cond_rows, x, time_vector, velocity,
                   vx::Stream(stream));
}

int vx_dit_velocity(vx_dit* dit, const float* mu, const float* cond_latent,
                    const float* x, float t, float* velocity, void* stream) {
  if (dit == nullptr || mu == nullptr || cond_latent == nullptr ||
      x == nullptr || velocity == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_dit_velocity: null pointer");
  hipStream_t s = vx::Stream(stream);
  const float* time = nullptr;
  VX_TRY(dit->CachedTime(t, &time, s));
  VX_TRY(dit->CondRows(cond_latent, dit->cond_rows, s));
  return dit->Eval(mu, dit->cond_rows, x, time, velocity, s);
}

int vx_dit_patch(vx_dit* dit, const float* mu, const float* cond_latent,
                 float* x, const float* t, const float* dt,
                 const int32_t* evaluate, size_t steps, float cfg,
                 int zero_star, void* stream) {
  if (dit == nullptr || mu == nullptr || cond_latent == nullptr ||
      x == nullptr || t == nullptr || dt == nullptr || evaluate == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_dit_patch: null pointer");
  if (steps == 0 || steps > 1000)
    return vx::Fail(VX_BAD_ARG, "vx_dit_patch: steps must be in 1..1000");
  hipStream_t s = vx::Stream(stream);
  GraphKey key;
  key.mu = mu;
  key.cond_latent = cond_latent;
  key.x = x;
  key.t.assign(t, t + steps);
  key.dt.assign(dt, dt + steps);
  key.evaluate.assign(evaluate, evaluate + steps);
  key.cfg = cfg;
  key.zero_star = zero_star;
  key.path = dit->Resolved();
  key.stream = s;
  // Time vectors first (cached per t; they synchronize on first use).
  std::vector<const float*> times(steps, nullptr);
  for (std::size_t step = 0; step < steps; ++step)
    if (evaluate[step])
      VX_TRY(dit->CachedTime(t[step], &times[step], s));
  if (s == nullptr) {
    // The null stream cannot be captured: run the launches directly.
    VX_TRY(dit->CondRows(cond_latent, dit->cond_rows, s));
    return dit->Sample(mu, x, key, times, s);
  }
  if (dit->graph == nullptr || !(dit->graph_key == key)) {
    if (dit->graph != nullptr) {
      (void)hipGraphExecDestroy(dit->graph);
      dit->graph = nullptr;
    }
    VX_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal),
           "vx_dit_patch: begin capture");
    int status = dit->CondRows(cond_latent, dit->cond_rows, s);
    if (status == VX_OK)
      status = dit->Sample(mu, x, key, times, s);
    hipGraph_t graph = nullptr;
    const hipError_t ended = hipStreamEndCapture(s, &graph);
    if (status != VX_OK) {
      if (graph != nullptr)
        (void)hipGraphDestroy(graph);
      return status;
    }
    if (ended != hipSuccess)
      return vx::FailHip(ended, "vx_dit_patch: end capture");
    const hipError_t instantiated =
        hipGraphInstantiate(&dit->graph, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (instantiated != hipSuccess) {
      dit->graph = nullptr;
      return vx::FailHip(instantiated, "vx_dit_patch: instantiate");
    }
    dit->graph_key = key;
  }
  VX_HIP(hipGraphLaunch(dit->graph, s), "vx_dit_patch: graph launch");
  return vx::Succeed();
}

int vx_dit_set_path(vx_dit* dit, int path) {
  if (dit == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_dit_set_path: null handle");
  if (path == VX_DIT_PATH_PERSISTENT && !dit->persistent)
    return vx::Fail(VX_UNSUPPORTED, "vx_dit_set_path: no persistent kernel for this shape");
  if ((path == VX_DIT_PATH_FUSED || path == VX_DIT_PATH_FUSED_REFERENCE_ORDER) && !dit->fused)
    return vx::Fail(VX_UNSUPPORTED, "vx_dit_set_path: no fused kernels for this shape");
  if (path != VX_DIT_PATH_AUTO && path != VX_DIT_PATH_PERSISTENT &&
      path != VX_DIT_PATH_FUSED && path != VX_DIT_PATH_UNFUSED &&
      path != VX_DIT_PATH_FUSED_REFERENCE_ORDER)
    return vx::Fail(VX_BAD_ARG, "vx_dit_set_path: unknown path");
  dit->path = path;
  return vx::Succeed();
}

int vx_dit_set_trace(vx_dit* dit, void* buffer, size_t bytes) {
  if (dit == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_dit_set_trace: null handle");
  if (buffer != nullptr &&
      bytes < vx::persistent::TraceWords(static_cast<int>(dit->shape.layers), dit->grid) *
                  sizeof(unsigned long long))
    return vx::Fail(VX_BAD_ARG, "vx_dit_set_trace: buffer too small");
  dit->trace = static_cast<unsigned long long*>(buffer);
  return vx::Succeed();
}

size_t vx_dit_trace_bytes(const vx_dit* dit) {
  if (dit == nullptr || !dit->persistent)
    return 0;
  return vx::persistent::TraceWords(static_cast<int>(dit->shape.layers), dit->grid) *
         sizeof(unsigned long long);
}

int vx_dit_path(const vx_dit* dit) {
  return dit == nullptr ? -1 : dit->Resolved();
}

int vx_dit_status(vx_dit* dit) {
  if (dit == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_dit_status: null handle");
  if (!dit->persistent)
    return vx::Succeed();
  unsigned error = 0;
  VX_HIP(hipMemcpy(&error, dit->workspace.sync + vx::persistent::ErrorWord(),
                   sizeof error, hipMemcpyDeviceToHost),
         "vx_dit_status: read");
  if (error == 0)
    return vx::Succeed();
  // A barrier wait timed out: clear the counters for the next launch.
  VX_HIP(hipMemset(dit->workspace.sync, 0,
                   vx::persistent::SyncWords(dit->fused_shape,
                                             static_cast<int>(dit->shape.layers)) *
                       sizeof(unsigned)),
         "vx_dit_status: reset");
  return vx::Fail(VX_HIP_ERROR,
                  "vx_dit_status: a persistent evaluation timed out at a grid "
                  "barrier; its results are invalid");
}

int vx_euler_schedule(size_t timesteps, float sway, int skip, float* t,
                      float* dt, int32_t* evaluate) {
  // generator.cpp:21-37 (torch.linspace in float32), 63-80.
  if (timesteps == 0 || t == nullptr || dt == nullptr || evaluate == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_euler_schedule: bad arguments");
  const std::size_t count = timesteps + 1;
  std::vector<float> span(count);
  const float step = (0.0F - 1.0F) / static_cast<float>(count - 1);
  const std::size_t halfway = count / 2;
  // One rounding per value, as torch.linspace's float32 kernel does.
  for (std::size_t i = 0; i < count; ++i)
    span[i] = i < halfway
                  ? std::fma(step, static_cast<float>(i), 1.0F)
                  : std::fma(-step, static_cast<float>(count - i - 1), 0.0F);
  const auto quarter_turn = static_cast<float>(M_PI / 2.0);
  for (float& value : span)
    value = value + sway * (std::cos(quarter_turn * value) - 1.0F + value);
  const std::size_t zero_steps = std::max<std::size_t>(
      1, static_cast<std::size_t>(static_cast<double>(count) * 0.04));
  float time = span[0];
  float delta = span[0] - span[1];
  for (std::size_t i = 1; i < count; ++i) {
    t[i - 1] = time;
    dt[i - 1] = delta;
    evaluate[i - 1] = skip != 0 ? (i > zero_steps ? 1 : 0) : 1;
    time = time - delta;
    if (i < count - 1)
      delta = time - span[i + 1];
  }
  return vx::Succeed();
}

int vx_rope_table(double theta, size_t dim, const double* factors,
                  float scaling, size_t positions, float* table) {
  // transformer.cpp:20-45: all in float32.
  if (dim == 0 || dim % 2 != 0 || table == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_rope_table: bad arguments");
  const std::size_t half = dim / 2;
  std::vector<float> inverse(half), factor_inverse(half);
  for (std::size_t i = 0; i < half; ++i) {
    const float exponent = static_cast<float>(2 * i) / static_cast<float>(dim);
    inverse[i] = 1.0F / std::pow(static_cast<float>(theta), exponent);
    factor_inverse[i] =
        1.0F / (factors != nullptr ? static_cast<float>(factors[i]) : 1.0F);
  }
  for (std::size_t p = 0; p < positions; ++p)
    for (std::size_t i = 0; i < half; ++i) {
      const float angle = static_cast<float>(p) * factor_inverse[i] * inverse[i];
      table[p * dim + i] = std::cos(angle) * scaling;
      table[p * dim + half + i] = std::sin(angle) * scaling;
    }
  return vx::Succeed();
}

}  // extern "C"
