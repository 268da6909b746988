/*
 * CPU oracle of VoxCPM2's per-patch DiT hot path -- TEST INFRASTRUCTURE ONLY.
 * See oracle.h. Built with -ffp-contract=off so that every float32 operation
 * rounds as written (no fused multiply-adds beyond the explicit fmaf).
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---- scalar conversions ------------------------------------------------ */

uint16_t vo_bf16_bits(float value) {
  /* kernels/device_math.hpp:13-19 */
  uint32_t bits;
  memcpy(&bits, &value, sizeof bits);
  if ((bits & 0x7F800000u) == 0x7F800000u && (bits & 0x007FFFFFu) != 0)
    return (uint16_t)((bits >> 16) | 0x40u);
  return (uint16_t)((bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16);
}

float vo_bf16_value(uint16_t bits) {
  const uint32_t wide = (uint32_t)bits << 16;
  float value;
  memcpy(&value, &wide, sizeof value);
  return value;
}

float vo_half_value(uint16_t bits) {
  /* tests/products_test.cpp:46-57, plus infinities and NaN */
  const uint32_t sign = (bits >> 15) & 1u;
  const uint32_t exponent = (bits >> 10) & 0x1Fu;
  const uint32_t mantissa = bits & 0x3FFu;
  float value;
  if (exponent == 0x1F)
    value = mantissa == 0 ? INFINITY : NAN;
  else if (exponent == 0)
    value = ldexpf((float)mantissa, -24);
  else
    value = ldexpf((float)(mantissa | 0x400u), (int)exponent - 25);
  return sign ? -value : value;
}

uint16_t vo_half_bits(float value) {
  /* IEEE binary16, round to nearest even, subnormals kept. */
  uint32_t bits;
  memcpy(&bits, &value, sizeof bits);
  const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
  const float magnitude = fabsf(value);
  if (isnan(value))
    return (uint16_t)(sign | 0x7E00u);
  if (magnitude >= 65520.0f)
    return (uint16_t)(sign | 0x7C00u);
  if (magnitude < ldexpf(1.0f, -14)) {
    /* subnormal: units of 2^-24, ties to even by rintf */
    const float units = rintf(ldexpf(magnitude, 24));
    return (uint16_t)(sign | (uint16_t)units);
  }
  int exponent;
  const float fraction = frexpf(magnitude, &exponent); /* [0.5, 1) */
  float mantissa = rintf(ldexpf(fraction, 11));        /* [1024, 2048] */
  if (mantissa >= 2048.0f) {
    mantissa = 1024.0f;
    exponent += 1;
  }
  const int biased = exponent - 1 + 15;
  return (uint16_t)(sign | (uint16_t)(biased << 10) |
                    ((uint16_t)mantissa & 0x3FFu));
}

void vo_bf16_round_array(const float* input, uint16_t* output, size_t count) {
  for (size_t i = 0; i < count; ++i)
    output[i] = vo_bf16_bits(input[i]);
}

/* ---- Q8_0 --------------------------------------------------------------- */

static uint16_t block_scale(const uint8_t* block) {
  return (uint16_t)(block[0] | (block[1] << 8));
}

void vo_q8_dequant_bf16(const uint8_t* blocks, size_t n, size_t k,
                        uint16_t* output) {
  /* kernels/wmma_products.hip:94-112: Bf16Bits(HalfToFloat(scale) * q) */
  const size_t per_row = k / 32;
  for (size_t row = 0; row < n; ++row) {
    for (size_t b = 0; b < per_row; ++b) {
      const uint8_t* block = blocks + (row * per_row + b) * 34;
      const float scale = vo_half_value(block_scale(block));
      for (size_t i = 0; i < 32; ++i) {
        const float q = (float)(int8_t)block[2 + i];
        output[row * k + b * 32 + i] = vo_bf16_bits(scale * q);
      }
    }
  }
}

void vo_q8_values(const uint8_t* blocks, size_t n, size_t k, double* output) {
  const size_t per_row = k / 32;
  for (size_t row = 0; row < n; ++row) {
    for (size_t b = 0; b < per_row; ++b) {
      const uint8_t* block = blocks + (row * per_row + b) * 34;
      const double scale = vo_half_value(block_scale(block));
      for (size_t i = 0; i < 32; ++i)
        output[row * k + b * 32 + i] = scale * (double)(int8_t)block[2 + i];
    }
  }
}

typedef struct linear_job {
  const uint16_t* x;
  const uint8_t* blocks; /* Q8_0 blocks, or NULL for bf16 rows */
  const uint16_t* w16;   /* bf16 rows [n][k] */
  float* y;
  size_t m, k, n, first, last;
  int accumulate;
} linear_job;

/* kernels/wmma_products.hip:210-213: a float32 sum per 16-column chunk
 * (one WMMA step) added into the accumulator in k order. */
static void bf16_columns(const linear_job* job) {
  const size_t k = job->k;
  for (size_t row = 0; row < job->m; ++row) {
    const uint16_t* xr = job->x + row * k;
    for (size_t col = job->first; col < job->last; ++col) {
      const uint16_t* wr = job->w16 + col * k;
      float acc = 0.0f;
      for (size_t c0 = 0; c0 < k; c0 += 16) {
        const size_t c1 = c0 + 16 < k ? c0 + 16 : k;
        float chunk = 0.0f;
        for (size_t c = c0; c < c1; ++c)
          chunk += vo_bf16_value(xr[c]) * vo_bf16_value(wr[c]);
        acc += chunk;
      }
      float* target = job->y + row * job->n + col;
      *target = job->accumulate ? *target + acc : acc;
    }
  }
}

static void linear_columns(const linear_job* job) {
  if (job->blocks == NULL) {
    bf16_columns(job);
    return;
  }
  const size_t per_row = job->k / 32;
  float xs[32];
  for (size_t row = 0; row < job->m; ++row) {
    const uint16_t* xr = job->x + row * job->k;
    for (size_t col = job->first; col < job->last; ++col) {
      const uint8_t* w = job->blocks + col * per_row * 34;
      float acc = 0.0f;
      for (size_t b = 0; b < per_row; ++b) {
        const uint8_t* block = w + b * 34;
        for (size_t i = 0; i < 32; ++i)
          xs[i] = vo_bf16_value(xr[b * 32 + i]);
        /* The products of int8 and bf16 values are exact in float32. */
        float sum = 0.0f;
        for (size_t i = 0; i < 32; ++i)
          sum += (float)(int8_t)block[2 + i] * xs[i];
        acc = fmaf(vo_half_value(block_scale(block)), sum, acc);
      }
      float* target = job->y + row * job->n + col;
      *target = job->accumulate ? *target + acc : acc;
    }
  }
}

static void* linear_thread(void* argument) {
  linear_columns((const linear_job*)argument);
  return NULL;
}

static void run_linear(linear_job base, int threads);

void vo_q8_linear(const uint16_t* x, const uint8_t* blocks, float* y, size_t m,
                  size_t k, size_t n, int accumulate, int threads) {
  const linear_job base = {x, blocks, NULL, y, m, k, n, 0, 0, accumulate};
  run_linear(base, threads);
}

void vo_bf16_linear(const uint16_t* x, const uint16_t* w, float* y, size_t m,
                    size_t k, size_t n, int accumulate, int threads) {
  const linear_job base = {x, NULL, w, y, m, k, n, 0, 0, accumulate};
  run_linear(base, threads);
}

/* Columns n split over `threads` POSIX threads: identical results for any
 * count. */
static void run_linear(linear_job base, int threads) {
  const size_t n = base.n;
  if (threads < 1)
    threads = 1;
  if ((size_t)threads > n)
    threads = n > 0 ? (int)n : 1;
  linear_job jobs[256];
  pthread_t ids[256];
  if (threads > 256)
    threads = 256;
  const size_t chunk = (n + (size_t)threads - 1) / (size_t)threads;
  int started = 0;
  for (int t = 0; t < threads; ++t) {
    linear_job job = base;
    job.first = (size_t)t * chunk;
    job.last = (size_t)(t + 1) * chunk;
    if (job.last > n)
      job.last = n;
    if (job.first >= job.last)
      break;
    jobs[t] = job;
    ++started;
  }
  if (started == 1) {
    linear_columns(&jobs[0]);
    return;
  }
  for (int t = 0; t < started; ++t)
    pthread_create(&ids[t], NULL, linear_thread, &jobs[t]);
  for (int t = 0; t < started; ++t)
    pthread_join(ids[t], NULL);
}

double vo_q8_check(const float* y, const uint16_t* x, const uint8_t* blocks,
                   const float* before, size_t m, size_t k, size_t n) {
  /* tests/products_test.cpp:117-145 */
  const size_t per_row = k / 32;
  double worst = 0.0;
  for (size_t row = 0; row < m; ++row) {
    for (size_t col = 0; col < n; ++col) {
      double exact = before != NULL ? (double)before[row * n + col] : 0.0;
      double magnitude = 0.0;
      for (size_t b = 0; b < per_row; ++b) {
        const uint8_t* block = blocks + (col * per_row + b) * 34;
        const double scale = vo_half_value(block_scale(block));
        for (size_t i = 0; i < 32; ++i) {
          const double product = (double)vo_bf16_value(x[row * k + b * 32 + i]) *
                                 scale * (double)(int8_t)block[2 + i];
          exact += product;
          magnitude += fabs(product);
        }
      }
      const double error = fabs((double)y[row * n + col] - exact) /
                           (magnitude > 1e-30 ? magnitude : 1e-30);
      if (!(error <= worst))
        worst = error; /* NaN propagates as the worst */
    }
  }
  return worst;
}

/* ---- bfloat16 weights --------------------------------------------------- */

double vo_bf16_check(const float* y, const uint16_t* x, const uint16_t* w,
                     const float* before, size_t m, size_t k, size_t n) {
  /* tests/products_test.cpp:117-145 */
  double worst = 0.0;
  for (size_t row = 0; row < m; ++row) {
    for (size_t col = 0; col < n; ++col) {
      double exact = before != NULL ? (double)before[row * n + col] : 0.0;
      double magnitude = 0.0;
      for (size_t c = 0; c < k; ++c) {
        const double product =
            (double)vo_bf16_value(x[row * k + c]) * (double)vo_bf16_value(w[col * k + c]);
        exact += product;
        magnitude += fabs(product);
      }
      const double error = fabs((double)y[row * n + col] - exact) /
                           (magnitude > 1e-30 ? magnitude : 1e-30);
      if (!(error <= worst))
        worst = error; /* NaN propagates as the worst */
    }
  }
  return worst;
}

/* ---- generator kernels -------------------------------------------------- */

void vo_rms_norm(const float* input, const uint16_t* weight, uint16_t* output,
                 float* output_f32, size_t rows, size_t width, float epsilon) {
  /* kernels/generator_kernels.hip:91-108 */
  for (size_t row = 0; row < rows; ++row) {
    const float* x = input + row * width;
    float sum = 0.0f;
    for (size_t i = 0; i < width; ++i)
      sum += x[i] * x[i];
    const float inverse = 1.0f / sqrtf(sum / (float)width + epsilon);
    for (size_t i = 0; i < width; ++i) {
      const float value = x[i] * inverse * vo_bf16_value(weight[i]);
      output[row * width + i] = vo_bf16_bits(value);
      if (output_f32 != NULL)
        output_f32[row * width + i] = value;
    }
  }
}

void vo_rope_table(double theta, size_t dim, const double* factors,
                   float scaling, size_t positions, float* table) {
  /* transformer.cpp:20-45 */
  const size_t half = dim / 2;
  float* inverse = (float*)malloc(half * sizeof(float));
  float* factor_inverse = (float*)malloc(half * sizeof(float));
  for (size_t i = 0; i < half; ++i) {
    const float exponent = (float)(2 * i) / (float)dim;
    inverse[i] = 1.0f / powf((float)theta, exponent);
    factor_inverse[i] = 1.0f / (factors != NULL ? (float)factors[i] : 1.0f);
  }
  for (size_t p = 0; p < positions; ++p) {
    for (size_t i = 0; i < half; ++i) {
      const float angle = (float)p * factor_inverse[i] * inverse[i];
      table[p * dim + i] = cosf(angle) * scaling;
      table[p * dim + half + i] = sinf(angle) * scaling;
    }
  }
  free(inverse);
  free(factor_inverse);
}

void vo_qkv_rope(const float* qkv, const float* cos_sin,
                 const int32_t* positions, const int32_t* cache_rows, float* q,
                 float* k_cache, float* v_cache, size_t rows, size_t heads,
                 size_t kv_heads, size_t head_dim, size_t capacity) {
  /* kernels/generator_kernels.hip:110-158 */
  const size_t half = head_dim / 2;
  const size_t width = (heads + 2 * kv_heads) * head_dim;
  for (size_t row = 0; row < rows; ++row) {
    const float* source = qkv + row * width;
    const float* table =
        cos_sin == NULL ? NULL : cos_sin + (size_t)positions[row] * head_dim;
    const size_t cache_row = (size_t)cache_rows[row];
    for (size_t head = 0; head < heads + kv_heads; ++head) {
      for (size_t i = 0; i < half; ++i) {
        const float a = source[head * head_dim + i];
        const float b = source[head * head_dim + half + i];
        float first = a, second = b;
        if (table != NULL) {
          const float c = table[i], s = table[half + i];
          first = a * c - b * s;
          second = b * c + a * s;
        }
        float* target =
            head < heads
                ? q + (row * heads + head) * head_dim
                : k_cache + ((head - heads) * capacity + cache_row) * head_dim;
        target[i] = first;
        target[half + i] = second;
      }
    }
    const float* v = source + (heads + kv_heads) * head_dim;
    for (size_t index = 0; index < kv_heads * head_dim; ++index) {
      const size_t head = index / head_dim;
      v_cache[(head * capacity + cache_row) * head_dim + index % head_dim] =
          v[index];
    }
  }
}

void vo_attention(const float* q, const float* k_cache, const float* v_cache,
                  uint16_t* output, size_t rows, size_t rows_per_sequence,
                  size_t keys_per_sequence, size_t past, int causal,
                  size_t heads, size_t kv_heads, size_t head_dim,
                  size_t capacity) {
  /* kernels/generator_kernels.hip:160-241: scaled query, online softmax. */
  const float scale = 1.0f / sqrtf((float)head_dim);
  float* query = (float*)malloc(head_dim * sizeof(float));
  float* out = (float*)malloc(head_dim * sizeof(float));
  for (size_t row = 0; row < rows; ++row) {
    const size_t sequence = row / rows_per_sequence;
    const size_t local = row % rows_per_sequence;
    const size_t count = past + (causal ? local + 1 : rows_per_sequence);
    const size_t first_key = sequence * keys_per_sequence;
    for (size_t head = 0; head < heads; ++head) {
      const size_t kv_head = head / (heads / kv_heads);
      const float* keys = k_cache + (kv_head * capacity + first_key) * head_dim;
      const float* values =
          v_cache + (kv_head * capacity + first_key) * head_dim;
      for (size_t d = 0; d < head_dim; ++d) {
        query[d] = q[(row * heads + head) * head_dim + d] * scale;
        out[d] = 0.0f;
      }
      float maximum = -INFINITY, sum = 0.0f;
      for (size_t key = 0; key < count; ++key) {
        float score = 0.0f;
        for (size_t d = 0; d < head_dim; ++d)
          score += query[d] * keys[key * head_dim + d];
        const float next = fmaxf(maximum, score);
        const float decay = expf(maximum - next);
        const float weight = expf(score - next);
        sum = sum * decay + weight;
        for (size_t d = 0; d < head_dim; ++d)
          out[d] = out[d] * decay + weight * values[key * head_dim + d];
        maximum = next;
      }
      const float inverse = 1.0f / sum;
      for (size_t d = 0; d < head_dim; ++d)
        output[(row * heads + head) * head_dim + d] =
            vo_bf16_bits(out[d] * inverse);
    }
  }
  free(query);
  free(out);
}

void vo_swiglu(const float* gate_up, uint16_t* output, size_t rows,
               size_t width) {
  /* kernels/generator_kernels.hip:243-254 */
  for (size_t row = 0; row < rows; ++row) {
    for (size_t i = 0; i < width; ++i) {
      const float gate = gate_up[row * 2 * width + i];
      const float up = gate_up[row * 2 * width + width + i];
      output[row * width + i] = vo_bf16_bits(gate / (1.0f + expf(-gate)) * up);
    }
  }
}

void vo_add_bias(float* data, const uint16_t* bias, size_t rows, size_t width) {
  /* kernels/generator_kernels.hip:256-262 */
  for (size_t i = 0; i < rows * width; ++i)
    data[i] += vo_bf16_value(bias[i % width]);
}

void vo_to_bf16(const float* input, uint16_t* output, size_t count, int silu) {
  /* kernels/generator_kernels.hip:264-274 */
  for (size_t i = 0; i < count; ++i) {
    float value = input[i];
    if (silu)
      value = value / (1.0f + expf(-value));
    output[i] = vo_bf16_bits(value);
  }
}

void vo_gather_rows(const float* input, const int32_t* indices, float* output,
                    size_t rows, size_t width) {
  /* kernels/generator_kernels.hip:82-89 */
  for (size_t row = 0; row < rows; ++row)
    memcpy(output + row * width, input + (size_t)indices[row] * width,
           width * sizeof(float));
}

void vo_assemble_dit(const float* mu, const float* time, const float* cond,
                     const float* x, float* output, size_t patch,
                     size_t width) {
  /* kernels/generator_kernels.hip:320-340 */
  const size_t length = 3 + 2 * patch;
  for (size_t sequence = 0; sequence < 2; ++sequence) {
    for (size_t row = 0; row < length; ++row) {
      float* target = output + (sequence * length + row) * width;
      for (size_t i = 0; i < width; ++i) {
        float value;
        if (row < 2)
          value = sequence == 0 ? mu[row * width + i] : 0.0f;
        else if (row == 2)
          value = time[i];
        else if (row < 3 + patch)
          value = cond[(row - 3) * width + i];
        else
          value = x[(row - 3 - patch) * width + i];
        target[i] = value;
      }
    }
  }
}

void vo_guided_euler(const float* velocity, float* x, size_t count, float cfg,
                     float dt, int zero_star) {
  /* kernels/generator_kernels.hip:342-360 */
  const float* c = velocity;
  const float* u = velocity + count;
  float dot = 0.0f, norm = 0.0f;
  for (size_t i = 0; i < count; ++i) {
    dot += c[i] * u[i];
    norm += u[i] * u[i];
  }
  const float s = zero_star ? dot / (norm + 1e-8f) : 1.0f;
  for (size_t i = 0; i < count; ++i) {
    const float guided = u[i] * s + cfg * (c[i] - u[i] * s);
    x[i] -= dt * guided;
  }
}

/* ---- sampler ------------------------------------------------------------ */

void vo_linspace(float start, float end, size_t steps, float* values) {
  /* generator.cpp:21-37: the first half counts up from start, the second
   * half down from end. Each value rounds once, as torch.linspace's float32
   * kernel does (the reference's start + step * index contracted to a
   * fused multiply-add). */
  if (steps == 1) {
    values[0] = start;
    return;
  }
  const float step = (end - start) / (float)(steps - 1);
  const size_t halfway = steps / 2;
  for (size_t index = 0; index < steps; ++index)
    values[index] = index < halfway
                        ? fmaf(step, (float)index, start)
                        : fmaf(-step, (float)(steps - index - 1), end);
}

void vo_euler_schedule(size_t timesteps, float sway, int skip, float* t_out,
                       float* dt_out, int32_t* evaluate) {
  /* generator.cpp:63-80 */
  const size_t count = timesteps + 1;
  float* span = (float*)malloc(count * sizeof(float));
  vo_linspace(1.0f, 0.0f, count, span);
  const float quarter_turn = (float)(M_PI / 2.0);
  for (size_t i = 0; i < count; ++i)
    span[i] = span[i] + sway * (cosf(quarter_turn * span[i]) - 1.0f + span[i]);
  size_t zero_steps = (size_t)((double)count * 0.04);
  if (zero_steps < 1)
    zero_steps = 1;
  float t = span[0];
  float dt = span[0] - span[1];
  for (size_t step = 1; step < count; ++step) {
    t_out[step - 1] = t;
    dt_out[step - 1] = dt;
    evaluate[step - 1] = skip ? (step > zero_steps) : 1;
    t = t - dt;
    if (step < count - 1)
      dt = t - span[step + 1];
  }
  free(span);
}

void vo_sinusoid(float t, size_t width, float* embedding) {
  /* generator.cpp:40-53 */
  const size_t half = width / 2;
  const float exponent = (float)(log(10000.0) / (double)(half - 1));
  const float scaled = 1000.0f * t;
  for (size_t i = 0; i < half; ++i) {
    const float frequency = expf((float)i * -exponent);
    const float angle = scaled * frequency;
    embedding[i] = sinf(angle);
    embedding[half + i] = cosf(angle);
  }
}

/* ---- the local DiT ------------------------------------------------------ */

/* Project (transformer.cpp:47-53): y = x W^T (+ b). */
/* A product on the DiT's matrices: Q8_0 blocks, or bf16 rows when
 * `bf16_weights` is set (the reference's kBf16Tiles stacks). */
static void dit_linear(const vo_dit* dit, const uint16_t* x, const uint8_t* w,
                       float* y, size_t rows, size_t in, size_t out,
                       int accumulate) {
  if (dit->bf16_weights)
    vo_bf16_linear(x, (const uint16_t*)w, y, rows, in, out, accumulate,
                   dit->threads);
  else
    vo_q8_linear(x, w, y, rows, in, out, accumulate, dit->threads);
}

static void project(const vo_dit* dit, const vo_projection* p,
                    const uint16_t* x, float* y, size_t rows, size_t in,
                    size_t out) {
  dit_linear(dit, x, p->weight, y, rows, in, out, 0);
  if (p->bias != NULL)
    vo_add_bias(y, p->bias, rows, out);
}

void vo_dit_time_vector(const vo_dit* dit, float t, float* vector) {
  /* generator.cpp:212-237 and the delta_time precomputation :150-167 */
  const size_t width = dit->hidden;
  const size_t in = dit->time_in;
  const size_t wide = in > width ? in : width;
  float* embedding = (float*)malloc(wide * sizeof(float));
  uint16_t* bf16 = (uint16_t*)malloc(wide * sizeof(uint16_t));
  float* middle = (float*)malloc(width * sizeof(float));
  if (dit->has_delta) {
    vo_sinusoid(0.0f, in, embedding);
    vo_to_bf16(embedding, bf16, in, 0);
    project(dit, &dit->delta_1, bf16, middle, 1, in, width);
    vo_to_bf16(middle, bf16, width, 1);
    project(dit, &dit->delta_2, bf16, vector, 1, width, width);
  } else {
    memset(vector, 0, width * sizeof(float));
  }
  vo_sinusoid(t, in, embedding);
  vo_to_bf16(embedding, bf16, in, 0);
  project(dit, &dit->time_1, bf16, middle, 1, in, width);
  vo_to_bf16(middle, bf16, width, 1);
  /* vector (the delta term) += time_2 . silu(middle), then the bias */
  dit_linear(dit, bf16, dit->time_2.weight, vector, 1, width, width, 1);
  if (dit->time_2.bias != NULL)
    vo_add_bias(vector, dit->time_2.bias, 1, width);
  free(embedding);
  free(bf16);
  free(middle);
}

void vo_dit_cond_rows(const vo_dit* dit, const float* cond_latent,
                      float* cond_rows) {
  const size_t values = dit->patch * dit->feat;
  uint16_t* bf16 = (uint16_t*)malloc(values * sizeof(uint16_t));
  vo_to_bf16(cond_latent, bf16, values, 0);
  project(dit, &dit->cond_proj, bf16, cond_rows, dit->patch, dit->feat,
          dit->hidden);
  free(bf16);
}

void vo_dit_eval(const vo_dit* dit, const float* mu, const float* cond_rows,
                 const float* x, const float* time_vector, float* velocity) {
  /* generator.cpp:297-324, transformer.cpp:55-100 */
  const size_t width = dit->hidden, patch = dit->patch, feat = dit->feat;
  const size_t length = 3 + 2 * patch;
  const size_t rows = 2 * length;
  const size_t q_width = dit->heads * dit->head_dim;
  const size_t kv_width = dit->kv_heads * dit->head_dim;
  const size_t qkv_width = q_width + 2 * kv_width;
  const size_t ffn = dit->ffn;
  const size_t wide = ffn > qkv_width ? ffn : qkv_width;
  uint16_t* bf16 = (uint16_t*)malloc(rows * (wide > width ? wide : width) *
                                     sizeof(uint16_t));
  float* x_rows = (float*)malloc(patch * width * sizeof(float));
  float* hidden = (float*)malloc(rows * width * sizeof(float));
  float* output = (float*)malloc(rows * width * sizeof(float));
  float* qkv = (float*)malloc(rows * qkv_width * sizeof(float));
  float* q = (float*)malloc(rows * q_width * sizeof(float));
  float* k_cache = (float*)malloc(rows * kv_width * sizeof(float));
  float* v_cache = (float*)malloc(rows * kv_width * sizeof(float));
  float* gate_up = (float*)malloc(rows * 2 * ffn * sizeof(float));
  int32_t* positions = (int32_t*)malloc(rows * sizeof(int32_t));
  int32_t* cache_rows = (int32_t*)malloc(rows * sizeof(int32_t));
  int32_t* outputs = (int32_t*)malloc(2 * patch * sizeof(int32_t));
  for (size_t row = 0; row < rows; ++row) {
    positions[row] = (int32_t)(row % length);
    cache_rows[row] = (int32_t)row;
  }
  for (size_t s = 0; s < 2; ++s)
    for (size_t i = 0; i < patch; ++i)
      outputs[s * patch + i] = (int32_t)(s * length + 3 + patch + i);

  vo_to_bf16(x, bf16, patch * feat, 0);
  project(dit, &dit->in_proj, bf16, x_rows, patch, feat, width);
  vo_assemble_dit(mu, time_vector, cond_rows, x_rows, hidden, patch, width);
  for (size_t l = 0; l < dit->layers; ++l) {
    const vo_layer* layer = &dit->layer[l];
    vo_rms_norm(hidden, layer->input_norm, bf16, NULL, rows, width, dit->eps);
    dit_linear(dit, bf16, layer->qkv, qkv, rows, width, qkv_width, 0);
    vo_qkv_rope(qkv, dit->rope, positions, cache_rows, q, k_cache, v_cache,
                rows, dit->heads, dit->kv_heads, dit->head_dim, rows);
    vo_attention(q, k_cache, v_cache, bf16, rows, length, length, 0, 0,
                 dit->heads, dit->kv_heads, dit->head_dim, rows);
    dit_linear(dit, bf16, layer->o, hidden, rows, q_width, width, 1);
    vo_rms_norm(hidden, layer->post_norm, bf16, NULL, rows, width, dit->eps);
    dit_linear(dit, bf16, layer->gate_up, gate_up, rows, width, 2 * ffn, 0);
    vo_swiglu(gate_up, bf16, rows, ffn);
    dit_linear(dit, bf16, layer->down, hidden, rows, ffn, width, 1);
  }
  vo_rms_norm(hidden, dit->norm, bf16, output, rows, width, dit->eps);
  vo_gather_rows(output, outputs, hidden, 2 * patch, width);
  vo_to_bf16(hidden, bf16, 2 * patch * width, 0);
  project(dit, &dit->out_proj, bf16, velocity, 2 * patch, width, feat);

  free(bf16);
  free(x_rows);
  free(hidden);
  free(output);
  free(qkv);
  free(q);
  free(k_cache);
  free(v_cache);
  free(gate_up);
  free(positions);
  free(cache_rows);
  free(outputs);
}

void vo_dit_velocity(const vo_dit* dit, const float* mu,
                     const float* cond_latent, const float* x, float t,
                     float* velocity) {
  /* generator.cpp:515-538 */
  float* cond_rows = (float*)malloc(dit->patch * dit->hidden * sizeof(float));
  float* time = (float*)malloc(dit->hidden * sizeof(float));
  vo_dit_cond_rows(dit, cond_latent, cond_rows);
  vo_dit_time_vector(dit, t, time);
  vo_dit_eval(dit, mu, cond_rows, x, time, velocity);
  free(cond_rows);
  free(time);
}

void vo_dit_patch(const vo_dit* dit, const float* mu, const float* cond_latent,
                  float* x, const float* t, const float* dt,
                  const int32_t* evaluate, size_t steps, float cfg,
                  int zero_star) {
  /* generator.cpp:448-463 */
  const size_t values = dit->patch * dit->feat;
  float* cond_rows = (float*)malloc(dit->patch * dit->hidden * sizeof(float));
  float* time = (float*)malloc(dit->hidden * sizeof(float));
  float* velocity = (float*)malloc(2 * values * sizeof(float));
  vo_dit_cond_rows(dit, cond_latent, cond_rows);
  for (size_t step = 0; step < steps; ++step) {
    if (!evaluate[step])
      continue; /* zero velocity */
    vo_dit_time_vector(dit, t[step], time);
    vo_dit_eval(dit, mu, cond_rows, x, time, velocity);
    vo_guided_euler(velocity, x, values, cfg, dt[step], zero_star);
  }
  free(cond_rows);
  free(time);
  free(velocity);
}

/* ---- one MiniCPM4 stack with a key/value cache --------------------------- */

static void stack_linear(const vo_stack* stack, const uint16_t* x,
                         const uint8_t* w, float* y, size_t rows, size_t in,
                         size_t out, int accumulate) {
  if (stack->bf16_weights)
    vo_bf16_linear(x, (const uint16_t*)w, y, rows, in, out, accumulate,
                   stack->threads);
  else
    vo_q8_linear(x, w, y, rows, in, out, accumulate, stack->threads);
}

void vo_stack_forward(const vo_stack* stack, float* hidden, float* output,
                      size_t rows, const int32_t* positions,
                      const int32_t* cache_rows, size_t rows_per_sequence,
                      size_t keys_per_sequence, size_t past, int causal,
                      float* k_cache, float* v_cache, size_t capacity) {
  /* transformer.cpp:55-100 */
  const size_t width = stack->hidden;
  const size_t q_width = stack->heads * stack->head_dim;
  const size_t kv_width = stack->kv_heads * stack->head_dim;
  const size_t qkv_width = q_width + 2 * kv_width;
  const size_t ffn = stack->ffn;
  const size_t layer_stride = stack->kv_heads * capacity * stack->head_dim;
  size_t wide = ffn > qkv_width ? ffn : qkv_width;
  if (width > wide)
    wide = width;
  uint16_t* bf16 = (uint16_t*)malloc(rows * wide * sizeof(uint16_t));
  float* qkv = (float*)malloc(rows * qkv_width * sizeof(float));
  float* q = (float*)malloc(rows * q_width * sizeof(float));
  float* gate_up = (float*)malloc(rows * 2 * ffn * sizeof(float));
  for (size_t l = 0; l < stack->layers; ++l) {
    const vo_layer* layer = &stack->layer[l];
    float* keys = k_cache + l * layer_stride;
    float* values = v_cache + l * layer_stride;
    vo_rms_norm(hidden, layer->input_norm, bf16, NULL, rows, width, stack->eps);
    stack_linear(stack, bf16, layer->qkv, qkv, rows, width, qkv_width, 0);
    vo_qkv_rope(qkv, stack->rope, positions, cache_rows, q, keys, values, rows,
                stack->heads, stack->kv_heads, stack->head_dim, capacity);
    vo_attention(q, keys, values, bf16, rows, rows_per_sequence,
                 keys_per_sequence, past, causal, stack->heads,
                 stack->kv_heads, stack->head_dim, capacity);
    stack_linear(stack, bf16, layer->o, hidden, rows, q_width, width, 1);
    vo_rms_norm(hidden, layer->post_norm, bf16, NULL, rows, width, stack->eps);
    stack_linear(stack, bf16, layer->gate_up, gate_up, rows, width, 2 * ffn, 0);
    vo_swiglu(gate_up, bf16, rows, ffn);
    stack_linear(stack, bf16, layer->down, hidden, rows, ffn, width, 1);
  }
  vo_rms_norm(hidden, stack->norm, bf16, output, rows, width, stack->eps);
  free(bf16);
  free(qkv);
  free(q);
  free(gate_up);
}

/* ---- AudioVAE V2's causal decoder --------------------------------------- */

/* x + (1 / (alpha + 1e-9)) sin^2(alpha x) (kernels/vae_kernels.hip:19-34),
 * after the optional rate conditioning x scale + bias. */
static void vae_snake(float* data, size_t t, size_t c, const float* alpha,
                      const float* scale, const float* bias) {
  for (size_t i = 0; i < t * c; ++i) {
    const size_t ch = i % c;
    float y = data[i];
    if (scale != NULL)
      y = y * scale[ch] + bias[ch];
    const float a = alpha[ch];
    const float s = sinf(a * y);
    data[i] = y + (1.0f / (a + 1e-9f)) * (s * s);
  }
}

/* Causal depthwise convolution, kernel 7, dilation d, zero history
 * (vae_kernels.hip:36-53). */
static void vae_depthwise(const float* in, const float* w, const float* b,
                          float* out, size_t t, size_t c, size_t d) {
  for (size_t f = 0; f < t; ++f)
    for (size_t ch = 0; ch < c; ++ch) {
      float sum = b[ch];
      for (size_t j = 0; j < 7; ++j) {
        const long src = (long)f + (long)(j * d) - (long)(6 * d);
        if (src >= 0)
          sum += w[ch * 7 + j] * in[(size_t)src * c + ch];
      }
      out[f * c + ch] = sum;
    }
}

/* y[t][o] (+)= sum_i w[o][i] x[t][i] + b[o]. */
static void vae_pointwise(const float* x, const float* w, const float* b,
                          float* y, size_t t, size_t in, size_t out,
                          int accumulate) {
  for (size_t f = 0; f < t; ++f)
    for (size_t o = 0; o < out; ++o) {
      float sum = 0.0f;
      for (size_t i = 0; i < in; ++i)
        sum += w[o * in + i] * x[f * in + i];
      sum += b[o];
      y[f * out + o] = accumulate ? y[f * out + o] + sum : sum;
    }
}

void vo_vae_decode(const vo_vae* vae, const float* latents, size_t frames,
                   float* samples) {
  /* vae.cpp:415-481 */
  size_t widest = frames * (vae->latent > vae->decoder_dim ? vae->latent
                                                           : vae->decoder_dim);
  size_t length = frames, channels = vae->decoder_dim;
  for (size_t b = 0; b < vae->block_count; ++b) {
    length *= vae->blocks[b].stride;
    channels /= 2;
    if (length * channels > widest)
      widest = length * channels;
  }
  float* hidden = (float*)malloc(widest * sizeof(float));
  float* next = (float*)malloc(widest * sizeof(float));
  float* work = (float*)malloc(widest * sizeof(float));
  float* scratch = (float*)malloc(widest * sizeof(float));

  /* Input: depthwise (latent channels), then pointwise to decoder_dim. */
  vae_depthwise(latents, vae->in_depthwise, vae->in_depthwise_bias, scratch,
                frames, vae->latent, 1);
  vae_pointwise(scratch, vae->in_pointwise, vae->in_pointwise_bias, hidden,
                frames, vae->latent, vae->decoder_dim, 0);
  size_t t = frames, c = vae->decoder_dim;
  static const size_t dilations[3] = {1, 3, 9};
  for (size_t b = 0; b < vae->block_count; ++b) {
    const vo_vae_block* block = &vae->blocks[b];
    const size_t in = c, out = c / 2, s = block->stride;
    memcpy(work, hidden, t * in * sizeof(float));
    vae_snake(work, t, in, block->alpha, block->scale, block->bias);
    /* ConvTranspose1d, kernel 2s, stride s, the first t s outputs:
     * out[f s + r][o] = b[o] + sum_i W[i][o][r] x[f][i]
     *                        + sum_i W[i][o][r + s] x[f - 1][i]. */
    for (size_t f = 0; f < t; ++f)
      for (size_t r = 0; r < s; ++r)
        for (size_t o = 0; o < out; ++o) {
          float sum = 0.0f;
          for (size_t i = 0; i < in; ++i)
            sum += block->up[(i * out + o) * 2 * s + r] * work[f * in + i];
          if (f > 0)
            for (size_t i = 0; i < in; ++i)
              sum += block->up[(i * out + o) * 2 * s + r + s] *
                     work[(f - 1) * in + i];
          next[(f * s + r) * out + o] = sum + block->up_bias[o];
        }
    t *= s;
    c = out;
    memcpy(hidden, next, t * c * sizeof(float));
    for (size_t u = 0; u < 3; ++u) {
      const vo_vae_unit* unit = &block->units[u];
      memcpy(work, hidden, t * c * sizeof(float));
      vae_snake(work, t, c, unit->alpha_in, NULL, NULL);
      vae_depthwise(work, unit->depthwise, unit->depthwise_bias, scratch, t, c,
                    dilations[u]);
      vae_snake(scratch, t, c, unit->alpha_out, NULL, NULL);
      vae_pointwise(scratch, unit->pointwise, unit->pointwise_bias, hidden, t,
                    c, c, 1);
    }
  }
  /* Output: Snake, causal conv c -> 1 (kernel 7), tanh
   * (vae_kernels.hip:70-93). */
  memcpy(work, hidden, t * c * sizeof(float));
  vae_snake(work, t, c, vae->out_alpha, NULL, NULL);
  for (size_t f = 0; f < t; ++f) {
    float sum = 0.0f;
    for (size_t ch = 0; ch < c; ++ch)
      for (size_t j = 0; j < 7; ++j) {
        const long src = (long)f + (long)j - 6;
        if (src >= 0)
          sum += vae->out_conv[ch * 7 + j] * work[(size_t)src * c + ch];
      }
    samples[f] = tanhf(sum + vae->out_bias);
  }
  free(hidden);
  free(next);
  free(work);
  free(scratch);
}
