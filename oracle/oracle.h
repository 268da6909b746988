/*
 * CPU oracle of VoxCPM2's per-patch DiT hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * A scalar restatement, in plain C, of the arithmetic of the reference
 * (gufo-extensions/voxcpm) on the path: GGML Q8_0 block decoding, the
 * block-scaled Q8_0 x bfloat16 products, the generator kernels of the local
 * DiT, its CFM Euler sampler and the time embedding. Each function cites the
 * reference file:line it follows.
 *
 * Only the tests, the smoke check and the benchmark's CPU-baseline leg use
 * this library, as the checker and as the timed CPU baseline. The product
 * path (voxcpm_amd) never links, loads or calls it.
 */
#ifndef VOXCPM_ORACLE_H_
#define VOXCPM_ORACLE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions ------------------------------------------------ */

/* float32 -> bfloat16 bits, round to nearest even, NaN kept quiet
 * (kernels/device_math.hpp:13-19). */
uint16_t vo_bf16_bits(float value);
float vo_bf16_value(uint16_t bits);
/* float16 bits -> float32 with subnormals (tests/products_test.cpp:46-57). */
float vo_half_value(uint16_t bits);
/* float32 -> float16 bits, round to nearest even (synthetic scales only). */
uint16_t vo_half_bits(float value);

void vo_bf16_round_array(const float* input, uint16_t* output, size_t count);

/* ---- Q8_0 --------------------------------------------------------------- */

/* bf16(f32(f16 scale) * q) of GGML Q8_0 blocks [n][k/32]
 * (kernels/wmma_products.hip:94-112, kernels/convert_kernels.hip:27-38). */
void vo_q8_dequant_bf16(const uint8_t* blocks, size_t n, size_t k,
                        uint16_t* output);

/* The exact values scale * q in double (tests/products_test.cpp:65-86). */
void vo_q8_values(const uint8_t* blocks, size_t n, size_t k, double* output);

/* y[m][n] (+)= x[m][k] . W[n][k]^T for bf16 x and Q8_0 W, in the reference
 * order (kernels/wmma_products.hip:203-209, 242-243): per 32-column block a
 * float32 sum of the exact products, then acc = fmaf(scale, sum, acc);
 * y = accumulate ? y + acc : acc. `threads` > 1 splits the columns n over
 * POSIX threads (identical results for any count). */
void vo_q8_linear(const uint16_t* x, const uint8_t* blocks, float* y, size_t m,
                  size_t k, size_t n, int accumulate, int threads);

/* Worst |y - exact| / sum|x*w| over all outputs, exact in double
 * (tests/products_test.cpp:117-145). `before` is the y the product
 * accumulated into, or NULL. */
double vo_q8_check(const float* y, const uint16_t* x, const uint8_t* blocks,
                   const float* before, size_t m, size_t k, size_t n);

/* ---- bfloat16 weights --------------------------------------------------- */

/* y[m][n] (+)= x[m][k] . W[n][k]^T for bf16 x and bf16 rows W, in the
 * reference's bf16 order (kernels/wmma_products.hip:210-213): per
 * 16-column chunk (one v_wmma_f32_16x16x16_bf16) a float32 sum of the
 * products, added into the float32 accumulator in k order; the order
 * inside a chunk is the hardware's. y = accumulate ? y + acc : acc.
 * k a multiple of 8 (a last, short chunk is summed the same way).
 * `threads` splits the columns n (identical results for any count). */
void vo_bf16_linear(const uint16_t* x, const uint16_t* w, float* y, size_t m,
                    size_t k, size_t n, int accumulate, int threads);

/* Worst |y - exact| / sum|x*w| over all outputs for bf16 rows W, exact in
 * double (tests/products_test.cpp:117-145, used with bf16 weights at
 * :234-237). `before` is the y the product accumulated into, or NULL. */
double vo_bf16_check(const float* y, const uint16_t* x, const uint16_t* w,
                     const float* before, size_t m, size_t k, size_t n);

/* ---- generator kernels (kernels/generator_kernels.hip) ---------------- */

/* :91-108 */
void vo_rms_norm(const float* input, const uint16_t* weight, uint16_t* output,
                 float* output_f32, size_t rows, size_t width, float epsilon);

/* transformer.cpp:20-45: [positions][cos (dim/2) | sin (dim/2)]. `factors`
 * holds dim/2 LongRoPE factors or is NULL (all 1). */
void vo_rope_table(double theta, size_t dim, const double* factors,
                   float scaling, size_t positions, float* table);

/* :110-158 */
void vo_qkv_rope(const float* qkv, const float* cos_sin,
                 const int32_t* positions, const int32_t* cache_rows, float* q,
                 float* k_cache, float* v_cache, size_t rows, size_t heads,
                 size_t kv_heads, size_t head_dim, size_t capacity);

/* :160-241 (any head_dim) */
void vo_attention(const float* q, const float* k_cache, const float* v_cache,
                  uint16_t* output, size_t rows, size_t rows_per_sequence,
                  size_t keys_per_sequence, size_t past, int causal,
                  size_t heads, size_t kv_heads, size_t head_dim,
                  size_t capacity);

/* :243-254 */
void vo_swiglu(const float* gate_up, uint16_t* output, size_t rows,
               size_t width);
/* :256-262 */
void vo_add_bias(float* data, const uint16_t* bias, size_t rows, size_t width);
/* :264-274 */
void vo_to_bf16(const float* input, uint16_t* output, size_t count, int silu);
/* :82-89 */
void vo_gather_rows(const float* input, const int32_t* indices, float* output,
                    size_t rows, size_t width);
/* :320-340 */
void vo_assemble_dit(const float* mu, const float* time, const float* cond,
                     const float* x, float* output, size_t patch, size_t width);
/* :342-360; zero_star = 0 takes s = 1 (plain CFG). */
void vo_guided_euler(const float* velocity, float* x, size_t count, float cfg,
                     float dt, int zero_star);

/* ---- sampler (generator.cpp) ------------------------------------------ */

/* :21-37 torch.linspace in float32 */
void vo_linspace(float start, float end, size_t steps, float* values);
/* :63-80; `skip` marks the first max(1, int(0.04 (n + 1))) steps as not
 * evaluated (CFG-Zero*). Writes n entries. */
void vo_euler_schedule(size_t timesteps, float sway, int skip, float* t,
                       float* dt, int32_t* evaluate);
/* :40-53 */
void vo_sinusoid(float t, size_t width, float* embedding);

/* ---- the local DiT ------------------------------------------------------ */

typedef struct vo_projection {
  const uint8_t* weight; /* GGML Q8_0 blocks [out][in/32], or bf16 rows
                            [out][in] (vo_dit.bf16_weights) */
  const uint16_t* bias;  /* bf16 [out] or NULL */
} vo_projection;

typedef struct vo_layer {
  const uint16_t* input_norm; /* bf16 [hidden] */
  const uint8_t* qkv;         /* [(heads + 2 kv_heads) head_dim][hidden] */
  const uint8_t* o;           /* [hidden][heads head_dim] */
  const uint16_t* post_norm;  /* bf16 [hidden] */
  const uint8_t* gate_up;     /* [2 ffn][hidden]: gate rows, then up rows */
  const uint8_t* down;        /* [hidden][ffn] */
} vo_layer;

typedef struct vo_dit {
  size_t hidden, heads, kv_heads, head_dim, ffn, layers;
  size_t patch, feat, time_in;
  float eps;
  int has_delta;     /* delta_time_mlp(sinusoid(0)) is added */
  const float* rope; /* [>= 3 + 2 patch][head_dim] or NULL */
  const vo_layer* layer;
  const uint16_t* norm; /* final norm, bf16 [hidden] */
  vo_projection in_proj, cond_proj, out_proj;
  vo_projection time_1, time_2, delta_1, delta_2;
  int threads; /* for the products */
  int bf16_weights; /* every matrix is bf16 rows [out][in] instead of Q8_0
                       blocks (weights.cpp:281-282, kBf16Tiles stacks) */
} vo_dit;

/* TimeVector (generator.cpp:212-237, 150-167): [hidden]. */
void vo_dit_time_vector(const vo_dit* dit, float t, float* vector);
/* cond_proj of the prefix latent [patch][feat] -> [patch][hidden]
 * (generator.cpp:448-451). */
void vo_dit_cond_rows(const vo_dit* dit, const float* cond_latent,
                      float* cond_rows);
/* One CFG-pair evaluation, EvaluateDit (generator.cpp:297-324) with
 * ForwardStack (transformer.cpp:55-100): velocity [2][patch][feat]. */
void vo_dit_eval(const vo_dit* dit, const float* mu, const float* cond_rows,
                 const float* x, const float* time_vector, float* velocity);
/* Velocity (generator.cpp:515-538). */
void vo_dit_velocity(const vo_dit* dit, const float* mu,
                     const float* cond_latent, const float* x, float t,
                     float* velocity);
/* The sampler of Step (generator.cpp:448-463) over a given schedule. */
void vo_dit_patch(const vo_dit* dit, const float* mu, const float* cond_latent,
                  float* x, const float* t, const float* dt,
                  const int32_t* evaluate, size_t steps, float cfg,
                  int zero_star);

/* ---- one MiniCPM4 stack with a key/value cache (the LMs, the encoder) -- */

typedef struct vo_stack {
  size_t hidden, heads, kv_heads, head_dim, ffn, layers;
  float eps;
  const float* rope; /* rotary table [positions][head_dim], or NULL for a
                        stack without rotary embedding (the residual LM) */
  const vo_layer* layer;
  const uint16_t* norm; /* final norm, bf16 [hidden] */
  int threads;          /* for the products */
  int bf16_weights;     /* bf16 rows [out][in] instead of Q8_0 blocks */
} vo_stack;

/* ForwardStack (transformer.cpp:55-100): `rows` rows of the float32
 * residual stream hidden [rows][hidden] (updated in place) through every
 * layer, the final norm's float32 output to output [rows][hidden]. Each
 * layer writes its rows' keys and values into k_cache / v_cache
 * [layer][kv_head][capacity][head_dim] at cache_rows and attends as
 * vo_attention does (rows_per_sequence, keys_per_sequence, past, causal). */
void vo_stack_forward(const vo_stack* stack, float* hidden, float* output,
                      size_t rows, const int32_t* positions,
                      const int32_t* cache_rows, size_t rows_per_sequence,
                      size_t keys_per_sequence, size_t past, int causal,
                      float* k_cache, float* v_cache, size_t capacity);

/* ---- AudioVAE V2's causal decoder (float32, time-major [t][c]) ---------- */

typedef struct vo_vae_unit {   /* a residual unit of `c` channels */
  const float* alpha_in;       /* [c] */
  const float* depthwise;      /* [c][7] */
  const float* depthwise_bias; /* [c] */
  const float* alpha_out;      /* [c] */
  const float* pointwise;      /* [c][c] (out, in) */
  const float* pointwise_bias; /* [c] */
} vo_vae_unit;

typedef struct vo_vae_block {  /* in -> out = in / 2 channels, x stride */
  size_t stride;
  const float* scale;          /* [in]: the rate bucket's conditioning */
  const float* bias;           /* [in] */
  const float* alpha;          /* [in] */
  const float* up;             /* ConvTranspose1d [in][out][2 stride] */
  const float* up_bias;        /* [out] */
  vo_vae_unit units[3];        /* dilations 1, 3, 9 */
} vo_vae_block;

typedef struct vo_vae {
  size_t latent, decoder_dim, block_count;
  const float* in_depthwise;      /* [latent][7] */
  const float* in_depthwise_bias; /* [latent] */
  const float* in_pointwise;      /* [decoder_dim][latent] */
  const float* in_pointwise_bias; /* [decoder_dim] */
  const vo_vae_block* blocks;
  const float* out_alpha;         /* [c] of the last block */
  const float* out_conv;          /* [c][7] */
  float out_bias;
} vo_vae;

/* The decoder over whole sequences from zero history (vae.cpp:415-481 for
 * one chunk; weight normalization already folded): latents
 * [frames][latent] -> samples [frames * prod(strides)]. */
void vo_vae_decode(const vo_vae* vae, const float* latents, size_t frames,
                   float* samples);

#ifdef __cplusplus
}
#endif

#endif /* VOXCPM_ORACLE_H_ */
