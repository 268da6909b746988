/*
 * voxcpm_amd -- the C ABI of an MI355X-native (gfx950, CDNA4, wave64)
 * implementation of VoxCPM2's per-patch DiT hot path: Q8_0-weight x
 * bfloat16-activation products and the local diffusion transformer they
 * drive through the Euler/CFG sampler.
 *
 * Conventions (all entry points):
 *  - Every data pointer is a device pointer unless documented otherwise;
 *    `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *    Work is enqueued on `stream` and nothing synchronizes internally
 *    unless documented.
 *  - The caller owns activations, outputs and weights, as the reference's
 *    callers do (device.hpp:33-77); handles own only their scratch.
 *  - No exception crosses the ABI. Each call returns a vx_status:
 *    VX_UNSUPPORTED corresponds to the reference launchers returning false
 *    ("nothing launched", kernels/wmma_products.hpp:87-89), VX_BAD_ARG to
 *    the reference's std::invalid_argument/WeightError paths, VX_HIP_ERROR
 *    to its GpuError (device.hpp:16-30). vx_last_error() returns the message
 *    of the calling thread's last failure.
 *  - bf16 values are raw bfloat16 bits (uint16_t), as in the reference
 *    (kernels/wmma_products.hpp:26-27).
 */
#ifndef VOXCPM_AMD_H_
#define VOXCPM_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum vx_status {
  VX_OK = 0,
  VX_UNSUPPORTED = 1,
  VX_BAD_ARG = 2,
  VX_HIP_ERROR = 3,
} vx_status;

/* The calling thread's last failure message ("" after success). */
const char* vx_last_error(void);
/* The hipError_t of the calling thread's last VX_HIP_ERROR (0 if none). */
int vx_last_hip_error(void);
/* Library version string. */
const char* vx_version(void);

/* ------------------------------------------------------------------------
 * Q8_0 weights in the gfx950 panel layout.
 *
 * GGML Q8_0 stores a [n][k] matrix as blocks of 34 bytes (float16 scale,
 * then 32 int8 values) along k. The panel layout keeps every value and
 * scale exactly and orders them for 64-lane MFMA operands: 16 weight rows
 * x 64 columns (two blocks) per 1088-byte unit, 16 bytes per lane, then the
 * 16 rows' pairs of float16 scales; units run along k, then down the rows.
 * Rows are padded to 16 and columns to 64 with zero values and scales.
 * ---------------------------------------------------------------------- */

/* Bytes of a packed [n][k] matrix (k a multiple of 32).
 * Replaces kernels::Q8TilesBytes (kernels/wmma_products.hpp:34-38). */
size_t vx_q8_packed_bytes(size_t n, size_t k);

/* GGML Q8_0 blocks [n][k/32] (34 bytes each) -> panels.
 * Replaces kernels::Q8_0ToTiles (kernels/wmma_products.hpp:45-49). */
int vx_q8_pack(const uint8_t* blocks, size_t n, size_t k, void* packed,
               void* stream);

/* Panels -> GGML Q8_0 blocks, the exact inverse of vx_q8_pack. No
 * reference counterpart: it lets the packed form be checked and exported. */
int vx_q8_unpack_blocks(const void* packed, size_t n, size_t k,
                        uint8_t* blocks, void* stream);

/* Panels -> bfloat16 [n][k]: bf16_rne(f32(f16 scale) * q), the conversion
 * the reference applies before products of more than 128 rows.
 * Replaces kernels::Q8TilesToBf16 (kernels/wmma_products.hpp:55-58). */
int vx_q8_unpack_bf16(const void* packed, size_t n, size_t k, uint16_t* out,
                      void* stream);

/* ------------------------------------------------------------------------
 * Products y[m][n] (+)= x[m][k] . W[n][k]^T, x bf16 row-major, W panels,
 * y float32 row-major.
 *
 * m <= 128 (the reference's kChunkedRows, gemm.cpp:48-49) keeps the Q8_0
 * arithmetic exact: int8 -> bf16 exactly, a float32 sum per 32-column
 * block, acc = fmaf(f16 scale, sum, acc), partial sums added in a fixed
 * order (deterministic run to run). m > 128 follows the reference's
 * expansion (gemm.cpp:305-312): W as bf16(scale * q), one float32 sum over
 * k on the matrix cores.
 * ---------------------------------------------------------------------- */

/* Split-reduction scratch of the products: partial sums and counters that
 * are zero between products (the products leave them so), like
 * Bf16Gemm::State's partials/counters (gemm.cpp:95-98). One scratch serves
 * one stream at a time. vx_scratch_create(max_m, max_n) (max_m <= 128)
 * holds 16 max_m max_n floats of partial sums: the splits of products up
 * to max_m x max_n. Products of more than 128 rows split k only on grids
 * of few tiles and use at most VX_PREFILL_SPLIT_FLOATS floats (the split
 * is skipped when the scratch holds fewer than it needs): a scratch of
 * 16 max_m max_n >= VX_PREFILL_SPLIT_FLOATS serves all of them, e.g.
 * vx_scratch_create(128, 1536). */
#define VX_PREFILL_SPLIT_FLOATS (3u << 20)
typedef struct vx_scratch vx_scratch;
int vx_scratch_create(vx_scratch** scratch, size_t max_m, size_t max_n);
void vx_scratch_destroy(vx_scratch* scratch);

/* Replaces kernels::WmmaQ8 and Bf16Gemm::Linear on Q8_0 weights
 * (kernels/wmma_products.hpp:87-93; gemm.hpp:56-58). `scratch` may be NULL,
 * in which case no split reduction across workgroups is used. */
int vx_q8_linear(const uint16_t* x, const void* packed, float* y, size_t m,
                 size_t k, size_t n, int accumulate, vx_scratch* scratch,
                 void* stream);

/* The same product with a bf16 (round to nearest even) output instead of
 * float32 and no accumulation. No reference counterpart (the reference's
 * products write float32); it is the bf16 epilogue of a standalone product. */
int vx_q8_linear_bf16(const uint16_t* x, const void* packed, uint16_t* y,
                      size_t m, size_t k, size_t n, vx_scratch* scratch,
                      void* stream);

/* vx_q8_linear for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): no
 * counterpart in the reference. It allocates nothing and takes no
 * vx_scratch: the k-split partial sums of products of more than 128 rows
 * live in a static device array of VX_PREFILL_SPLIT_FLOATS floats (12 MiB)
 * per GPU, held until the process ends; the product plans never split
 * into more than that. Same arguments as vx_q8_linear; its results are bit
 * for bit vx_q8_linear's with a scratch of at least VX_PREFILL_SPLIT_FLOATS
 * partial-sum floats (vx_scratch_create(128, 1536) or larger), with which
 * both take the same split; a smaller scratch may split k less and round
 * differently. Its first call on a GPU looks up the array's address there
 * (hipGetSymbolAddress), which may happen under stream capture. Every call
 * on one GPU shares that GPU's array, so calls that overlap on one GPU (two
 * streams at once) race. */
int vx_q8_linear_noalloc(const uint16_t* x, const void* packed, float* y,
                         size_t m, size_t k, size_t n, int accumulate,
                         void* stream);

/* ------------------------------------------------------------------------
 * bfloat16 weights (the HF checkpoint's format): the same products on bf16
 * W, as panels (16 rows x 64 columns per 2048-byte unit, the two 32-column
 * blocks' MFMA operands one after the other, zero past n and k) or as rows
 * [n][k]. Each 32-column block's products are summed into the float32
 * accumulators on the matrix cores in k order, as the reference's bf16
 * products do (kernels/wmma_products.hip:210-213); there is no per-block
 * scale.
 * ---------------------------------------------------------------------- */

/* Bytes of a packed bf16 [n][k] matrix (k a multiple of 32).
 * Replaces kernels::Bf16TilesBytes (kernels/wmma_products.hpp:39-43). */
size_t vx_bf16_packed_bytes(size_t n, size_t k);

/* bf16 rows [n][k] -> panels (a byte shuffle).
 * Replaces kernels::Bf16ToTiles (kernels/wmma_products.hpp:51-53). */
int vx_bf16_pack(const uint16_t* rows, size_t n, size_t k, void* packed,
                 void* stream);

/* Panels -> bf16 rows [n][k], the exact inverse of vx_bf16_pack.
 * Replaces kernels::Bf16TilesToRows (kernels/wmma_products.hpp:60-62). */
int vx_bf16_unpack(const void* packed, size_t n, size_t k, uint16_t* rows,
                   void* stream);

/* y[m][n] (+)= x[m][k] . W[n][k]^T on bf16 panels, any m (k a multiple of
 * 32). Replaces kernels::WmmaBf16 and Bf16Gemm::Linear on kBf16Tiles
 * weights (kernels/wmma_products.hpp:95-99; gemm.cpp:259-303, where more
 * than 128 rows unpack the tiles for hipBLASLt: here the same tiled
 * kernel as the Q8_0 products takes them). */
int vx_bf16_linear(const uint16_t* x, const void* packed, float* y, size_t m,
                   size_t k, size_t n, int accumulate, vx_scratch* scratch,
                   void* stream);

/* The same on bf16 rows [n][k] as they come, m <= 32, k a multiple of 8
 * (VX_UNSUPPORTED beyond 32 rows, where the reference hands the product to
 * hipBLASLt). Replaces kernels::SkinnyGemm and Bf16Gemm::LinearRows
 * (kernels/skinny_gemm.hpp:17-24; gemm.cpp:315-330). */
int vx_bf16_linear_rows(const uint16_t* x, const uint16_t* w, float* y,
                        size_t m, size_t k, size_t n, int accumulate,
                        void* stream);

/* ------------------------------------------------------------------------
 * Generator kernels: one entry per reference launcher on the path
 * (kernels/generator_kernels.hpp), same argument meaning, any head_dim that
 * is a multiple of 2 up to 256.
 * ---------------------------------------------------------------------- */

/* kernels::RmsNorm (generator_kernels.hpp:32-36). */
int vx_rms_norm(const float* input, const uint16_t* weight, uint16_t* output,
                float* output_f32, size_t rows, size_t width, float epsilon,
                void* stream);
/* kernels::QkvRope (generator_kernels.hpp:38-47); cos_sin may be NULL. */
int vx_qkv_rope(const float* qkv, const float* cos_sin,
                const int32_t* positions, const int32_t* cache_rows, float* q,
                float* k_cache, float* v_cache, size_t rows, size_t heads,
                size_t kv_heads, size_t head_dim, size_t capacity,
                void* stream);
/* kernels::Attention (generator_kernels.hpp:49-58). */
int vx_attention(const float* q, const float* k_cache, const float* v_cache,
                 uint16_t* output, size_t rows, size_t rows_per_sequence,
                 size_t keys_per_sequence, size_t past, int causal,
                 size_t heads, size_t kv_heads, size_t head_dim,
                 size_t capacity, void* stream);
/* kernels::SwiGlu (generator_kernels.hpp:60-62). */
int vx_swiglu(const float* gate_up, uint16_t* output, size_t rows,
              size_t width, void* stream);
/* kernels::AddBias (generator_kernels.hpp:64-66). */
int vx_add_bias(float* data, const uint16_t* bias, size_t rows, size_t width,
                void* stream);
/* kernels::ToBf16 (generator_kernels.hpp:68-70). */
int vx_to_bf16(const float* input, uint16_t* output, size_t count, int silu,
               void* stream);
/* kernels::GatherRows (generator_kernels.hpp:28-30). */
int vx_gather_rows(const float* input, const int32_t* indices, float* output,
                   size_t rows, size_t width, void* stream);
/* kernels::AssembleDit (generator_kernels.hpp:94-99). */
int vx_assemble_dit(const float* mu, const float* time, const float* cond,
                    const float* x, float* output, size_t patch_size,
                    size_t width, void* stream);
/* kernels::GuidedEuler (generator_kernels.hpp:101-106). zero_star = 1 is the
 * reference's CFG-Zero* scale s = <c,u>/(|u|^2 + 1e-8); zero_star = 0 takes
 * s = 1 (plain CFG: x -= dt (u + cfg (c - u))). */
int vx_guided_euler(const float* velocity, float* x, size_t count, float cfg,
                    float dt, int zero_star, void* stream);

/* ------------------------------------------------------------------------
 * The local DiT and its sampler (generator.cpp:297-324, 424-463, 515-538;
 * transformer.cpp:55-100).
 * ---------------------------------------------------------------------- */

typedef struct vx_dit_shape {
  uint32_t hidden;    /* 1024 */
  uint32_t heads;     /* query heads */
  uint32_t kv_heads;  /* heads % kv_heads == 0 */
  uint32_t head_dim;  /* even, <= 256 */
  uint32_t ffn;       /* intermediate size */
  uint32_t layers;
  uint32_t patch;     /* latent frames per patch (4) */
  uint32_t feat;      /* latent channels (64) */
  uint32_t time_in;   /* width of the sinusoidal time embedding */
  uint32_t has_delta; /* add delta_time_mlp(sinusoid(0)) to the time vector */
  float eps;          /* RMSNorm epsilon */
} vx_dit_shape;

typedef struct vx_dit_projection {
  const void* weight;   /* panels [out][in] (Q8_0 or bf16, `format`) */
  const uint16_t* bias; /* bf16 [out], or NULL */
} vx_dit_projection;

typedef struct vx_dit_layer {
  const uint16_t* input_norm; /* bf16 [hidden] */
  const void* qkv;            /* panels [(heads + 2 kv_heads) head_dim][hidden]:
                                 q rows, then k rows, then v rows */
  const void* o;              /* panels [hidden][heads head_dim] */
  const uint16_t* post_norm;  /* bf16 [hidden] */
  const void* gate_up;        /* panels [2 ffn][hidden]: gate rows, up rows */
  const void* down;           /* panels [hidden][ffn] */
} vx_dit_layer;

/* The format of every matrix of a DiT (vx_dit_weights.format): Q8_0
 * panels (vx_q8_pack) or bf16 panels (vx_bf16_pack), as the reference's
 * StackWeights hold kQ8Tiles or kBf16Tiles (weights.cpp:281-292). */
typedef enum vx_weight_format {
  VX_WEIGHTS_Q8_0 = 0,
  VX_WEIGHTS_BF16 = 1
} vx_weight_format;

typedef struct vx_dit_weights {
  const vx_dit_layer* layers; /* host array of `layers` entries */
  const uint16_t* norm;       /* final norm, bf16 [hidden] */
  const float* rope;          /* [>= 3 + 2 patch][head_dim] cos|sin table, or
                                 NULL for no rotation */
  vx_dit_projection in_proj;  /* feat -> hidden */
  vx_dit_projection cond_proj;
  vx_dit_projection out_proj; /* hidden -> feat */
  vx_dit_projection time_1;   /* time_in -> hidden */
  vx_dit_projection time_2;   /* hidden -> hidden */
  vx_dit_projection delta_1;  /* time_in -> hidden (has_delta) */
  vx_dit_projection delta_2;  /* hidden -> hidden (has_delta) */
  uint32_t format;            /* vx_weight_format of every matrix above (0:
                                 Q8_0 panels; the persistent path takes
                                 Q8_0 only) */
} vx_dit_weights;

typedef struct vx_dit vx_dit;

/* Creates a DiT over caller-owned device weights (the handle keeps the
 * pointers, not copies). Allocates the handle's scratch. */
int vx_dit_create(vx_dit** dit, const vx_dit_shape* shape,
                  const vx_dit_weights* weights);
void vx_dit_destroy(vx_dit* dit);

/* time_mlp(sinusoid(t)) (+ delta_time_mlp(sinusoid(0))) -> [hidden]
 * (generator.cpp:212-237). */
int vx_dit_time_vector(vx_dit* dit, float t, float* vector, void* stream);
/* cond_proj(bf16(cond_latent [patch][feat])) -> [patch][hidden]
 * (generator.cpp:448-451). */
int vx_dit_cond_rows(vx_dit* dit, const float* cond_latent, float* cond_rows,
                     void* stream);
/* One CFG-pair evaluation (EvaluateDit, generator.cpp:297-324):
 * mu [2 hidden], cond_rows [patch][hidden], x [patch][feat],
 * time_vector [hidden] -> velocity [2][patch][feat] (conditional first). */
int vx_dit_eval(vx_dit* dit, const float* mu, const float* cond_rows,
                const float* x, const float* time_vector, float* velocity,
                void* stream);
/* Generator::Velocity (generator.cpp:515-538) on device data. */
int vx_dit_velocity(vx_dit* dit, const float* mu, const float* cond_latent,
                    const float* x, float t, float* velocity, void* stream);
/* The sampler of Generator::Step (generator.cpp:448-463): x [patch][feat]
 * is updated in place over `steps` Euler steps; t, dt, evaluate are HOST
 * arrays (EulerStep, generator.hpp:38-44). The whole patch after its first
 * call with the same arguments replays as one HIP graph. */
int vx_dit_patch(vx_dit* dit, const float* mu, const float* cond_latent,
                 float* x, const float* t, const float* dt,
                 const int32_t* evaluate, size_t steps, float cfg,
                 int zero_star, void* stream);

/* Synchronizes with the device and reports whether every evaluation so far
 * completed: VX_HIP_ERROR when a persistent evaluation gave up waiting at
 * a grid barrier (its results are invalid; the handle is reset for later
 * calls). No reference counterpart: the reference's launches cannot wait
 * on each other, and its GpuError (device.hpp:16-30) covers launch errors,
 * which every entry point here still returns. */
int vx_dit_status(vx_dit* dit);

/* EulerSchedule (generator.cpp:63-80, generator.hpp:34-44) on the host:
 * writes `timesteps` entries. skip = 1 marks CFG-Zero*'s zero-velocity
 * first steps as not evaluated; sway = 0 gives the uniform schedule. */
int vx_euler_schedule(size_t timesteps, float sway, int skip, float* t,
                      float* dt, int32_t* evaluate);

/* ---- one MiniCPM4 stack with a key/value cache --------------------------
 *
 * ForwardStack (transformer.cpp:55-100) as one call: VoxCPM2's base LM and
 * residual LM (one row per decode step, generator.cpp:482-510) and the
 * local encoder (patch + 1 rows per patch, generator.cpp:252-295). */

typedef struct vx_stack_shape {
  size_t hidden;   /* TransformerConfig (config.hpp:15-31) */
  size_t heads;
  size_t kv_heads;
  size_t head_dim;
  size_t ffn;      /* intermediate */
  size_t layers;
  float eps;
  int rope;        /* 1: rotary embedding from vx_stack_weights.rope;
                      0: none (the residual LM, config.rope = false) */
} vx_stack_shape;

typedef struct vx_stack_weights {
  const vx_dit_layer* layers; /* host array of `layers` entries
                                 (StackWeights, weights.hpp:28-41) */
  const uint16_t* norm;       /* final norm, bf16 [hidden] */
  const float* rope;          /* device table [positions][head_dim]
                                 (vx_rope_table), or NULL without rope */
  uint32_t format;            /* vx_weight_format of every matrix */
} vx_stack_weights;

typedef struct vx_stack vx_stack;

/* Creates a stack over caller-owned device weights (the handle keeps the
 * pointers); scratch grows with the rows and cache lengths it is given. */
int vx_stack_create(vx_stack** stack, const vx_stack_shape* shape,
                    const vx_stack_weights* weights);
void vx_stack_destroy(vx_stack* stack);

/* ForwardStack (transformer.cpp:55-100, transformer.hpp:69-72): `rows`
 * rows of the float32 residual stream hidden [rows][hidden] (updated in
 * place) through every layer; the final norm's float32 output to
 * output [rows][hidden]. The cache is the reference's KvCache
 * (transformer.hpp:18-36): k_cache and v_cache [layers][kv_heads]
 * [capacity][head_dim] float32, caller-owned; each layer writes its rows'
 * keys and values at cache_rows [rows] (device) and rotates them at
 * positions [rows] (device), then row r of sequence r / rows_per_sequence
 * attends to keys s keys_per_sequence + 0 .. past + (causal ? r % rows_per_
 * sequence + 1 : rows_per_sequence) - 1 (AttentionLayout,
 * transformer.hpp:41-48). VX_BAD_ARG when rows is not a multiple of
 * rows_per_sequence or the attended keys pass the capacity; positions and
 * cache_rows must index the rotary table and the cache. */
int vx_stack_forward(vx_stack* stack, float* hidden, float* output,
                     size_t rows, const int32_t* positions,
                     const int32_t* cache_rows, size_t rows_per_sequence,
                     size_t keys_per_sequence, size_t past, int causal,
                     float* k_cache, float* v_cache, size_t capacity,
                     void* stream);

/* ---- GGUF ingest -----------------------------------------------------------
 *
 * The audio.cpp VoxCPM2 GGUF the reference opens in ModelFiles::Open
 * (model_files.cpp:111-184, model_files.hpp:34-45): a read-only map of the
 * file, the generator's tensors (VX_GGUF_MODEL, names without "weights/")
 * and AudioVAE's (VX_GGUF_VAE, without "audiovae_weights/"), abbreviated
 * names resolved through audiocpp.tensor_names, shapes outermost first
 * (PyTorch's order), config.json and tokenizer.json from the embedded
 * files. A Q8_0 matrix goes to the panel layout in one call, as the
 * reference's Uploader writes kQ8Tiles (weights.cpp:160-186). */

#define VX_GGUF_MODEL 0
#define VX_GGUF_VAE 1

typedef struct vx_gguf vx_gguf;

/* voxcpm2_layout = 1: the audio.cpp VoxCPM2 layout (VX_BAD_ARG when the
 * file is not one); 0: any GGUF of version 2 or 3, every tensor under
 * VX_GGUF_MODEL with the file's own names. VX_BAD_ARG for a malformed file
 * (vx_gguf_last_error says why). */
int vx_gguf_open(const char* path, int voxcpm2_layout, vx_gguf** gguf);
void vx_gguf_close(vx_gguf* gguf);
/* The message of the last failed vx_gguf_* call of this thread. */
const char* vx_gguf_last_error(void);
size_t vx_gguf_tensor_count(const vx_gguf* gguf, int component);
/* Tensor `index` of a component: name, GGML type (0 F32, 1 F16, 8 Q8_0,
 * 26 I32, 30 BF16), shape [rank] outermost first (rank <= 8), the mapped
 * bytes and their count. Any output may be NULL. */
int vx_gguf_tensor(const vx_gguf* gguf, int component, size_t index,
                   const char** name, uint32_t* type, size_t* shape,
                   size_t* rank, const void** data, uint64_t* bytes);
int vx_gguf_find(const vx_gguf* gguf, int component, const char* name,
                 size_t* index);
/* "config.json" or "tokenizer.json" of the VoxCPM2 layout (NULL otherwise);
 * the text lives as long as the handle. */
const char* vx_gguf_embedded(const vx_gguf* gguf, const char* file,
                             size_t* bytes);
/* A Q8_0 matrix [out][in] into Q8_0 panels (`packed`: device, at least
 * vx_q8_packed_bytes(out, in) bytes) on `stream`; returns when done. */
int vx_gguf_upload_q8(const vx_gguf* gguf, int component, size_t index,
                      void* packed, size_t packed_bytes, void* stream);

/* ---- AudioVAE V2's decoder ---------------------------------------------------
 *
 * AudioVae's decoding (vae.hpp:25-80, vae.cpp:370-481): float32, time-major
 * [t][c], chunk by chunk with each causal convolution's history kept in the
 * handle (decoding in chunks equals decoding at once). Weights are the
 * checkpoint's tensors with weight normalization folded, in PyTorch's
 * layouts, device float32; the rate conditioning is the bucket of the
 * output rate (AudioVaeConfig::rate_bucket, config.cpp:269-275). */

typedef struct vx_vae_unit {    /* a residual unit of c channels */
  const float* alpha_in;        /* [c] Snake */
  const float* depthwise;       /* [c][7] */
  const float* depthwise_bias;  /* [c] */
  const float* alpha_out;       /* [c] Snake */
  const float* pointwise;       /* [c][c] (out, in) */
  const float* pointwise_bias;  /* [c] */
} vx_vae_unit;

typedef struct vx_vae_block {   /* in -> in / 2 channels, rate x frames */
  const float* scale;           /* [in] the rate bucket's scale_embed row */
  const float* bias;            /* [in] the rate bucket's bias_embed row */
  const float* alpha;           /* [in] Snake */
  const float* up;              /* ConvTranspose1d [in][in / 2][2 rate] */
  const float* up_bias;         /* [in / 2] */
  vx_vae_unit units[3];         /* dilations 1, 3, 9 */
} vx_vae_block;

typedef struct vx_vae_shape {
  size_t latent_dim;            /* AudioVaeConfig (config.hpp:55-72) */
  size_t decoder_dim;
  size_t rate_count;            /* decoder blocks, at most 8 */
  size_t rates[8];
} vx_vae_shape;

typedef struct vx_vae_weights {
  const float* in_depthwise;       /* [latent][7] */
  const float* in_depthwise_bias;  /* [latent] */
  const float* in_pointwise;       /* [decoder_dim][latent] */
  const float* in_pointwise_bias;  /* [decoder_dim] */
  const vx_vae_block* blocks;      /* host array of rate_count entries */
  const float* out_alpha;          /* [c] of the last block */
  const float* out_conv;           /* [c][7] (Conv1d to one channel) */
  float out_bias;
} vx_vae_weights;

typedef struct vx_vae vx_vae;

/* Creates a decoder over caller-owned device weights (the handle keeps the
 * pointers; the transposed convolutions are repacked into its own
 * buffers), its history cleared. */
int vx_vae_create(vx_vae** vae, const vx_vae_shape* shape,
                  const vx_vae_weights* weights);
void vx_vae_destroy(vx_vae* vae);
/* AudioVae::Reset: a new stream (zero history), cleared by a kernel (no
 * memset node when the caller captures it). */
int vx_vae_reset(vx_vae* vae, void* stream);
/* Output samples per latent frame (AudioVaeConfig::decode_hop). */
size_t vx_vae_hop(const vx_vae* vae);
/* AudioVae::Decode / Enqueue on device data: latents [frames][latent]
 * -> samples [frames * hop] at the output rate, continuing the stream.
 * Chunks of up to 16 frames replay as one HIP graph from their second call
 * with the same buffers. A chunk holds at most vx_vae_max_frames(vae)
 * frames (VX_BAD_ARG beyond: decode longer audio in several chunks). */
int vx_vae_decode(vx_vae* vae, const float* latents, size_t frames,
                  float* samples, void* stream);
/* Most latent frames per vx_vae_decode call (65535 x 32 output samples /
 * hop: 1092 frames, 43.7 s at 48 kHz, for VoxCPM2's hop of 1920). */
size_t vx_vae_max_frames(const vx_vae* vae);

/* The rotary table of MiniCPM's LongRoPE on the host, float32 as the
 * reference computes it (transformer.cpp:20-45): [positions][dim], cos in
 * the first half, sin in the second. factors: dim/2 values or NULL. */
int vx_rope_table(double theta, size_t dim, const double* factors,
                  float scaling, size_t positions, float* table);

#ifdef __cplusplus
}
#endif

#endif /* VOXCPM_AMD_H_ */
