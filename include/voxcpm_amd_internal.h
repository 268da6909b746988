/*
 * voxcpm_amd -- entry points for tests and tuning, beside the drop-in ABI
 * of voxcpm_amd.h. Same conventions (device pointers, vx_status returns).
 */
#ifndef VOXCPM_AMD_INTERNAL_H_
#define VOXCPM_AMD_INTERNAL_H_

#include <stddef.h>
#include <stdint.h>

#include "voxcpm_amd.h"

#ifdef __cplusplus
extern "C" {
#endif

/* vx_q8_linear (m <= 128) with a forced split plan: `row_groups` row groups
 * per workgroup, `waves` waves per workgroup, `splits` workgroups along k
 * (0 = the default choice). The reference's tests force split plans the
 * same way through PlanWmma's target_waves (kernels/wmma_products.hpp:82-85,
 * tests/products_test.cpp:224-238). */
int vx_q8_linear_planned(const uint16_t* x, const void* packed, float* y,
                         size_t m, size_t k, size_t n, int accumulate,
                         vx_scratch* scratch, int row_groups, int waves,
                         int splits, void* stream);

/* vx_q8_linear's engine (the one-pass skinny kernel) with a forced plan,
 * 17..32 rows, y = x W^T: `row_groups` row groups per workgroup (1, 2,
 * 4), `waves` waves per workgroup (4, 8, 16; 16 only up to 2 row groups),
 * `pairs_per_wave` pairs of k per wave per pass (1, 2), `row_blocks`
 * blocks of rows per tile (1..4); VX_UNSUPPORTED otherwise. The plan
 * search behind the default plans, as the reference's PlanWmma is forced
 * through target_waves (kernels/wmma_products.hpp:82-85). */
int vx_q8_linear_engine(const uint16_t* x, const void* packed, float* y,
                        size_t m, size_t k, size_t n, int row_groups,
                        int waves, int pairs_per_wave, int row_blocks,
                        void* stream);

/* The prefill product (more than 128 rows, Q8_0 panels expanded) with a
 * forced plan: tile `shape` 0 (256 x 256, one step prefetched), 1
 * (128 x 256), 2 (128 x 128), 3 (256 x 128), 4 (256 x 256, two steps),
 * 5 (128 x 64), k split over `splits` workgroups (the scratch must hold
 * splits m n floats when splits > 1); shape 6 is the skinny engine in
 * blocks of 64 rows (no split). VX_UNSUPPORTED for other shapes. The plan
 * search behind vx_q8_linear's prefill plans. */
int vx_q8_linear_gemm(const uint16_t* x, const void* packed, float* y,
                      size_t m, size_t k, size_t n, int shape, int splits,
                      vx_scratch* scratch, void* stream);

/* vx_q8_linear_gemm for bf16 panels (vx_bf16_pack's layout). */
int vx_bf16_linear_gemm(const uint16_t* x, const void* packed, float* y,
                        size_t m, size_t k, size_t n, int shape, int splits,
                        vx_scratch* scratch, void* stream);

/* The default plan of an m x k x n product (m <= 128):
 * out7 = {activation tiles, row groups per workgroup, waves per workgroup,
 * workgroup tiles, splits, pairs per split, pairs per wave}. Counterpart of
 * PlanWmma (kernels/wmma_products.hpp:82-85). */
int vx_q8_plan(size_t m, size_t k, size_t n, vx_scratch* scratch,
               int32_t* out7);

/* The plan of an m x k x n product of more than 128 rows (the expanded
 * path) with this scratch: out4 = {kernel (0 the tiled kernel, 1 the
 * 32 x 32 MFMA kernel, 2 the skinny engine in blocks of 64 rows), rows per
 * tile, columns per tile, splits along k}.
 * Counterpart of the plan gemm.cpp:259-313 picks between hipBLASLt and
 * its chunked products. */
int vx_q8_prefill_plan(size_t m, size_t k, size_t n, vx_scratch* scratch, int32_t* out4);

/* float32 [n] -> bf16 bits [n] through the conversion the fused kernels use
 * for their bf16 activations (gfx950's v_cvt_pk_bf16_f32), so that tests can
 * check it bit for bit against the reference's rounding
 * (kernels/device_math.hpp:13-19). n must be even. */
int vx_test_pack_bf16(const float* input, uint16_t* output, size_t n,
                      void* stream);

/* Reads `bytes` (a multiple of 16) at `data` once with coalesced 16-byte
 * loads, one load per thread, and writes nothing unless the data's XOR is
 * `never` (then `sink` [1] receives it). The achievable per-launch ceiling
 * beside the products: the same bytes, launched and rotated the same way,
 * with no arithmetic. Counterpart of ReadProbe
 * (kernels/skinny_gemm.hip:340-358), the reference benchmark's plain-read
 * reference. */
int vx_stream_read(const void* data, size_t bytes, uint32_t never,
                   uint32_t* sink, void* stream);

/* One launch of `workgroups` workgroups of `threads` threads in which every
 * workgroup reads all `bytes` (a multiple of 16) of `in` and the workgroups
 * together write `out` = in + 1 per 32-bit word (workgroup b its b-th
 * share); `sink` [1] receives the XOR of what was read only if it equals
 * `never`. With bytes = 0 it is an empty launch of that grid: the
 * per-launch floor. Launches alternating two buffers form a chain of
 * dependent hand-offs, the pattern of the DiT's kernels, each of which reads
 * the whole activation block the previous one wrote. Timed the way the
 * reference's benchmark times its launches (event-timed repeats,
 * tools/bench/gemm_bench.cpp:50-84). */
int vx_handoff(const void* in, void* out, size_t bytes, int workgroups, int threads,
               uint32_t never, uint32_t* sink, void* stream);

/* The DiT evaluation paths. AUTO (the default) takes FUSED where the shape
 * allows (five launches per layer on fragment-order activations), else
 * UNFUSED (the reference's launch sequence of transformer.cpp:55-100:
 * norm, qkv, rotary, attention, o, norm, gate_up, SwiGLU, down).
 * PERSISTENT (one launch per evaluation, grid barriers between the layer's
 * phases, weights loaded ahead of each barrier) is selected explicitly; it
 * exists only where vx_dit_create found every workgroup of its grid
 * resident at once. Its evaluations cannot report a grid barrier that gave
 * up waiting through their own return value (they return before the
 * device runs them): their results are valid only once vx_dit_status has
 * returned VX_OK. Tests pin every path against the same oracle. */
#define VX_DIT_PATH_AUTO 0
#define VX_DIT_PATH_PERSISTENT 1
#define VX_DIT_PATH_FUSED 2
#define VX_DIT_PATH_UNFUSED 3
/* The fused kernels with each RMSNorm applied before its product's bf16
 * rounding (the reference's order: bf16((x * r) * gamma)); VX_DIT_PATH_FUSED
 * has the residual updates write bf16(x * gamma) and scales the products'
 * outputs by r instead, which is faster and within the same tolerance. */
#define VX_DIT_PATH_FUSED_REFERENCE_ORDER 4

/* Selects the evaluation path of later calls (VX_UNSUPPORTED when the
 * shape has no such path). No reference counterpart: the reference has one
 * path. */
int vx_dit_set_path(vx_dit* dit, int path);
/* The path that runs now (AUTO resolved), or -1 for a null handle. */
int vx_dit_path(const vx_dit* dit);

/* Timestamps of later persistent evaluations into a device buffer of at
 * least vx_dit_trace_bytes() bytes (NULL stops recording): per workgroup
 * and grid barrier, s_memrealtime (100 MHz) at arrival and at exit, and
 * within the phase before it when its activations and its products were
 * done; slot 0 holds the launch's start and end. Counterpart of Generator::set_trace
 * (generator.hpp:58-95), which times the reference's stages. */
int vx_dit_set_trace(vx_dit* dit, void* buffer, size_t bytes);
size_t vx_dit_trace_bytes(const vx_dit* dit);

/* The stack's paths: AUTO takes ROWS up to 8 rows (one-tile products on
 * the row-major residual stream, the norms folded into qkv and gate_up,
 * SwiGLU into gate_up's epilogue, the residual adds into o and down), FUSED
 * up to 32 rows (the DiT's fused layer kernels on fragment-order rows),
 * else UNFUSED (transformer.cpp:55-100's launch sequence); every path
 * shares the rotary/cache kernel and the split attention. A path that
 * cannot take a call's rows runs UNFUSED. */
#define VX_STACK_PATH_AUTO 0
#define VX_STACK_PATH_FUSED 2
#define VX_STACK_PATH_UNFUSED 3
#define VX_STACK_PATH_ROWS 4

/* Selects the path of later vx_stack_forward calls (VX_UNSUPPORTED when the
 * shape has no fused kernels). */
int vx_stack_set_path(vx_stack* stack, int path);
/* The path a call of `rows` rows takes now, or -1 for a null handle. */
int vx_stack_path(const vx_stack* stack, size_t rows);

/* The stack's attention on one layer's cache (the arguments of
 * vx_attention, kernels/generator_kernels.hpp): the keys of each (row, KV
 * head) in chunks of 64 scored by separate workgroups, a second launch
 * merging the chunks' statistics in chunk order when there are several;
 * output bf16 [rows][heads][head_dim]. `partials` holds
 * vx_split_attention_floats(...) floats (NULL when that is 0). */
int vx_split_attention(const float* q, const float* k_cache,
                       const float* v_cache, uint16_t* output, size_t rows,
                       size_t rows_per_sequence, size_t keys_per_sequence,
                       size_t past, int causal, size_t heads, size_t kv_heads,
                       size_t head_dim, size_t capacity, float* partials,
                       size_t partial_floats, void* stream);
size_t vx_split_attention_floats(size_t rows, size_t heads, size_t head_dim,
                                 size_t past, size_t rows_per_sequence);

#ifdef __cplusplus
}
#endif

#endif /* VOXCPM_AMD_INTERNAL_H_ */
