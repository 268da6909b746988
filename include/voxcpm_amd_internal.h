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

/* The default plan of an m x k x n product (m <= 128):
 * out7 = {activation tiles, row groups per workgroup, waves per workgroup,
 * workgroup tiles, splits, pairs per split, pairs per wave}. Counterpart of
 * PlanWmma (kernels/wmma_products.hpp:82-85). */
int vx_q8_plan(size_t m, size_t k, size_t n, vx_scratch* scratch,
               int32_t* out7);

/* float32 [n] -> bf16 bits [n] through the conversion the fused kernels use
 * for their bf16 activations (gfx950's v_cvt_pk_bf16_f32), so that tests can
 * check it bit for bit against the reference's rounding
 * (kernels/device_math.hpp:13-19). n must be even. */
int vx_test_pack_bf16(const float* input, uint16_t* output, size_t n,
                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VOXCPM_AMD_INTERNAL_H_ */
