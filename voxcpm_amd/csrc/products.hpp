// Internal interface of the Q8_0 product kernels (q8_products.hip,
// q8_tiled.hip) for the C ABI and the DiT.
#ifndef VOXCPM_AMD_PRODUCTS_HPP_
#define VOXCPM_AMD_PRODUCTS_HPP_

#include <hip/hip_runtime.h>

#include <cstddef>

#include "common.hpp"
#include "q8.hpp"
#include "voxcpm_amd.h"

namespace vx {

/// Rows up to which products keep the exact per-block Q8_0 arithmetic; more
/// rows take the reference's expansion to bf16(scale * q) (gemm.cpp:48-49,
/// 272, 305-312).
constexpr std::size_t kExactRows = 128;

/// How a skinny product is split: `rg` row groups per workgroup, `waves`
/// waves per workgroup splitting its pairs, `splits` workgroups along k.
/// `engine` plans run the one-pass engine (q8_tile.hpp: every wave one pair
/// at a time, the next in flight); the others the split kernel, which can
/// also split k over workgroups.
struct ProductPlan {
  bool engine = false;
  int mt = 1;
  int rg = 1;
  int waves = 4;
  int tiles = 1;
  int splits = 1;
  int pairs_per_split = 0;
  int pairs_per_wave = 0;
  int row_blocks = 1;  // engine plans: activation-row blocks per tile
  int pw = 1;          // engine plans: pairs per wave in flight per pass
};

/// Largest row-group count per workgroup the kernels have for `mt` tiles.
int MaxRowGroups(int mt);
/// Largest wave count per workgroup of the kernel for (`mt`, `rg`).
int MaxWaves(int mt, int rg);

/// The plan of an m x k x n product (m <= 128) on weights of `kind`.
/// Positive `rg`, `waves` and `splits` force those values; the split falls
/// back to 1 when the scratch cannot hold its partials.
ProductPlan PlanSkinny(std::size_t m, std::size_t k, std::size_t n,
                       std::size_t scratch_floats, std::size_t scratch_counters,
                       int rg = 0, int waves = 0, int splits = 0,
                       q8::Weights kind = q8::Weights::kQ8);

/// Launches the product (m <= 128) with `plan`: Q8_0 panels with the exact
/// arithmetic, or bf16 weights (panels, or rows [n][k] for m <= 32) on the
/// engine plans.
int RunSkinny(const Bf16* x, const void* w, float* y, Bf16* y_bf16,
              std::size_t m, std::size_t k, std::size_t n, bool accumulate,
              const ProductPlan& plan, float* partials, unsigned* counters,
              hipStream_t stream, q8::Weights kind = q8::Weights::kQ8);

/// Whether an m > 128 product runs on the skinny engine in blocks of 64
/// rows (RunRowBlocks) rather than the tiled or the 32 x 32 MFMA kernel:
/// the smaller prefill products, where those kernels' grids are few tiles
/// (`q8`: Q8_0 panels, else bf16 panels).
bool UseRowBlocks(std::size_t m, std::size_t k, std::size_t n, bool q8);

/// More than 128 rows on the skinny engine in blocks of 64 rows, each
/// staged per wave: Q8_0 panels with the reference's expanded arithmetic
/// (bf16(scale * q) per weight, one float32 sum over k; gemm.cpp:305-312),
/// or bf16 panels. No scratch.
int RunRowBlocks(const Bf16* x, const void* w, float* y, Bf16* y_bf16, std::size_t m,
                 std::size_t k, std::size_t n, bool accumulate, bool bf16, hipStream_t stream);

/// The engine on 17..32 row-major rows with a forced plan (tuning and
/// tests): `rg` row groups per workgroup (1, 2, 4), `waves` waves (4, 8,
/// 16), `pw` pairs per wave per pass (1, 2), `row_blocks` (1..4).
int RunEngineTuned(const Bf16* x, const void* w, float* y, std::size_t m, std::size_t k,
                   std::size_t n, int rg, int waves, int pw, int row_blocks,
                   hipStream_t stream);

/// Most floats of split partial sums any default plan uses (12 MiB): the
/// products' k splits stay within it, so that a static scratch of this size
/// serves every product (vx_q8_linear_noalloc).
constexpr std::size_t kMaxSplitFloats = VX_PREFILL_SPLIT_FLOATS;

/// Whether an m > 128 product takes the 32 x 32 MFMA kernel (q8_gemm.hip)
/// rather than the tiled kernel (q8_tiled.hip), which measured faster on the
/// smaller, latency-bound prefill shapes.
bool UseGemm(std::size_t m, std::size_t n);

/// The prefill product's launch shape (q8_gemm.hip): `shape` 0 (256 x 256
/// tiles), 1 (128 x 256) or 2 (128 x 128), `tiles` workgroup tiles,
/// `splits` workgroups along k (their partial sums need splits m n floats
/// of scratch when splits > 1).
struct GemmPlan {
  int shape = 2;
  int bm = 128;
  int bn = 128;
  int tiles = 1;
  int splits = 1;
};

/// The prefill plan of an m x k x n product whose scratch holds
/// `partial_floats` floats of partial sums.
/// A non-negative `shape` (0..5) forces that tile shape with `splits` splits.
GemmPlan PlanGemm(std::size_t m, std::size_t k, std::size_t n, std::size_t partial_floats,
                  int shape = -1, int splits = 1);

/// The prefill product (m > 128) on the 32 x 32 x 16 matrix cores: Q8_0
/// panels expanded to bf16(scale * q) (gemm.cpp:305-312) or bf16 panels,
/// float32 sums over k; y (+)= x W^T, or its bf16 rounding into y_bf16.
int RunGemm(const Bf16* x, const void* w, float* y, Bf16* y_bf16, std::size_t m, std::size_t k,
            std::size_t n, bool accumulate, bool bf16_weights, float* partials,
            std::size_t partial_floats, hipStream_t stream, int shape = -1, int splits = 1);

/// What the tiled kernel multiplies: Q8_0 panels expanded to bf16(scale * q)
/// (the reference's arithmetic beyond 128 rows) or bf16 panels.
enum class TiledMode : int { kQ8Expanded = 1, kBf16 = 2 };

/// VX_OK, or VX_BAD_ARG (with the message) for product arguments the
/// kernels cannot take: null pointers, m, n or k zero, k not a multiple of
/// 32, shapes past the kernels' 32-bit offsets, x or the weights not 16-byte
/// aligned. `what` names the entry point in the message.
int CheckProduct(const void* x, const void* w, const void* y, std::size_t m, std::size_t k,
                 std::size_t n, const char* what);

/// The tiled product's launch shape: `bm` activation rows per tile,
/// `m_tiles` row tiles, `splits` workgroups along k (their partial sums
/// need splits m n floats of scratch when splits > 1).
struct TiledPlan {
  int bm = 64;
  int m_tiles = 1;
  int splits = 1;
};

/// The tiled plan of an m x k x n product whose scratch holds
/// `partial_floats` floats of partial sums.
TiledPlan PlanTiled(std::size_t m, std::size_t k, std::size_t n, std::size_t partial_floats);

/// Launches the LDS-tiled product (q8_tiled.hip; m > 128). Small
/// grids split k over workgroups when `partials` holds partial_floats >=
/// 2 m n floats (a second launch adds the splits in order).
int RunTiled(const Bf16* x, const void* w, float* y, Bf16* y_bf16, std::size_t m,
             std::size_t k, std::size_t n, bool accumulate, TiledMode mode,
             float* partials, std::size_t partial_floats, hipStream_t stream);

}  // namespace vx

#endif  // VOXCPM_AMD_PRODUCTS_HPP_
