// The C ABI's error state, the product scratch and the product entry points.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "common.hpp"
#include "products.hpp"
#include "q8.hpp"
#include "q8_tile.hpp"

namespace vx {
namespace {

thread_local std::string last_error;
thread_local int last_hip_error = 0;

}  // namespace

int Fail(int status, const std::string& message) {
  last_error = message;
  return status;
}

int FailHip(hipError_t error, const char* what) {
  last_hip_error = static_cast<int>(error);
  last_error = std::string(what) + ": " + hipGetErrorString(error);
  return VX_HIP_ERROR;
}

int Succeed() {
  last_error.clear();
  last_hip_error = 0;
  return VX_OK;
}

int LaunchStatus(const char* what) {
  const hipError_t error = hipGetLastError();
  if (error != hipSuccess)
    return FailHip(error, what);
  return Succeed();
}

}  // namespace vx

struct vx_scratch {
  float* partials = nullptr;
  std::size_t partial_floats = 0;
  unsigned* counters = nullptr;
  std::size_t counter_count = 0;
};

namespace {

__global__ void PackBf16Kernel(const float* input, std::uint32_t* output,
                               std::size_t pairs) {
  const std::size_t i =
      static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < pairs)
    output[i] = vx::q8::PackBf16x2(input[2 * i], input[2 * i + 1]);
}

// One 16-byte load per thread of `chunks` chunks; the XOR of the loaded
// words is stored only when it equals `never`, so the loads stay live and
// nothing is written.
__global__ __launch_bounds__(256) void StreamReadKernel(const uint4* data,
                                                        std::size_t chunks,
                                                        std::uint32_t never,
                                                        std::uint32_t* sink) {
  const std::size_t i = static_cast<std::size_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= chunks)
    return;
  const uint4 v = data[i];
  const std::uint32_t x = v.x ^ v.y ^ v.z ^ v.w;
  if (x == never)
    sink[0] = x;
}

bool Aligned(const void* pointer, std::size_t bytes) {
  return reinterpret_cast<std::uintptr_t>(pointer) % bytes == 0;
}

}  // namespace

namespace vx {

int CheckProduct(const void* x, const void* w, const void* y, std::size_t m,
                 std::size_t k, std::size_t n, const char* what) {
  if (x == nullptr || w == nullptr || y == nullptr)
    return vx::Fail(VX_BAD_ARG, std::string(what) + ": null pointer");
  if (m == 0 || n == 0 || k == 0 || k % 32 != 0)
    return vx::Fail(VX_BAD_ARG, std::string(what) +
                                    ": m, n must be positive and k a positive "
                                    "multiple of 32");
  // Activation offsets are 32-bit byte offsets (x below 1 GiB).
  if (m > (1U << 24) || n > (1U << 24) || k > (1U << 22) ||
      static_cast<unsigned long long>(m) * k > (1ULL << 29))
    return vx::Fail(VX_BAD_ARG, std::string(what) + ": shape too large");
  if (!Aligned(x, 16) || !Aligned(w, 16))
    return vx::Fail(VX_BAD_ARG,
                    std::string(what) + ": x and the panels must be 16-byte "
                                        "aligned");
  return VX_OK;
}

}  // namespace vx

namespace {

using vx::CheckProduct;

int Product(const uint16_t* x, const void* packed, float* y, uint16_t* y_bf16,
            size_t m, size_t k, size_t n, int accumulate, vx_scratch* scratch,
            int rg, int waves, int splits, void* stream,
            vx::q8::Weights kind = vx::q8::Weights::kQ8) {
  if (vx::UseRowBlocks(m, k, n, kind == vx::q8::Weights::kQ8))
    return vx::RunRowBlocks(x, packed, y, y_bf16, m, k, n, accumulate != 0,
                            kind != vx::q8::Weights::kQ8, vx::Stream(stream));
  if (m > vx::kExactRows && vx::UseGemm(m, n))
    return vx::RunGemm(x, packed, y, y_bf16, m, k, n, accumulate != 0,
                       kind != vx::q8::Weights::kQ8,
                       scratch != nullptr ? scratch->partials : nullptr,
                       scratch != nullptr ? scratch->partial_floats : 0, vx::Stream(stream));
  if (m > vx::kExactRows)
    return vx::RunTiled(x, packed, y, y_bf16, m, k, n, accumulate != 0,
                        kind == vx::q8::Weights::kQ8 ? vx::TiledMode::kQ8Expanded
                                                     : vx::TiledMode::kBf16,
                        scratch != nullptr ? scratch->partials : nullptr,
                        scratch != nullptr ? scratch->partial_floats : 0,
                        vx::Stream(stream));
  const vx::ProductPlan plan = vx::PlanSkinny(
      m, k, n, scratch != nullptr ? scratch->partial_floats : 0,
      scratch != nullptr ? scratch->counter_count : 0, rg, waves, splits, kind);
  return vx::RunSkinny(x, packed, y, y_bf16, m, k, n, accumulate != 0, plan,
                       scratch != nullptr ? scratch->partials : nullptr,
                       scratch != nullptr ? scratch->counters : nullptr,
                       vx::Stream(stream), kind);
}

}  // namespace

extern "C" {

const char* vx_last_error(void) { return vx::last_error.c_str(); }

int vx_last_hip_error(void) { return vx::last_hip_error; }

const char* vx_version(void) { return "voxcpm_amd 0.1.0 gfx950"; }

int vx_scratch_create(vx_scratch** scratch, size_t max_m, size_t max_n) {
  if (scratch == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_scratch_create: null handle pointer");
  *scratch = nullptr;
  if (max_m == 0 || max_n == 0 || max_m > vx::kExactRows || max_n > (1U << 24))
    return vx::Fail(VX_BAD_ARG,
                    "vx_scratch_create: max_m must be in 1..128 and max_n "
                    "positive");
  auto* created = new vx_scratch();
  // Up to 16 splits of the largest product; one counter per row group.
  created->partial_floats = 16 * max_m * max_n;
  created->counter_count = vx::q8::Groups(max_n);
  hipError_t error = hipMalloc(reinterpret_cast<void**>(&created->partials),
                               created->partial_floats * sizeof(float));
  if (error == hipSuccess)
    error = hipMalloc(reinterpret_cast<void**>(&created->counters),
                      created->counter_count * sizeof(unsigned));
  if (error == hipSuccess)
    error = hipMemset(created->counters, 0,
                      created->counter_count * sizeof(unsigned));
  if (error != hipSuccess) {
    vx_scratch_destroy(created);
    return vx::FailHip(error, "vx_scratch_create");
  }
  *scratch = created;
  return vx::Succeed();
}

void vx_scratch_destroy(vx_scratch* scratch) {
  if (scratch == nullptr)
    return;
  if (scratch->partials != nullptr)
    (void)hipFree(scratch->partials);
  if (scratch->counters != nullptr)
    (void)hipFree(scratch->counters);
  delete scratch;
}

int vx_q8_linear(const uint16_t* x, const void* packed, float* y, size_t m,
                 size_t k, size_t n, int accumulate, vx_scratch* scratch,
                 void* stream) {
  VX_TRY(CheckProduct(x, packed, y, m, k, n, "vx_q8_linear"));
  return Product(x, packed, y, nullptr, m, k, n, accumulate, scratch, 0, 0, 0,
                 stream);
}

int vx_q8_linear_bf16(const uint16_t* x, const void* packed, uint16_t* y,
                      size_t m, size_t k, size_t n, vx_scratch* scratch,
                      void* stream) {
  VX_TRY(CheckProduct(x, packed, y, m, k, n, "vx_q8_linear_bf16"));
  return Product(x, packed, nullptr, y, m, k, n, 0, scratch, 0, 0, 0, stream);
}

int vx_bf16_linear(const uint16_t* x, const void* packed, float* y, size_t m, size_t k,
                   size_t n, int accumulate, vx_scratch* scratch, void* stream) {
  VX_TRY(CheckProduct(x, packed, y, m, k, n, "vx_bf16_linear"));
  if (vx::q8::Bf16PackedBytes(n, k) > (1ULL << 31) - 16)
    return vx::Fail(VX_BAD_ARG, "vx_bf16_linear: shape too large");
  return Product(x, packed, y, nullptr, m, k, n, accumulate, scratch, 0, 0, 0, stream,
                 vx::q8::Weights::kBf16);
}

int vx_bf16_linear_rows(const uint16_t* x, const uint16_t* w, float* y, size_t m, size_t k,
                        size_t n, int accumulate, void* stream) {
  if (x == nullptr || w == nullptr || y == nullptr)
    return vx::Fail(VX_BAD_ARG, "vx_bf16_linear_rows: null pointer");
  if (m == 0 || n == 0 || k == 0 || k % 8 != 0)
    return vx::Fail(VX_BAD_ARG,
                    "vx_bf16_linear_rows: m, n must be positive and k a positive multiple "
                    "of 8");
  if (m > 32)
    return vx::Fail(VX_UNSUPPORTED, "vx_bf16_linear_rows: at most 32 rows");
  // Byte offsets into x and w are 32-bit.
  if (n > (1U << 24) || k > (1U << 22) || 2ULL * n * k > (1ULL << 31) - 16)
    return vx::Fail(VX_BAD_ARG, "vx_bf16_linear_rows: shape too large");
  if (!Aligned(x, 16) || !Aligned(w, 16))
    return vx::Fail(VX_BAD_ARG, "vx_bf16_linear_rows: x and w must be 16-byte aligned");
  return Product(x, w, y, nullptr, m, k, n, accumulate, nullptr, 0, 0, 0, stream,
                 vx::q8::Weights::kBf16Rows);
}

/* Testing and tuning entry (declared in voxcpm_amd_internal.h): the product
 * with a forced split plan, as PlanWmma's target_waves argument lets the
 * reference's tests force splits (kernels/wmma_products.hpp:82-85). */
int vx_q8_linear_planned(const uint16_t* x, const void* packed, float* y,
                         size_t m, size_t k, size_t n, int accumulate,
                         vx_scratch* scratch, int row_groups, int waves,
                         int splits, void* stream) {
  VX_TRY(CheckProduct(x, packed, y, m, k, n, "vx_q8_linear_planned"));
  if (m > vx::kExactRows)
    return vx::Fail(VX_BAD_ARG,
                    "vx_q8_linear_planned: plans apply to m <= 128");
  return Product(x, packed, y, nullptr, m, k, n, accumulate, scratch,
                 row_groups, waves, splits, stream);
}

/* Testing and tuning entry: the engine with a forced plan (17..32 rows). */
int vx_q8_linear_engine(const uint16_t* x, const void* packed, float* y, size_t m, size_t k,
                        size_t n, int row_groups, int waves, int pairs_per_wave,
                        int row_blocks, void* stream) {
  VX_TRY(CheckProduct(x, packed, y, m, k, n, "vx_q8_linear_engine"));
  return vx::RunEngineTuned(x, packed, y, m, k, n, row_groups, waves, pairs_per_wave,
                            row_blocks, vx::Stream(stream));
}

/* Testing and tuning entry: the prefill product (m > 128) with a forced
 * tile shape and split. */
int vx_q8_linear_gemm(const uint16_t* x, const void* packed, float* y, size_t m, size_t k,
                      size_t n, int shape, int splits, vx_scratch* scratch, void* stream) {
  VX_TRY(CheckProduct(x, packed, y, m, k, n, "vx_q8_linear_gemm"));
  if (m <= vx::kExactRows || shape < 0)
    return vx::Fail(VX_BAD_ARG, "vx_q8_linear_gemm: more than 128 rows and a shape");
  if (shape == 6)  // the skinny engine in blocks of 64 rows
    return vx::RunRowBlocks(x, packed, y, nullptr, m, k, n, false, false, vx::Stream(stream));
  return vx::RunGemm(x, packed, y, nullptr, m, k, n, false, false,
                     scratch != nullptr ? scratch->partials : nullptr,
                     scratch != nullptr ? scratch->partial_floats : 0, vx::Stream(stream),
                     shape, splits);
}

/* Testing and tuning entry: vx_q8_linear_gemm for bf16 panels. */
int vx_bf16_linear_gemm(const uint16_t* x, const void* packed, float* y, size_t m, size_t k,
                        size_t n, int shape, int splits, vx_scratch* scratch, void* stream) {
  VX_TRY(CheckProduct(x, packed, y, m, k, n, "vx_bf16_linear_gemm"));
  if (m <= vx::kExactRows || shape < 0)
    return vx::Fail(VX_BAD_ARG, "vx_bf16_linear_gemm: more than 128 rows and a shape");
  if (shape == 6)
    return vx::RunRowBlocks(x, packed, y, nullptr, m, k, n, false, true, vx::Stream(stream));
  return vx::RunGemm(x, packed, y, nullptr, m, k, n, false, true,
                     scratch != nullptr ? scratch->partials : nullptr,
                     scratch != nullptr ? scratch->partial_floats : 0, vx::Stream(stream),
                     shape, splits);
}

int vx_test_pack_bf16(const float* input, uint16_t* output, size_t n,
                      void* stream) {
  if (input == nullptr || output == nullptr || n % 2 != 0 ||
      !Aligned(output, 4))
    return vx::Fail(VX_BAD_ARG, "vx_test_pack_bf16: bad arguments");
  if (n == 0)
    return vx::Succeed();
  const std::size_t pairs = n / 2;
  PackBf16Kernel<<<static_cast<unsigned>((pairs + 255) / 256), 256, 0,
                   vx::Stream(stream)>>>(
      input, reinterpret_cast<std::uint32_t*>(output), pairs);
  return vx::LaunchStatus("vx_test_pack_bf16");
}

int vx_stream_read(const void* data, size_t bytes, uint32_t never,
                   uint32_t* sink, void* stream) {
  if (data == nullptr || sink == nullptr || bytes % 16 != 0 || !Aligned(data, 16))
    return vx::Fail(VX_BAD_ARG, "vx_stream_read: bad arguments");
  if (bytes == 0)
    return vx::Succeed();
  const std::size_t chunks = bytes / 16;
  StreamReadKernel<<<static_cast<unsigned>((chunks + 255) / 256), 256, 0,
                     vx::Stream(stream)>>>(static_cast<const uint4*>(data), chunks, never,
                                            sink);
  return vx::LaunchStatus("vx_stream_read");
}

/* The plan vx_q8_linear would use: {mt, rg, waves, tiles, splits,
 * pairs_per_split, pairs_per_wave}. */
int vx_q8_plan(size_t m, size_t k, size_t n, vx_scratch* scratch,
               int32_t* out7) {
  if (out7 == nullptr || m == 0 || m > vx::kExactRows || k % 32 != 0 ||
      k == 0 || n == 0)
    return vx::Fail(VX_BAD_ARG, "vx_q8_plan: bad arguments");
  const vx::ProductPlan plan = vx::PlanSkinny(
      m, k, n, scratch != nullptr ? scratch->partial_floats : 0,
      scratch != nullptr ? scratch->counter_count : 0);
  out7[0] = plan.mt;
  out7[1] = plan.rg;
  out7[2] = plan.waves;
  out7[3] = plan.tiles;
  out7[4] = plan.splits;
  out7[5] = plan.pairs_per_split;
  out7[6] = plan.pairs_per_wave;
  return vx::Succeed();
}

int vx_q8_prefill_plan(size_t m, size_t k, size_t n, vx_scratch* scratch, int32_t* out4) {
  if (out4 == nullptr || m <= vx::kExactRows || k % 32 != 0 || k == 0 || n == 0)
    return vx::Fail(VX_BAD_ARG, "vx_q8_prefill_plan: bad arguments");
  const std::size_t floats = scratch != nullptr ? scratch->partial_floats : 0;
  if (vx::UseRowBlocks(m, k, n, true)) {
    out4[0] = 2;
    out4[1] = 64;
    out4[2] = static_cast<int32_t>(16 * (n > 4096 ? 2 : 1));  // columns per workgroup
    out4[3] = 1;
  } else if (vx::UseGemm(m, n)) {
    const vx::GemmPlan plan = vx::PlanGemm(m, k, n, floats);
    out4[0] = 1;
    out4[1] = plan.bm;
    out4[2] = plan.bn;
    out4[3] = plan.splits;
  } else {
    const vx::TiledPlan plan = vx::PlanTiled(m, k, n, floats);
    out4[0] = 0;
    out4[1] = plan.bm;
    out4[2] = 128;  // the tiled kernel's columns per tile
    out4[3] = plan.splits;
  }
  return vx::Succeed();
}

}  // extern "C"
