// noalloc.hip — sf_gemm_noalloc: sf_gemm for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).
//
// sf_gemm's split plans (the split tail of the 256 x 256 kernel, split-K of
// small fp32 and 16-bit problems) park fp32 partial tiles and per-tile
// arrival counters in a per-device workspace that sf_gemm allocates on
// demand.  This entry point runs exactly the same plans (so its results are
// bit-identical to sf_gemm's) with that workspace taken from `scratch`, a
// file-scope device array of SF_NOALLOC_SCRATCH_BYTES that every GPU the
// library runs on holds until the process ends.  It never calls hipMalloc,
// hipFree or any allocating routine.
//
// The array's name is a host-side stand-in, not a device address: the
// first call on a device (with that device current) looks the array up
// with hipGetSymbolAddress and keeps the address per device; kernels only
// ever receive that address.  Every call on a device shares its array, so
// calls that overlap on one device (on different streams, or from several
// host threads without ordering) race; calls on one stream are ordered by
// the stream.  The counters must start at zero: each split call clears them
// with a fill kernel on its stream first (a kernel, not a memset, so the
// call can be captured into a graph).
#include <mutex>

#include "sf_internal.hpp"

namespace sf {

// Largest workspace any sf_gemm plan needs on a 256-CU device: a split
// plan cuts at most one tile per CU into parts, R * s <= CUs, 256 KB of
// fp32 partial per part (64 MiB), plus one counter per split tile.
static constexpr size_t kNoallocPartBytes = size_t(64) << 20;
static constexpr size_t kNoallocCounterBytes = 4096;
static_assert(SF_NOALLOC_SCRATCH_BYTES == kNoallocPartBytes + kNoallocCounterBytes, "header and library agree");

static __device__ __align__(256) uint8_t scratch[kNoallocPartBytes + kNoallocCounterBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64];  // per device ordinal; nullptr until looked up

// The device address of this device's `scratch`, looked up on first use.
static int scratch_on_current_device(void** out) {
  int dev = 0;
  int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (rc != SF_OK) return rc;
  if (dev < 0 || dev >= 64) return fail(SF_ERR_UNSUPPORTED, "sf_gemm_noalloc: device ordinal %d above 63", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    rc = check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress (sf_gemm_noalloc scratch)");
    if (rc != SF_OK) return rc;
    if (ptr == nullptr) return fail(SF_ERR_HIP, "sf_gemm_noalloc: scratch has no device address");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return SF_OK;
}

}  // namespace sf

using namespace sf;

extern "C" int sf_gemm_noalloc(int transA, int transB, int64_t M, int64_t N, int64_t K, int64_t batch,
                               const void* A, int64_t lda, int64_t strideA, const void* B, int64_t ldb,
                               int64_t strideB, void* C, int64_t ldc, int64_t strideC, sf_dtype ab_dtype,
                               sf_dtype c_dtype, float alpha, const void* bias, sf_epilogue epi, void* stream) {
  GemmPlan plan;
  int rc = gemm_prepare(transA, transB, M, N, K, batch, A, lda, strideA, B, ldb, strideB, C, ldc, strideC,
                        ab_dtype, c_dtype, alpha, bias, epi, nullptr, 0, 0, true, plan);
  if (rc != SF_OK || plan.noop) return rc;
  size_t part_bytes = 0;
  int counters = 0;
  gemm_split_needs(plan, &part_bytes, &counters);
  if (part_bytes > kNoallocPartBytes || (size_t)counters * sizeof(int) > kNoallocCounterBytes)
    return fail(SF_ERR_UNSUPPORTED,
                "sf_gemm_noalloc: this problem's split plan needs %zu bytes of partials and %d counters, above "
                "the fixed scratch of %zu + %zu bytes (use sf_gemm)",
                part_bytes, counters, kNoallocPartBytes, kNoallocCounterBytes);
  void* base = nullptr;
  rc = scratch_on_current_device(&base);
  if (rc != SF_OK) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (part_bytes > 0) {
    plan.p.ws = static_cast<float*>(base);
    plan.p.counters = reinterpret_cast<int*>(static_cast<uint8_t*>(base) + kNoallocPartBytes);
    rc = launch_zero(plan.p.counters, (size_t)counters * sizeof(int), st);
    if (rc != SF_OK) return rc;
  }
  return gemm_launch_plan(plan, batch, ab_dtype, c_dtype, st);
}
