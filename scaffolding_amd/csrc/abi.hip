// abi.hip — the extern "C" surface of libsfgemm (include/sfgemm.h):
// argument validation, kernel selection, runtime wrappers and the native
// caching allocator.
//
// Validation runs before any HIP call, so argument errors are reported the
// same way with or without a GPU.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "sf_internal.hpp"

namespace sf {

static thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return SF_OK;
  // The runtime also keeps the error as the thread's last error; it is
  // reported here, so it must not resurface in the next launch check.
  (void)hipGetLastError();
  if (e == hipErrorOutOfMemory) return fail(SF_ERR_OOM, "%s: %s", what, hipGetErrorString(e));
  if (e == hipErrorNoDevice || e == hipErrorInvalidDevice)
    return fail(SF_ERR_NO_DEVICE, "%s: %s", what, hipGetErrorString(e));
  return fail(SF_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int check_launch(const char* what) { return check_hip(hipGetLastError(), what); }

const char* tile_name(int cfg) {
  switch (cfg) {
    case TILE_256x256: return "gemm tile 256x256";
    case TILE_256x128: return "gemm tile 256x128";
    case TILE_128x128: return "gemm tile 128x128";
    case TILE_256x64: return "gemm tile 256x64";
    case TILE_64x64: return "gemm tile 64x64";
    case TILE_GENERIC: return "gemm tile generic";
    case TILE_SKINNY: return "gemm skinny";
    case TILE_NT_BIG: return "gemm nt 256x256 lds-dma";
    case TILE_SKINNY_LINE: return "gemm skinny line";
    case TILE32_SMALL1: return "gemm small 16x16";
    case TILE32_SMALL2: return "gemm small 16x32";
    case TILE32_DMA: return "gemm tile 64x64 lds-dma k-groups";
    case TILE32_DMA_SPLIT: return "gemm tile 64x64 lds-dma";
    case TILE_NT_K64: return "gemm nt 128x128 k64 lds-dma";
  }
  return "gemm";
}

void tile_dims(int cfg, bool fp32, int& bm, int& bn) {
  switch (cfg) {
    case TILE_256x256: bm = 256; bn = 256; return;
    case TILE_NT_BIG: bm = 256; bn = 256; return;
    case TILE_256x128: bm = 256; bn = 128; return;
    case TILE_128x128: bm = 128; bn = 128; return;
    case TILE_NT_K64: bm = 128; bn = 128; return;
    case TILE_256x64: bm = 256; bn = 64; return;
    case TILE_SKINNY: bm = 16; bn = 32; return;
    case TILE_SKINNY_LINE: bm = 16; bn = 64; return;
    case TILE32_SMALL1: bm = 16; bn = 16; return;
    case TILE32_SMALL2: bm = 16; bn = 32; return;
    default: bm = 64; bn = 64; return;
  }
  (void)fp32;
}

int launch_gemm16(sf_dtype in, sf_dtype out, bool a_kmajor, bool b_kmajor, int cfg, const GemmParams& p,
                  int64_t batch, hipStream_t st) {
  unsigned gx;
  if (cfg == TILE_SKINNY)
    gx = static_cast<unsigned>((p.N + 31) / 32);
  else if (p.persist > 0)
    gx = static_cast<unsigned>(p.persist);
  else if (p.split > 0)
    gx = static_cast<unsigned>(p.full_tiles) +
         static_cast<unsigned>(p.tiles_m * p.tiles_n - p.full_tiles) * static_cast<unsigned>(p.split);
  else
    gx = static_cast<unsigned>(p.tiles_m) * static_cast<unsigned>(p.tiles_n);
  for (int64_t b0 = 0; b0 < batch; b0 += 65535) {
    const int64_t nb = (batch - b0) < 65535 ? (batch - b0) : 65535;
    GemmParams q = p;
    q.A = static_cast<const uint16_t*>(p.A) + b0 * p.sA;
    q.B = static_cast<const uint16_t*>(p.B) + b0 * p.sB;
    q.C = static_cast<uint8_t*>(p.C) + b0 * p.sC * (out == SF_F32 ? 4 : 2);
    if (p.res != nullptr) q.res = static_cast<const uint8_t*>(p.res) + b0 * p.sR * (out == SF_F32 ? 4 : 2);
    const int rc = (in == SF_BF16)
                       ? launch_gemm16_bf16(out, a_kmajor, b_kmajor, cfg, q, gx, static_cast<unsigned>(nb), st)
                       : launch_gemm16_f16(out, a_kmajor, b_kmajor, cfg, q, gx, static_cast<unsigned>(nb), st);
    if (rc != SF_OK) return rc;
  }
  return SF_OK;
}

// ---------------------------------------------------------------------
// Device properties cache (CU count drives tile selection).
// ---------------------------------------------------------------------
static std::mutex g_props_mu;
static std::unordered_map<int, int> g_cu_count;

// Without a device (sf_gemm_plan on a host with no GPU) the planner assumes
// 256 CUs, or the count in SF_PLAN_CU_COUNT, so the plans of other parts
// can be checked on the host; a visible device always reports its own.
static int cu_count_current() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    const char* s = getenv("SF_PLAN_CU_COUNT");
    const int v = s != nullptr ? atoi(s) : 0;
    return v > 0 && v <= 4096 ? v : 256;
  }
  std::lock_guard<std::mutex> lk(g_props_mu);
  auto it = g_cu_count.find(dev);
  if (it != g_cu_count.end()) return it->second;
  int cus = 256;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus = 256;
  g_cu_count[dev] = cus;
  return cus;
}

static int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Picks the 16-bit tile config.  Largest tile that still gives every CU at
// least one tile; narrow-N problems (P.V, N <= 64) use the 256x64 tile.  An
// A stored K x M (transA) takes the register-staged tiles only.
static int choose_tile16(int64_t M, int64_t N, int64_t K, int64_t batch, bool vec, bool a_kmajor,
                         bool b_kmajor, bool f32_out, int cus) {
  if (!vec) return TILE_GENERIC;
  if (a_kmajor && b_kmajor && M <= 16)
    return (K == 2048 || K == 4096 || K == 8192) ? TILE_SKINNY_LINE : TILE_SKINNY;
  if (f32_out) return TILE_128x128;
  auto tiles = [&](int64_t bm, int64_t bn) { return cdiv(M, bm) * cdiv(N, bn) * batch; };
  // The 256 x 256 LDS-DMA kernel: K-contiguous operands need K % 128 == 0;
  // two M/N-contiguous operands take any K >= 128.  It runs at least half a
  // wave of 256 x 256 tiles, or fewer for a single GEMM whose tiles the
  // split below cuts along k.
  const bool k_ok = K >= 128 && (K % 128 == 0 || (!a_kmajor && !b_kmajor));
  const int64_t t256 = tiles(256, 256);
  const bool fills = t256 >= cus || (!(a_kmajor && b_kmajor) && M > 64 &&
                                     (2 * t256 >= cus || (batch == 1 && K >= 1024 && 16 * t256 >= cus)));
  // K == 64 exactly (attention scores at head size 64), NT: bound by its
  // stores; the 128 x 128 kernel that holds four workgroups per CU, once
  // the 128 x 128 tiles fill the CUs.
  if (a_kmajor && b_kmajor && K == 64 && N > 64 && tiles(128, 128) >= cus) return TILE_NT_K64;
  if (k_ok && N > 64 && fills) return TILE_NT_BIG;
  if (N <= 64) return tiles(256, 64) >= cus ? TILE_256x64 : TILE_64x64;
  if (tiles(256, 256) >= cus) return TILE_256x256;
  if (tiles(256, 128) >= cus) return TILE_256x128;
  if (tiles(128, 128) >= cus) return TILE_128x128;
  return TILE_64x64;
}

// Picks the fp32 tile config.  Outputs of at most CUs / 4 tiles of 64 x 64
// with K <= 2048 take the small-block kernel (16 x 16 blocks while they
// number at most half the CUs, else 16 x 32); K-contiguous A with K % 32 ==
// 0 takes the LDS-DMA kernel (two k-groups when the slice count is even);
// the rest the register-staged tiles.  Measured: 64 x 512 x 512 NT 4.4 us
// small 16 x 16 against 9.4 us for 64 x 64 tiles in 4 k-parts; 512^3 NN
// 7.9 us small 16 x 32 against 12.5 us k-groups; 768 x 768 x 1024 NN 21.9 us
// k-groups against 28.6 us small and 35 us register-staged in 7 k-parts;
// 1024^3 NN 23.7 us k-groups against 27.1 us one group and 34 us
// register-staged; 4096^3 NN 85% of the fp32 MFMA peak against 77%.
static int choose_tile32(int64_t M, int64_t N, int64_t K, int64_t batch, bool vec, bool a_kmajor, bool dma_ok,
                         int cus) {
  if (!vec) return TILE_GENERIC;
  if (a_kmajor && 4 * cdiv(M, 64) * cdiv(N, 64) * batch <= cus && K <= 2048)
    return 2 * cdiv(M, 16) * cdiv(N, 16) * batch <= cus ? TILE32_SMALL1 : TILE32_SMALL2;
  if (dma_ok) return (K / 32) % 2 == 0 ? TILE32_DMA : TILE32_DMA_SPLIT;
  if (cdiv(M, 128) * cdiv(N, 128) * batch >= cus) return TILE_128x128;
  return TILE_64x64;
}

// ---------------------------------------------------------------------
// Per-device workspace of the split-tail GEMM: fp32 partial tiles and one
// counter per split tile.  Counters start at zero (cleared by a kernel when
// the buffer is created) and every split tile's last part resets its own,
// so the buffer is ready for the next launch.  Launches on one stream are
// ordered by the stream, and while every split launch has come on one
// stream nothing else is done (an event record costs about 3 us of host
// time per call).  The first split launch on a second stream synchronises
// the device once; from then on an event is recorded after every split
// launch and a launch on another stream first waits for it.  Growing the
// buffer synchronises the device before freeing the old one.  The lock is held
// from split_workspace_acquire to split_workspace_release, so calls from
// several host threads enqueue their workspace launches one at a time and
// each one's event wait sees the previous one's record.
// ---------------------------------------------------------------------
struct SplitWorkspace {
  void* base = nullptr;
  size_t part_bytes = 0;
  int counters = 0;
  hipEvent_t done = nullptr;
  hipStream_t last = nullptr;
  bool used = false;
  bool multi = false;  // split launches have come on more than one stream
};
static std::mutex g_ws_mu;
static std::unordered_map<int, SplitWorkspace> g_ws;

static int split_workspace_acquire_locked(int dev, size_t part_bytes, int ncounters, hipStream_t st, float** ws,
                                          int** cnt);

// On SF_OK the workspace lock stays held until split_workspace_release,
// which the caller must then call (after its launch, whatever that
// returned); on failure nothing stays locked.
static int split_workspace_acquire(size_t part_bytes, int ncounters, hipStream_t st, float** ws, int** cnt) {
  int dev = 0;
  int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (rc != SF_OK) return rc;
  g_ws_mu.lock();
  rc = split_workspace_acquire_locked(dev, part_bytes, ncounters, st, ws, cnt);
  if (rc != SF_OK) g_ws_mu.unlock();
  return rc;
}

static int split_workspace_acquire_locked(int dev, size_t part_bytes, int ncounters, hipStream_t st, float** ws,
                                          int** cnt) {
  int rc = SF_OK;
  SplitWorkspace& w = g_ws[dev];
  if (w.done == nullptr) {
    rc = check_hip(hipEventCreateWithFlags(&w.done, hipEventDisableTiming), "hipEventCreate (split workspace)");
    if (rc != SF_OK) return rc;
  }
  if (part_bytes > w.part_bytes || ncounters > w.counters) {
    const size_t pb = part_bytes > w.part_bytes ? part_bytes : w.part_bytes;
    const int nc = ncounters > w.counters ? ncounters : w.counters;
    if (w.base != nullptr) {
      rc = check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize (split workspace)");
      if (rc != SF_OK) return rc;
      (void)hipFree(w.base);
      w.base = nullptr;
      w.part_bytes = 0;
      w.counters = 0;
    }
    void* p = nullptr;
    rc = check_hip(hipMalloc(&p, pb + (size_t)nc * sizeof(int)), "hipMalloc (split workspace)");
    if (rc != SF_OK) return rc;
    rc = launch_zero(static_cast<uint8_t*>(p) + pb, (size_t)nc * sizeof(int), st);
    if (rc != SF_OK) {
      (void)hipFree(p);
      return rc;
    }
    w.base = p;
    w.part_bytes = pb;
    w.counters = nc;
    w.used = false;
  } else if (w.used && w.last != st) {
    if (w.multi) {
      rc = check_hip(hipStreamWaitEvent(st, w.done, 0), "hipStreamWaitEvent (split workspace)");
    } else {
      // No event was recorded after the earlier launches: wait for them
      // once (safe even if their stream has been destroyed since).
      rc = check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize (split workspace, second stream)");
      w.multi = true;
    }
    if (rc != SF_OK) return rc;
  }
  *ws = static_cast<float*>(w.base);
  *cnt = reinterpret_cast<int*>(static_cast<uint8_t*>(w.base) + w.part_bytes);
  return SF_OK;
}

// Records the event after the caller's launch (once split launches have
// come on more than one stream) and releases the lock taken by
// split_workspace_acquire.
static int split_workspace_release(hipStream_t st) {
  std::lock_guard<std::mutex> lk(g_ws_mu, std::adopt_lock);
  int dev = 0;
  int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (rc != SF_OK) return rc;
  SplitWorkspace& w = g_ws[dev];
  w.last = st;
  w.used = true;
  if (!w.multi) return SF_OK;
  return check_hip(hipEventRecord(w.done, st), "hipEventRecord (split workspace)");
}

static bool valid_dtype(int d) { return d == SF_F32 || d == SF_F16 || d == SF_BF16; }
static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

TestHooks g_test_hooks;

}  // namespace sf

using namespace sf;

extern "C" {

const char* sf_status_string(int status) {
  switch (status) {
    case SF_OK: return "success";
    case SF_ERR_HIP: return "HIP runtime error";
    case SF_ERR_INVALID_ARG: return "invalid argument";
    case SF_ERR_UNSUPPORTED: return "unsupported operation";
    case SF_ERR_NO_DEVICE: return "no usable GPU device";
    case SF_ERR_OOM: return "out of device memory";
  }
  return "unknown status";
}

const char* sf_last_error(void) { return g_err; }

int sf_version(void) { return 100; /* 0.1.0 */ }

int sf_set_test_hooks(int xcd_shift, int split_spins, int attn_parts) {
  if (xcd_shift < 0 || xcd_shift >= kNumXcd)
    return fail(SF_ERR_INVALID_ARG, "sf_set_test_hooks: xcd_shift %d outside [0, %d)", xcd_shift, kNumXcd);
  if (split_spins > kSplitArriveSpins)
    return fail(SF_ERR_INVALID_ARG, "sf_set_test_hooks: split_spins %d above %d", split_spins, kSplitArriveSpins);
  if (attn_parts != 0 && (attn_parts < 2 || attn_parts > 16))
    return fail(SF_ERR_INVALID_ARG, "sf_set_test_hooks: attn_parts %d is neither 0 nor in [2, 16]", attn_parts);
  g_test_hooks.xcd_shift.store(xcd_shift, std::memory_order_relaxed);
  g_test_hooks.split_spins.store(split_spins < 0 ? -1 : split_spins, std::memory_order_relaxed);
  g_test_hooks.attn_parts.store(attn_parts, std::memory_order_relaxed);
  return SF_OK;
}

}  // extern "C"

namespace sf {

// Validates sf_gemm's arguments and fills the launch plan (GemmPlan,
// sf_internal.hpp).  Returns SF_OK with plan.noop = true for an empty
// problem.  No HIP call before validation.
int gemm_prepare(int transA, int transB, int64_t M, int64_t N, int64_t K, int64_t batch, const void* A,
                 int64_t lda, int64_t strideA, const void* B, int64_t ldb, int64_t strideB, void* C, int64_t ldc,
                 int64_t strideC, sf_dtype ab_dtype, sf_dtype c_dtype, float alpha, const void* bias,
                 sf_epilogue epi, const void* R, int64_t ldr, int64_t strideR, bool need_c, GemmPlan& plan) {
  g_err[0] = 0;
  plan.noop = false;
  if (!valid_dtype(ab_dtype) || !valid_dtype(c_dtype))
    return fail(SF_ERR_INVALID_ARG, "sf_gemm: unknown dtype (%d, %d)", (int)ab_dtype, (int)c_dtype);
  if ((int)epi < SF_EPI_NONE || (int)epi > SF_EPI_GELU_TANH)
    return fail(SF_ERR_INVALID_ARG, "sf_gemm: unknown epilogue %d", (int)epi);
  if (c_dtype != ab_dtype && c_dtype != SF_F32)
    return fail(SF_ERR_UNSUPPORTED, "sf_gemm: output dtype must equal the input dtype or be F32");
  if (M < 0 || N < 0 || K < 0 || batch < 0)
    return fail(SF_ERR_INVALID_ARG, "sf_gemm: negative size (M=%lld N=%lld K=%lld batch=%lld)",
                (long long)M, (long long)N, (long long)K, (long long)batch);
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return fail(SF_ERR_INVALID_ARG, "sf_gemm: M, N, K must be < 2^31");
  const bool has_bias = epi_has_bias(epi);
  if (has_bias && bias == nullptr)
    return fail(SF_ERR_INVALID_ARG, "sf_gemm: epilogue %d needs a bias pointer", (int)epi);
  if (!has_bias && bias != nullptr)
    return fail(SF_ERR_INVALID_ARG, "sf_gemm: bias given but epilogue %d has no bias", (int)epi);
  if (M == 0 || N == 0 || batch == 0) {
    plan.noop = true;
    return SF_OK;
  }
  // op(A) = A (M x K, K-contiguous) or, with transA, the transpose of A
  // stored K x M; op(B) likewise with transB for B stored N x K.
  const bool a_kmajor = transA == 0;
  const bool b_kmajor = transB != 0;
  if ((need_c && C == nullptr) || (K > 0 && (A == nullptr || B == nullptr)))
    return fail(SF_ERR_INVALID_ARG, "sf_gemm: null operand pointer");
  if (lda < (a_kmajor ? (K > 0 ? K : 1) : M) || ldb < (b_kmajor ? (K > 0 ? K : 1) : N) || ldc < N)
    return fail(SF_ERR_INVALID_ARG,
                "sf_gemm: leading dimension too small (lda=%lld ldb=%lld ldc=%lld for M=%lld "
                "N=%lld K=%lld transA=%d transB=%d)",
                (long long)lda, (long long)ldb, (long long)ldc, (long long)M, (long long)N,
                (long long)K, transA, transB);
  if (strideA < 0 || strideB < 0 || strideC < 0)
    return fail(SF_ERR_INVALID_ARG, "sf_gemm: negative batch stride");
  // Batch entries of C must not overlap: whole matrices apart, or side by
  // side within each row (e.g. attention heads written into [S, heads * D]).
  if (batch > 1 && strideC < (M - 1) * ldc + N && !(strideC >= N && (batch - 1) * strideC + N <= ldc))
    return fail(SF_ERR_INVALID_ARG, "sf_gemm: strideC=%lld overlaps batch entries (need >= %lld, or "
                "side by side within rows of ldc)", (long long)strideC, (long long)((M - 1) * ldc + N));
  if (R != nullptr) {
    if (ldr < N || strideR < 0)
      return fail(SF_ERR_INVALID_ARG, "sf_gemm_add: residual ldr=%lld / strideR=%lld invalid for N=%lld",
                  (long long)ldr, (long long)strideR, (long long)N);
    if (R == C && (ldr != ldc || strideR != strideC))
      return fail(SF_ERR_INVALID_ARG, "sf_gemm_add: an in-place residual (R == C) needs ldr == ldc and "
                  "strideR == strideC");
  }

  GemmParams& p = plan.p;
  p.A = A; p.B = B; p.C = C; p.bias = bias;
  p.lda = lda; p.ldb = ldb; p.ldc = ldc;
  p.sA = strideA; p.sB = strideB; p.sC = strideC;
  p.M = (int)M; p.N = (int)N; p.K = (int)K;
  p.alpha = alpha;
  p.epi = (int)epi;
  p.res = R;
  p.ldr = ldr;
  p.sR = strideR;
  plan.a_kmajor = a_kmajor;
  plan.b_kmajor = b_kmajor;
  const int cus = cu_count_current();
  int bm, bn;
  if (ab_dtype == SF_F32) {
    const bool vec = al16(A) && al16(B) && (lda % 4 == 0) && (ldb % 4 == 0) &&
                     (strideA % 4 == 0) && (strideB % 4 == 0) && (K % 4 == 0) &&
                     (a_kmajor || M % 4 == 0) && (b_kmajor || N % 4 == 0);
    // The LDS-DMA kernel addresses each operand with 32-bit byte offsets.
    const bool dma_ok = a_kmajor && K % 32 == 0 && M * lda * 4 < (int64_t(1) << 31) &&
                        (b_kmajor ? N : K) * ldb * 4 < (int64_t(1) << 31);
    plan.fp32 = true;
    plan.cfg = choose_tile32(M, N, K, batch, vec, a_kmajor, dma_ok, cus);
  } else {
    const bool vec = al16(A) && al16(B) && (lda % 8 == 0) && (ldb % 8 == 0) &&
                     (strideA % 8 == 0) && (strideB % 8 == 0) && (K % 8 == 0) &&
                     (a_kmajor || M % 8 == 0) && (b_kmajor || N % 8 == 0);
    plan.fp32 = false;
    plan.cfg = choose_tile16(M, N, K, batch, vec, a_kmajor, b_kmajor, c_dtype == SF_F32, cus);
    // The LDS-DMA kernel addresses each operand (M or K rows of lda) with
    // 32-bit byte offsets.
    if (plan.cfg == TILE_NT_BIG && ((a_kmajor ? M : K) * lda * 2 >= (int64_t(1) << 31) ||
                                    (b_kmajor ? N : K) * ldb * 2 >= (int64_t(1) << 31)))
      plan.cfg = TILE_256x256;
    if (plan.cfg == TILE_NT_K64 && (M * lda * 2 >= (int64_t(1) << 31) || N * ldb * 2 >= (int64_t(1) << 31)))
      plan.cfg = TILE_128x128;
  }
  // The row-segment skinny kernel addresses 64 rows of W with 32-bit offsets.
  if (plan.cfg == TILE_SKINNY_LINE && ldb * 2 * 64 >= (int64_t(1) << 31)) plan.cfg = TILE_SKINNY;
  tile_dims(plan.cfg, plan.fp32, bm, bn);
  if (cdiv(M, bm) * cdiv(N, bn) > INT32_MAX)
    return fail(SF_ERR_UNSUPPORTED, "sf_gemm: %lld x %lld output needs more than 2^31 tiles",
                (long long)M, (long long)N);
  p.tiles_m = (int)cdiv(M, bm);
  p.tiles_n = (int)cdiv(N, bn);
  p.rows_per = 0;
  p.full_tiles = 0;
  p.split = 0;
  p.ws = nullptr;
  p.counters = nullptr;
  p.persist = 0;
  p.wave4 = 0;
  p.xcd_shift = 0;
  p.arrive_spins = kSplitArriveSpins;
  if (plan.fp32 && batch == 1 && K >= 128 && (plan.cfg == TILE32_DMA || plan.cfg == TILE32_DMA_SPLIT)) {
    // LDS-DMA fp32 with at most CUs / 4 tiles of 64 x 64 (K > 2048, past the
    // small-block kernel): split every tile along k, at most 8 parts of at
    // least 4 slices (64 x 4096 x 4096 NT: 37.9 us in 4 parts against
    // 52 us small 16 x 32 blocks and 72 us unsplit; 200 x 300 x 4096 NN:
    // 21.5 us in 8 parts against 71.6 us unsplit).  With more tiles two
    // k-groups beat two k-parts (768 x 768 x 1024 NN: 21.9 us against 27 us).
    const int64_t t64 = cdiv(M, 64) * cdiv(N, 64), KT = K / 32;
    int64_t sp = cus / (t64 > 0 ? t64 : 1);
    if (sp > kMaxSplit32) sp = kMaxSplit32;
    if (sp > KT / 4) sp = KT / 4;
    if (4 * t64 <= cus && sp >= 2) {
      plan.cfg = TILE32_DMA_SPLIT;
      p.split = (int)sp;
    }
  }
  if (plan.fp32 && batch == 1 && K >= 128 && (plan.cfg == TILE_128x128 || plan.cfg == TILE_64x64)) {
    // fp32 with fewer 64 x 64 tiles than CUs: split every tile along k (each
    // part at least 4 slices of 32), on 128 x 128 tiles when that reaches
    // half the CUs, else on 64 x 64 tiles.  With at least one 64 x 64 tile
    // per CU the unsplit 64 x 64 plan is faster (1024^3: 37.8 us against
    // 44.6 us for 128 x 128 tiles in 4 parts).
    const int64_t KT = cdiv(K, 32);
    auto parts = [&](int64_t t) {
      int64_t sp = cus / (t > 0 ? t : 1);
      if (sp > kMaxSplit32) sp = kMaxSplit32;
      if (sp > KT / 4) sp = KT / 4;
      return sp < 1 ? (int64_t)1 : sp;
    };
    const int64_t t128 = cdiv(M, 128) * cdiv(N, 128), t64 = cdiv(M, 64) * cdiv(N, 64);
    if (t128 < cus && t64 < cus) {
      const int64_t s128 = parts(t128), s64 = parts(t64);
      int cfg = -1;
      int64_t sp = 1;
      if (s128 >= 2 && 2 * t128 * s128 >= cus) {
        cfg = TILE_128x128;
        sp = s128;
      } else if (t64 < cus && s64 >= 2) {
        cfg = TILE_64x64;
        sp = s64;
      }
      if (cfg >= 0) {
        plan.cfg = cfg;
        tile_dims(plan.cfg, plan.fp32, bm, bn);
        p.tiles_m = (int)cdiv(M, bm);
        p.tiles_n = (int)cdiv(N, bn);
        p.full_tiles = 0;
        p.split = (int)sp;
      }
    }
  }
  if (plan.cfg == TILE_NT_BIG && batch == 1 && K >= 128) {
    // Tail split: with R = tiles % CUs left over after whole waves, run the
    // last R tiles as R * s parts of K / s each (s <= CUs / R), so the last
    // wave is full instead of R / CUs full.  With fewer tiles than half the
    // CUs every tile is split (split-K).  Behind whole waves the tail is
    // split for tiles of at least 32 k-units (K >= 4096), and in short
    // persistent launches (below) from 8 units: otherwise the parts' partial
    // sums cost more than a short tail (M = 17776, N = 1920: K = 1920 with
    // one part summing all: 127 us unsplit against 130 us in 5 parts; K =
    // 7680 runs 453 us in 5 parts against 535 us unsplit, both persistent).
    //
    // Persistent tiles (K-contiguous A: NT, or NN as in dX = dY W; more
    // tiles than CUs, CU count a multiple of 8): one workgroup per CU walks
    // its tiles, the next tile's first loads under the current tile's end.
    // Taken when the last round is at most half full or the tail is split;
    // with a fuller last round the hardware's dynamic dispatch balances
    // better (C5 QKV 1610 tiles 311 -> 301 us, MLP-up 2100 tiles 400 -> 387
    // us; C3 M = 4096 688 tiles 261 us one workgroup per tile against 270
    // us persistent).  NN (C5 backward dX, A/B twice): QKV backward 0.763 ->
    // 0.742 ms, out-projection 0.291 -> 0.282 ms, MLP-up and MLP-down
    // within 1 %.
    // Its split tail packs each tile's parts onto one XCD, at most CUs / 8
    // parts per XCD, and shares the final sum among the parts (each sums
    // and stores a slice of the rows).  A short persistent launch (under 3
    // rounds of tiles, where the tail round is a large share) also splits
    // below K = 4096, in parts of at least 5 units (so from K = 1280):
    // measured A/B, C5 out-projection (M = 17776, N = K = 1920, 560 tiles)
    // 128.7 us unsplit against 123.1 us in 3 parts (5 parts: no faster than
    // none); 4352 x 7936 x 1024 (527 tiles) 75.2 us unsplit against 80.5 us
    // in 2 parts of 4 units; at 6-8 rounds (C5 QKV, MLP-up, K = 1920) 2-4
    // parts were no faster than none.
    const int64_t T = (int64_t)p.tiles_m * p.tiles_n, R = T % cus, units = (K + 127) / 128;
    const bool can_persist = a_kmajor && T > cus && cus % kNumXcd == 0;  // NT, or NN (dX)
    const int64_t min_units = T <= R ? 2 : (can_persist && T < 3 * cus ? 10 : 32);
    if (R > 0 && 2 * R <= cus && units >= min_units && (T - R) % kNumXcd == 0) {
      int64_t sp = cus / R;
      if (sp > units) sp = units;
      if (T > R && units < 32 && sp > units / 5) sp = units / 5;
      if (sp > 8) sp = 8;
      if (can_persist) {
        const int64_t per_xcd = (R + kNumXcd - 1) / kNumXcd;  // tail tiles on the busiest XCD
        const int64_t cap = (cus / kNumXcd) / per_xcd;
        if (sp > cap) sp = cap;
      }
      if (sp >= 2) {
        p.full_tiles = (int)(T - R);
        p.split = (int)sp;
        if (can_persist) {
          p.persist = cus;
          // Test hooks (sf_set_test_hooks): a forced XCD mismatch, a capped
          // wait for the other parts.  Results must not change.
          p.xcd_shift = g_test_hooks.xcd_shift.load(std::memory_order_relaxed) & (kNumXcd - 1);
          const int spins = g_test_hooks.split_spins.load(std::memory_order_relaxed);
          if (spins >= 0) p.arrive_spins = spins > kSplitArriveSpins ? kSplitArriveSpins : spins;
        }
      }
    }
    if (p.split == 0 && can_persist && 2 * R <= cus) p.persist = cus;
    // One workgroup per tile, no split parts, deep K, C rows in whole
    // 128-byte lines: the one-wave-per-SIMD kernel.  Measured against the
    // 8-wave kernel on one box: 4096^3 92.4 -> 91.6 us, 4096 x 11008 x
    // 4096 256.9 -> 255.8 us, K = 8192 175.3 -> 173.0 us; at K = 2048 and
    // 1024 within 0.6 % either way, and 2.3 % slower with 4000-wide C rows
    // (its 256-byte row segments straddle more lines).
    if (a_kmajor && b_kmajor && p.split == 0 && p.persist == 0 && K >= 4096 && ldc % 64 == 0) p.wave4 = 1;
  }
  if (plan.cfg == TILE_SKINNY_LINE) {
    // One workgroup per CU where N allows, at most 64 rows of W each.
    int64_t rp = cdiv(N, cus);
    rp = rp < 1 ? 1 : (rp > 64 ? 64 : rp);
    p.rows_per = (int)rp;
    p.tiles_m = 1;
    p.tiles_n = (int)cdiv(N, rp);
  }
  return SF_OK;
}

void gemm_split_needs(const GemmPlan& plan, size_t* part_bytes, int* counters) {
  *part_bytes = 0;
  *counters = 0;
  if (plan.noop || plan.p.split <= 0) return;
  if (plan.fp32) {
    const int tiles = plan.p.tiles_m * plan.p.tiles_n;
    *part_bytes = (size_t)tiles * plan.p.split * (size_t)(plan.cfg == TILE_128x128 ? 16 : 4) * 256u * 16u;
    *counters = tiles;
  } else {
    const int nsplit = plan.p.tiles_m * plan.p.tiles_n - plan.p.full_tiles;
    *part_bytes = (size_t)nsplit * plan.p.split * (256u * 256u * 4u);
    // persistent: three words per split tile (split_handoff_shared)
    *counters = plan.p.persist > 0 ? 3 * nsplit : nsplit;
  }
}

int gemm_launch_plan(const GemmPlan& plan, int64_t batch, sf_dtype ab_dtype, sf_dtype c_dtype, hipStream_t st) {
  if (plan.fp32) return launch_gemm32(plan.a_kmajor, plan.b_kmajor, plan.cfg, plan.p, batch, st);
  return launch_gemm16(ab_dtype, c_dtype, plan.a_kmajor, plan.b_kmajor, plan.cfg, plan.p, batch, st);
}

}  // namespace sf

extern "C" {

static int gemm_run(int transA, int transB, int64_t M, int64_t N, int64_t K, int64_t batch, const void* A,
                    int64_t lda, int64_t strideA, const void* B, int64_t ldb, int64_t strideB, void* C,
                    int64_t ldc, int64_t strideC, sf_dtype ab_dtype, sf_dtype c_dtype, float alpha,
                    const void* bias, sf_epilogue epi, const void* R, int64_t ldr, int64_t strideR,
                    void* stream) {
  GemmPlan plan;
  int rc = gemm_prepare(transA, transB, M, N, K, batch, A, lda, strideA, B, ldb, strideB, C, ldc,
                        strideC, ab_dtype, c_dtype, alpha, bias, epi, R, ldr, strideR, true, plan);
  if (rc != SF_OK || plan.noop) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  size_t part_bytes = 0;
  int counters = 0;
  gemm_split_needs(plan, &part_bytes, &counters);
  if (part_bytes == 0) return gemm_launch_plan(plan, batch, ab_dtype, c_dtype, st);
  rc = split_workspace_acquire(part_bytes, counters, st, &plan.p.ws, &plan.p.counters);
  if (rc != SF_OK) return rc;
  rc = gemm_launch_plan(plan, batch, ab_dtype, c_dtype, st);
  const int rc2 = split_workspace_release(st);
  return rc != SF_OK ? rc : rc2;
}

int sf_gemm(int transA, int transB, int64_t M, int64_t N, int64_t K, int64_t batch, const void* A,
            int64_t lda, int64_t strideA, const void* B, int64_t ldb, int64_t strideB, void* C,
            int64_t ldc, int64_t strideC, sf_dtype ab_dtype, sf_dtype c_dtype, float alpha,
            const void* bias, sf_epilogue epi, void* stream) {
  return gemm_run(transA, transB, M, N, K, batch, A, lda, strideA, B, ldb, strideB, C, ldc, strideC, ab_dtype,
                  c_dtype, alpha, bias, epi, nullptr, 0, 0, stream);
}

int sf_gemm_add(int transA, int transB, int64_t M, int64_t N, int64_t K, int64_t batch, const void* A,
                int64_t lda, int64_t strideA, const void* B, int64_t ldb, int64_t strideB, void* C,
                int64_t ldc, int64_t strideC, sf_dtype ab_dtype, sf_dtype c_dtype, float alpha,
                const void* bias, sf_epilogue epi, const void* R, int64_t ldr, int64_t strideR,
                void* stream) {
  if (R == nullptr && M > 0 && N > 0 && batch > 0) {
    g_err[0] = 0;
    return fail(SF_ERR_INVALID_ARG, "sf_gemm_add: null residual pointer");
  }
  return gemm_run(transA, transB, M, N, K, batch, A, lda, strideA, B, ldb, strideB, C, ldc, strideC, ab_dtype,
                  c_dtype, alpha, bias, epi, R, ldr, strideR, stream);
}

int sf_gemm_plan(int transA, int transB, int64_t M, int64_t N, int64_t K, int64_t batch,
                 const void* A, int64_t lda, int64_t strideA, const void* B, int64_t ldb,
                 int64_t strideB, void* C, int64_t ldc, int64_t strideC, sf_dtype ab_dtype,
                 sf_dtype c_dtype, float alpha, const void* bias, sf_epilogue epi, char* buf,
                 int len) {
  if (buf == nullptr || len <= 0) return fail(SF_ERR_INVALID_ARG, "sf_gemm_plan: bad buffer");
  buf[0] = 0;
  GemmPlan plan;
  int rc = gemm_prepare(transA, transB, M, N, K, batch, A, lda, strideA, B, ldb, strideB, C, ldc,
                        strideC, ab_dtype, c_dtype, alpha, bias, epi, nullptr, 0, 0, false, plan);
  if (rc != SF_OK) return rc;
  char extra[64] = "";
  if (!plan.noop && plan.p.split > 0)
    snprintf(extra, sizeof(extra), "%s split-tail %dx%d", plan.p.persist > 0 ? " persistent" : "",
             plan.p.tiles_m * plan.p.tiles_n - plan.p.full_tiles, plan.p.split);
  else if (!plan.noop && plan.p.persist > 0)
    snprintf(extra, sizeof(extra), " persistent");
  else if (!plan.noop && plan.p.wave4 > 0)
    snprintf(extra, sizeof(extra), " 4-wave");
  const char* name = plan.noop ? "noop" : tile_name(plan.cfg);
  if (!plan.noop && plan.cfg == TILE_NT_BIG)  // the LDS-DMA kernel takes every operand layout
    name = plan.a_kmajor ? (plan.b_kmajor ? "gemm nt 256x256 lds-dma" : "gemm nn 256x256 lds-dma")
                         : (plan.b_kmajor ? "gemm tt 256x256 lds-dma" : "gemm tn 256x256 lds-dma");
  snprintf(buf, (size_t)len, "%s%s%s", name, plan.noop ? "" : (plan.fp32 ? " fp32" : " 16-bit"), extra);
  return SF_OK;
}

// (b, h) entries of one operand do not overlap: heads side by side within
// a row (hS >= D, (H-1) hS + D <= ld) or stacked as whole matrices
// (hS >= (S-1) ld + D), and batch entries past every head's last element.
static bool attn_out_disjoint(int64_t S, int64_t ld, int64_t sB, int64_t sH, int64_t B, int64_t H, int64_t D) {
  const int64_t mat = (S - 1) * ld + D;
  int64_t span;
  if (H <= 1)
    span = mat;
  else if (sH >= D && (H - 1) * sH + D <= ld)
    span = mat + (H - 1) * sH;
  else if (sH >= mat)
    span = (H - 1) * sH + mat;
  else
    return false;
  return B <= 1 || sB >= span;
}

int sf_attention_heads(const void* Q, int64_t ldq, int64_t strideQ, int64_t headQ, const void* K, int64_t ldk,
                       int64_t strideK, int64_t headK, const void* V, int64_t ldv, int64_t strideV, int64_t headV,
                       void* O, int64_t ldo, int64_t strideO, int64_t headO, int64_t batch, int64_t heads,
                       int64_t Sq, int64_t Sk, int64_t D, float scale, sf_dtype dtype, void* stream) {
  g_err[0] = 0;
  if (!valid_dtype(dtype)) return fail(SF_ERR_INVALID_ARG, "sf_attention: unknown dtype %d", (int)dtype);
  if (batch < 0 || heads < 0 || Sq < 0 || Sk < 0 || D < 0)
    return fail(SF_ERR_INVALID_ARG, "sf_attention: negative size");
  if (dtype == SF_F32) return fail(SF_ERR_UNSUPPORTED, "sf_attention: 16-bit dtypes only");
  if (D < 8 || D > 64 || D % 8 != 0)
    return fail(SF_ERR_UNSUPPORTED, "sf_attention: head size %lld (multiples of 8 up to 64)", (long long)D);
  if (!(scale > 0.0f) || scale > 3.0e38f)
    return fail(SF_ERR_UNSUPPORTED, "sf_attention: scale %g (positive and finite only)", (double)scale);
  if (batch == 0 || heads == 0 || Sq == 0) return SF_OK;
  if (Sk == 0) return fail(SF_ERR_INVALID_ARG, "sf_attention: softmax over zero keys");
  if (Q == nullptr || K == nullptr || V == nullptr || O == nullptr)
    return fail(SF_ERR_INVALID_ARG, "sf_attention: null pointer");
  if (ldq < D || ldk < D || ldv < D || ldo < D)
    return fail(SF_ERR_INVALID_ARG, "sf_attention: row stride below the head size");
  if (strideQ < 0 || strideK < 0 || strideV < 0 || strideO < 0 || headQ < 0 || headK < 0 || headV < 0 ||
      headO < 0)
    return fail(SF_ERR_INVALID_ARG, "sf_attention: negative batch or head stride");
  if (!attn_out_disjoint(Sq, ldo, strideO, headO, batch, heads, D))
    return fail(SF_ERR_INVALID_ARG, "sf_attention: output (batch, head) entries overlap");
  // Key rows up to the next multiple of 64 past Sk are addressed (and read
  // as zeros) with 32-bit offsets.
  if (Sq > INT32_MAX || heads > INT32_MAX || (Sk + 64) * (ldk > ldv ? ldk : ldv) * 2 >= (int64_t(1) << 31))
    return fail(SF_ERR_UNSUPPORTED, "sf_attention: K/V of one batch entry must stay below 2 GiB");
  if (!al16(Q) || !al16(K) || !al16(V) || !al16(O) || ldq % 8 || ldk % 8 || ldv % 8 || ldo % 8 ||
      strideQ % 8 || strideK % 8 || strideV % 8 || strideO % 8 || headQ % 8 || headK % 8 || headV % 8 ||
      headO % 8)
    return fail(SF_ERR_UNSUPPORTED, "sf_attention: rows must be 16-byte aligned");
  AttnShape a;
  a.Q = Q; a.K = K; a.V = V; a.O = O;
  a.ldq = ldq; a.ldk = ldk; a.ldv = ldv; a.ldo = ldo;
  a.sQ = strideQ; a.sK = strideK; a.sV = strideV; a.sO = strideO;
  a.hQ = headQ; a.hK = headK; a.hV = headV; a.hO = headO;
  a.batch = batch; a.heads = heads; a.Sq = Sq; a.Sk = Sk;
  a.D = D;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const AttnSplit sp = attn_split_plan(a, cu_count_current());
  if (sp.parts == 0) return launch_attention(a, scale, dtype, sp, nullptr, st);
  float* ws = nullptr;
  int* cnt = nullptr;
  int rc = split_workspace_acquire((size_t)(sp.items - sp.full) * (size_t)sp.parts * kAttnPartBytes, 0, st, &ws,
                                   &cnt);
  if (rc != SF_OK) return rc;
  rc = launch_attention(a, scale, dtype, sp, ws, st);
  const int rc2 = split_workspace_release(st);
  return rc != SF_OK ? rc : rc2;
}

int sf_attention(const void* Q, int64_t ldq, int64_t strideQ, const void* K, int64_t ldk, int64_t strideK,
                 const void* V, int64_t ldv, int64_t strideV, void* O, int64_t ldo, int64_t strideO,
                 int64_t batch, int64_t Sq, int64_t Sk, int64_t D, float scale, sf_dtype dtype, void* stream) {
  return sf_attention_heads(Q, ldq, strideQ, 0, K, ldk, strideK, 0, V, ldv, strideV, 0, O, ldo, strideO, 0, batch,
                            1, Sq, Sk, D, scale, dtype, stream);
}

int sf_layer_norm(const void* x, void* y, int64_t rows, int64_t cols, const void* gamma, const void* beta,
                  float eps, const void* mod_scale, const void* mod_shift, int64_t mod_ld, int64_t group_rows,
                  float* mean_out, float* rstd_out, sf_dtype dt, void* stream) {
  g_err[0] = 0;
  if (!valid_dtype(dt)) return fail(SF_ERR_INVALID_ARG, "sf_layer_norm: unknown dtype %d", (int)dt);
  if (rows < 0 || cols < 0) return fail(SF_ERR_INVALID_ARG, "sf_layer_norm: negative size");
  if (rows == 0) return SF_OK;
  if (cols == 0) return fail(SF_ERR_INVALID_ARG, "sf_layer_norm: normalising over zero columns");
  if (cols > INT32_MAX) return fail(SF_ERR_UNSUPPORTED, "sf_layer_norm: cols must be < 2^31");
  if (x == nullptr || y == nullptr) return fail(SF_ERR_INVALID_ARG, "sf_layer_norm: null pointer");
  if (!(eps >= 0.0f)) return fail(SF_ERR_INVALID_ARG, "sf_layer_norm: eps must be >= 0");
  const bool mod = mod_scale != nullptr || mod_shift != nullptr;
  if (mod && (mod_ld < cols || group_rows < 1))
    return fail(SF_ERR_INVALID_ARG, "sf_layer_norm: modulation needs mod_ld >= cols and group_rows >= 1 "
                "(mod_ld=%lld group_rows=%lld)", (long long)mod_ld, (long long)group_rows);
  NormArgs a;
  a.x = x; a.y = y; a.gamma = gamma; a.beta = beta;
  a.mscale = mod_scale; a.mshift = mod_shift;
  a.mean_out = mean_out; a.rstd_out = rstd_out;
  a.rows = rows; a.cols = cols; a.mld = mod ? mod_ld : 0; a.group_rows = mod ? group_rows : 1;
  a.eps = eps; a.rms = false;
  return launch_norm(a, dt, static_cast<hipStream_t>(stream));
}

int sf_rms_norm(const void* x, void* y, int64_t rows, int64_t cols, const void* gamma, float eps, sf_dtype dt,
                void* stream) {
  g_err[0] = 0;
  if (!valid_dtype(dt)) return fail(SF_ERR_INVALID_ARG, "sf_rms_norm: unknown dtype %d", (int)dt);
  if (rows < 0 || cols < 0) return fail(SF_ERR_INVALID_ARG, "sf_rms_norm: negative size");
  if (rows == 0) return SF_OK;
  if (cols == 0) return fail(SF_ERR_INVALID_ARG, "sf_rms_norm: normalising over zero columns");
  if (cols > INT32_MAX) return fail(SF_ERR_UNSUPPORTED, "sf_rms_norm: cols must be < 2^31");
  if (x == nullptr || y == nullptr) return fail(SF_ERR_INVALID_ARG, "sf_rms_norm: null pointer");
  if (!(eps >= 0.0f)) return fail(SF_ERR_INVALID_ARG, "sf_rms_norm: eps must be >= 0");
  NormArgs a;
  a.x = x; a.y = y; a.gamma = gamma; a.beta = nullptr;
  a.mscale = nullptr; a.mshift = nullptr;
  a.mean_out = nullptr; a.rstd_out = nullptr;
  a.rows = rows; a.cols = cols; a.mld = 0; a.group_rows = 1;
  a.eps = eps; a.rms = true;
  return launch_norm(a, dt, static_cast<hipStream_t>(stream));
}

int sf_add(const void* a, const void* b, void* y, int64_t n, sf_dtype dt, void* stream) {
  g_err[0] = 0;
  if (!valid_dtype(dt)) return fail(SF_ERR_INVALID_ARG, "sf_add: unknown dtype %d", (int)dt);
  if (n < 0) return fail(SF_ERR_INVALID_ARG, "sf_add: negative size");
  if (n == 0) return SF_OK;
  if (a == nullptr || b == nullptr || y == nullptr) return fail(SF_ERR_INVALID_ARG, "sf_add: null pointer");
  return launch_add(a, b, y, n, dt, static_cast<hipStream_t>(stream));
}

int sf_sum_dim(const void* x, void* out, int64_t outer, int64_t dim_size, int64_t inner, sf_dtype in_dtype,
               sf_dtype out_dtype, void* stream) {
  g_err[0] = 0;
  if (!valid_dtype(in_dtype) || !valid_dtype(out_dtype))
    return fail(SF_ERR_INVALID_ARG, "sf_sum_dim: unknown dtype");
  if (out_dtype != in_dtype && out_dtype != SF_F32)
    return fail(SF_ERR_UNSUPPORTED, "sf_sum_dim: output dtype must equal the input dtype or be F32");
  if (outer < 0 || dim_size < 0 || inner < 0) return fail(SF_ERR_INVALID_ARG, "sf_sum_dim: negative size");
  if (inner > INT32_MAX || dim_size > INT32_MAX || outer > INT32_MAX)
    return fail(SF_ERR_UNSUPPORTED, "sf_sum_dim: outer, dim_size and inner must be < 2^31");
  if (outer == 0 || inner == 0) return SF_OK;
  if (x == nullptr || out == nullptr) return fail(SF_ERR_INVALID_ARG, "sf_sum_dim: null pointer");
  if (inner > 1 && outer > 65535) return fail(SF_ERR_UNSUPPORTED, "sf_sum_dim: outer must be < 65536 when inner > 1");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int S = sum_dim_parts(outer, dim_size, inner, cu_count_current());
  if (S == 1) return launch_sum_dim(x, out, outer, dim_size, inner, in_dtype, out_dtype, nullptr, 1, st);
  float* ws = nullptr;
  int* cnt = nullptr;
  int rc = split_workspace_acquire((size_t)S * (size_t)outer * (size_t)inner * sizeof(float), 0, st, &ws, &cnt);
  if (rc != SF_OK) return rc;
  rc = launch_sum_dim(x, out, outer, dim_size, inner, in_dtype, out_dtype, ws, S, st);
  const int rc2 = split_workspace_release(st);
  return rc != SF_OK ? rc : rc2;
}

int sf_softmax_rows(const void* x, void* y, int64_t rows, int64_t cols, sf_dtype in_dtype,
                    sf_dtype out_dtype, float scale, void* stream) {
  g_err[0] = 0;
  if (!valid_dtype(in_dtype) || !valid_dtype(out_dtype))
    return fail(SF_ERR_INVALID_ARG, "sf_softmax_rows: unknown dtype");
  if (rows < 0 || cols < 0) return fail(SF_ERR_INVALID_ARG, "sf_softmax_rows: negative size");
  if (rows > INT32_MAX || cols > INT32_MAX)
    return fail(SF_ERR_INVALID_ARG, "sf_softmax_rows: rows and cols must be < 2^31");
  if (rows == 0 || cols == 0) return SF_OK;
  if (x == nullptr || y == nullptr) return fail(SF_ERR_INVALID_ARG, "sf_softmax_rows: null pointer");
  return launch_softmax(x, y, rows, cols, in_dtype, out_dtype, scale, static_cast<hipStream_t>(stream));
}

int sf_softmax_rows_masked(const void* x, void* y, int64_t rows, int64_t cols, sf_dtype dtype, float scale,
                           const void* mask, sf_dtype mask_dtype, int64_t rows_per_batch, int64_t inner_batches,
                           int64_t stride_outer, int64_t stride_inner, int64_t stride_row, int64_t stride_col,
                           void* stream) {
  g_err[0] = 0;
  if (!valid_dtype(dtype) || !valid_dtype(mask_dtype))
    return fail(SF_ERR_INVALID_ARG, "sf_softmax_rows_masked: unknown dtype");
  if (mask_dtype != dtype && mask_dtype != SF_F32)
    return fail(SF_ERR_UNSUPPORTED, "sf_softmax_rows_masked: the mask's dtype must be the scores' dtype or F32");
  if (rows < 0 || cols < 0) return fail(SF_ERR_INVALID_ARG, "sf_softmax_rows_masked: negative size");
  if (rows > INT32_MAX || cols > INT32_MAX)
    return fail(SF_ERR_INVALID_ARG, "sf_softmax_rows_masked: rows and cols must be < 2^31");
  if (rows == 0 || cols == 0) return SF_OK;
  if (x == nullptr || y == nullptr || mask == nullptr)
    return fail(SF_ERR_INVALID_ARG, "sf_softmax_rows_masked: null pointer");
  if (rows_per_batch < 1 || rows % rows_per_batch != 0 || inner_batches < 1)
    return fail(SF_ERR_INVALID_ARG, "sf_softmax_rows_masked: rows_per_batch must divide rows, inner_batches >= 1");
  if (stride_outer < 0 || stride_inner < 0 || stride_row < 0 || (stride_col != 0 && stride_col != 1))
    return fail(SF_ERR_INVALID_ARG, "sf_softmax_rows_masked: negative mask stride, or stride_col not 0 or 1");
  MaskArgs ma;
  ma.m = mask;
  ma.per = rows_per_batch;
  ma.inner = inner_batches;
  ma.souter = stride_outer;
  ma.sinner = stride_inner;
  ma.srow = stride_row;
  ma.scol = (int)stride_col;
  return launch_softmax_masked(x, y, rows, cols, dtype, scale, ma, mask_dtype, static_cast<hipStream_t>(stream));
}

static int unary_common(int op, const void* x, void* y, int64_t n, sf_dtype dt, float s,
                        void* stream, const char* name) {
  g_err[0] = 0;
  if (!valid_dtype(dt)) return fail(SF_ERR_INVALID_ARG, "%s: unknown dtype", name);
  if (n < 0) return fail(SF_ERR_INVALID_ARG, "%s: negative size", name);
  if (n == 0) return SF_OK;
  if (x == nullptr || y == nullptr) return fail(SF_ERR_INVALID_ARG, "%s: null pointer", name);
  return launch_unary(op, x, y, n, dt, s, static_cast<hipStream_t>(stream));
}

int sf_silu(const void* x, void* y, int64_t n, sf_dtype dt, void* stream) {
  return unary_common(0, x, y, n, dt, 1.0f, stream, "sf_silu");
}
int sf_gelu(const void* x, void* y, int64_t n, sf_dtype dt, void* stream) {
  return unary_common(1, x, y, n, dt, 1.0f, stream, "sf_gelu");
}
int sf_muls(const void* x, float s, void* y, int64_t n, sf_dtype dt, void* stream) {
  return unary_common(2, x, y, n, dt, s, stream, "sf_muls");
}

int sf_dropout(const void* x, void* y, void* mask, int64_t n, sf_dtype dt, float p, uint64_t seed,
               uint64_t offset, void* stream) {
  g_err[0] = 0;
  if (!valid_dtype(dt)) return fail(SF_ERR_INVALID_ARG, "sf_dropout: unknown dtype");
  if (n < 0) return fail(SF_ERR_INVALID_ARG, "sf_dropout: negative size");
  if (!(p >= 0.0f && p < 1.0f)) return fail(SF_ERR_INVALID_ARG, "sf_dropout: p must be in [0, 1)");
  if (n == 0) return SF_OK;
  if (x == nullptr || y == nullptr) return fail(SF_ERR_INVALID_ARG, "sf_dropout: null pointer");
  return launch_dropout(x, y, mask, n, dt, p, seed, offset, static_cast<hipStream_t>(stream));
}

int sf_bias_add_rows(void* C, const void* bias, int64_t M, int64_t N, sf_dtype dt, void* stream) {
  g_err[0] = 0;
  if (!valid_dtype(dt)) return fail(SF_ERR_INVALID_ARG, "sf_bias_add_rows: unknown dtype");
  if (M < 0 || N < 0) return fail(SF_ERR_INVALID_ARG, "sf_bias_add_rows: negative size");
  if (M == 0 || N == 0) return SF_OK;
  if (C == nullptr || bias == nullptr)
    return fail(SF_ERR_INVALID_ARG, "sf_bias_add_rows: null pointer");
  return launch_bias_rows(C, bias, M, N, dt, static_cast<hipStream_t>(stream));
}

int sf_cast(const void* x, sf_dtype in_dtype, void* y, sf_dtype out_dtype, int64_t n, void* stream) {
  g_err[0] = 0;
  if (!valid_dtype(in_dtype) || !valid_dtype(out_dtype))
    return fail(SF_ERR_INVALID_ARG, "sf_cast: unknown dtype");
  if (n < 0) return fail(SF_ERR_INVALID_ARG, "sf_cast: negative size");
  if (n == 0) return SF_OK;
  if (x == nullptr || y == nullptr) return fail(SF_ERR_INVALID_ARG, "sf_cast: null pointer");
  return launch_cast(x, in_dtype, y, out_dtype, n, static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------------
// Runtime
// ---------------------------------------------------------------------
int sf_get_device_count(int* count) {
  if (count == nullptr) return fail(SF_ERR_INVALID_ARG, "sf_get_device_count: null pointer");
  *count = 0;
  hipError_t e = hipGetDeviceCount(count);
  if (e == hipErrorNoDevice) {
    *count = 0;
    return SF_OK;
  }
  if (e != hipSuccess) *count = 0;
  return check_hip(e, "hipGetDeviceCount");
}

int sf_set_device(int device) { return check_hip(hipSetDevice(device), "hipSetDevice"); }

int sf_get_device(int* device) {
  if (device == nullptr) return fail(SF_ERR_INVALID_ARG, "sf_get_device: null pointer");
  return check_hip(hipGetDevice(device), "hipGetDevice");
}

int sf_device_synchronize(void) { return check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize"); }

int sf_get_device_name(int device, char* buf, int len) {
  if (buf == nullptr || len <= 0) return fail(SF_ERR_INVALID_ARG, "sf_get_device_name: bad buffer");
  hipDeviceProp_t prop;
  int rc = check_hip(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
  if (rc != SF_OK) return rc;
  snprintf(buf, (size_t)len, "%s", prop.name);
  return SF_OK;
}

int sf_get_device_arch(int device, char* buf, int len) {
  if (buf == nullptr || len <= 0) return fail(SF_ERR_INVALID_ARG, "sf_get_device_arch: bad buffer");
  hipDeviceProp_t prop;
  int rc = check_hip(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
  if (rc != SF_OK) return rc;
  snprintf(buf, (size_t)len, "%s", prop.gcnArchName);
  return SF_OK;
}

int sf_get_device_props(int device, int* cu_count, int64_t* total_mem, int* clock_khz,
                        int* l2_bytes) {
  hipDeviceProp_t prop;
  int rc = check_hip(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
  if (rc != SF_OK) return rc;
  if (cu_count) *cu_count = prop.multiProcessorCount;
  if (total_mem) *total_mem = (int64_t)prop.totalGlobalMem;
  if (clock_khz) *clock_khz = prop.clockRate;
  if (l2_bytes) *l2_bytes = prop.l2CacheSize;
  return SF_OK;
}

int sf_mem_get_info(size_t* free_bytes, size_t* total_bytes) {
  if (free_bytes == nullptr || total_bytes == nullptr)
    return fail(SF_ERR_INVALID_ARG, "sf_mem_get_info: null pointer");
  return check_hip(hipMemGetInfo(free_bytes, total_bytes), "hipMemGetInfo");
}

int sf_malloc(void** ptr, size_t nbytes) {
  if (ptr == nullptr) return fail(SF_ERR_INVALID_ARG, "sf_malloc: null pointer");
  *ptr = nullptr;
  return check_hip(hipMalloc(ptr, nbytes ? nbytes : 1), "hipMalloc");
}

int sf_free(void* ptr) { return check_hip(hipFree(ptr), "hipFree"); }

// ---------------------------------------------------------------------
// Caching allocator: per-device free lists keyed by the 256-byte-rounded
// size.  A freed block is kept for reuse; when the device's pooled bytes
// would exceed the limit (default 16 GiB of the 288 GB HBM), pooled blocks
// of the sizes least recently used are returned with hipFree first, so a
// pool filled by an earlier workload's sizes is emptied once instead of
// every free of the new sizes paying a hipFree (which synchronises the
// device).  A block larger than the limit itself is freed directly.  An
// allocation that fails with out-of-memory empties that device's pool and
// retries once.
// ---------------------------------------------------------------------
namespace {
struct Pool {
  std::unordered_map<size_t, std::vector<void*>> free_lists;
  std::unordered_map<size_t, uint64_t> last_use;  // size -> tick of its last alloc or free
  uint64_t tick = 0;
  size_t pooled = 0;
  size_t live = 0;
};
std::mutex g_pool_mu;
std::unordered_map<int, Pool> g_pools;
size_t g_pool_limit = size_t(16) << 30;

size_t round256(size_t n) { return n == 0 ? 256 : (n + 255) & ~size_t(255); }

// Frees every pooled block of `dev` (caller holds the lock and has made
// `dev` current).
void drain_pool(Pool& pool) {
  for (auto& kv : pool.free_lists)
    for (void* p : kv.second) (void)hipFree(p);
  pool.free_lists.clear();
  pool.pooled = 0;
}

// Frees pooled blocks of sizes other than `keep`, least recently used size
// first, until `need` more bytes fit under the limit (caller holds the lock
// and has made the pool's device current).
void evict_for(Pool& pool, size_t keep, size_t need) {
  std::vector<std::pair<uint64_t, size_t>> order;
  for (auto& kv : pool.free_lists)
    if (kv.first != keep && !kv.second.empty()) order.emplace_back(pool.last_use[kv.first], kv.first);
  std::sort(order.begin(), order.end());
  for (auto& o : order) {
    auto& lst = pool.free_lists[o.second];
    while (!lst.empty() && pool.pooled + need > g_pool_limit) {
      (void)hipFree(lst.back());
      lst.pop_back();
      pool.pooled -= o.second;
    }
    if (lst.empty()) pool.free_lists.erase(o.second);
    if (pool.pooled + need <= g_pool_limit) return;
  }
}

struct DeviceGuard {
  int prev = -1;
  bool switched = false;
  int enter(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) {
      int rc = check_hip(hipSetDevice(dev), "hipSetDevice");
      if (rc != SF_OK) return rc;
      switched = true;
    }
    return SF_OK;
  }
  ~DeviceGuard() {
    if (switched && prev >= 0) (void)hipSetDevice(prev);
  }
};
}  // namespace

int sf_cache_alloc(int device, size_t nbytes, void** ptr, size_t* got_bytes) {
  if (ptr == nullptr) return fail(SF_ERR_INVALID_ARG, "sf_cache_alloc: null pointer");
  *ptr = nullptr;
  const size_t sz = round256(nbytes);
  std::lock_guard<std::mutex> lk(g_pool_mu);
  Pool& pool = g_pools[device];
  pool.last_use[sz] = ++pool.tick;
  auto it = pool.free_lists.find(sz);
  if (it != pool.free_lists.end() && !it->second.empty()) {
    *ptr = it->second.back();
    it->second.pop_back();
    pool.pooled -= sz;
    pool.live += sz;
    if (got_bytes) *got_bytes = sz;
    return SF_OK;
  }
  DeviceGuard g;
  int rc = g.enter(device);
  if (rc != SF_OK) return rc;
  hipError_t e = hipMalloc(ptr, sz);
  if (e == hipErrorOutOfMemory && pool.pooled > 0) {
    (void)hipGetLastError();
    drain_pool(pool);
    e = hipMalloc(ptr, sz);
  }
  if (e != hipSuccess) {
    *ptr = nullptr;
    return check_hip(e, "hipMalloc (caching allocator)");
  }
  pool.live += sz;
  if (got_bytes) *got_bytes = sz;
  return SF_OK;
}

int sf_cache_free(int device, void* ptr, size_t nbytes) {
  if (ptr == nullptr) return SF_OK;
  const size_t sz = round256(nbytes);
  std::lock_guard<std::mutex> lk(g_pool_mu);
  Pool& pool = g_pools[device];
  pool.live = pool.live >= sz ? pool.live - sz : 0;
  pool.last_use[sz] = ++pool.tick;
  if (pool.pooled + sz > g_pool_limit) {
    DeviceGuard g;
    int rc = g.enter(device);
    if (rc != SF_OK) return rc;
    if (sz <= g_pool_limit) evict_for(pool, sz, sz);
    if (pool.pooled + sz > g_pool_limit) return check_hip(hipFree(ptr), "hipFree (caching allocator)");
  }
  pool.free_lists[sz].push_back(ptr);
  pool.pooled += sz;
  return SF_OK;
}

int sf_cache_empty(int device) {
  std::lock_guard<std::mutex> lk(g_pool_mu);
  for (auto& kv : g_pools) {
    if (device >= 0 && kv.first != device) continue;
    DeviceGuard g;
    int rc = g.enter(kv.first);
    if (rc != SF_OK) return rc;
    drain_pool(kv.second);
  }
  return SF_OK;
}

int sf_cache_stats(int device, size_t* pooled_bytes, size_t* live_bytes) {
  std::lock_guard<std::mutex> lk(g_pool_mu);
  size_t pooled = 0, live = 0;
  for (auto& kv : g_pools) {
    if (device >= 0 && kv.first != device) continue;
    pooled += kv.second.pooled;
    live += kv.second.live;
  }
  if (pooled_bytes) *pooled_bytes = pooled;
  if (live_bytes) *live_bytes = live;
  return SF_OK;
}

int sf_workspace_bytes(int device, size_t* bytes) {
  if (bytes == nullptr) return fail(SF_ERR_INVALID_ARG, "sf_workspace_bytes: null pointer");
  std::lock_guard<std::mutex> lk(g_ws_mu);
  size_t total = 0;
  for (auto& kv : g_ws) {
    if (device >= 0 && kv.first != device) continue;
    if (kv.second.base != nullptr) total += kv.second.part_bytes + (size_t)kv.second.counters * sizeof(int);
  }
  *bytes = total;
  return SF_OK;
}

int sf_cache_set_limit(size_t bytes_per_device) {
  std::lock_guard<std::mutex> lk(g_pool_mu);
  g_pool_limit = bytes_per_device;
  return SF_OK;
}

int sf_memcpy_h2d(void* dst, const void* src, size_t nbytes, void* stream) {
  if (nbytes == 0) return SF_OK;
  if (dst == nullptr || src == nullptr) return fail(SF_ERR_INVALID_ARG, "sf_memcpy_h2d: null pointer");
  if (stream == nullptr) return check_hip(hipMemcpy(dst, src, nbytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
  return check_hip(hipMemcpyAsync(dst, src, nbytes, hipMemcpyHostToDevice, (hipStream_t)stream),
                   "hipMemcpyAsync H2D");
}

int sf_memcpy_d2h(void* dst, const void* src, size_t nbytes, void* stream) {
  if (nbytes == 0) return SF_OK;
  if (dst == nullptr || src == nullptr) return fail(SF_ERR_INVALID_ARG, "sf_memcpy_d2h: null pointer");
  if (stream == nullptr) return check_hip(hipMemcpy(dst, src, nbytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
  return check_hip(hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToHost, (hipStream_t)stream),
                   "hipMemcpyAsync D2H");
}

int sf_memcpy_d2d(void* dst, const void* src, size_t nbytes, void* stream) {
  if (nbytes == 0) return SF_OK;
  if (dst == nullptr || src == nullptr) return fail(SF_ERR_INVALID_ARG, "sf_memcpy_d2d: null pointer");
  return check_hip(hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToDevice, (hipStream_t)stream),
                   "hipMemcpyAsync D2D");
}

int sf_zero(void* dst, size_t nbytes, void* stream) {
  if (nbytes == 0) return SF_OK;
  if (dst == nullptr) return fail(SF_ERR_INVALID_ARG, "sf_zero: null pointer");
  return launch_zero(dst, nbytes, (hipStream_t)stream);
}

int sf_stream_create(void** stream) {
  if (stream == nullptr) return fail(SF_ERR_INVALID_ARG, "sf_stream_create: null pointer");
  hipStream_t s = nullptr;
  int rc = check_hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags");
  *stream = s;
  return rc;
}

int sf_stream_destroy(void* stream) {
  if (stream == nullptr) return SF_OK;
  return check_hip(hipStreamDestroy((hipStream_t)stream), "hipStreamDestroy");
}

int sf_stream_synchronize(void* stream) {
  return check_hip(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
}

int sf_event_create(void** event) {
  if (event == nullptr) return fail(SF_ERR_INVALID_ARG, "sf_event_create: null pointer");
  hipEvent_t e = nullptr;
  int rc = check_hip(hipEventCreate(&e), "hipEventCreate");
  *event = e;
  return rc;
}

int sf_event_destroy(void* event) {
  if (event == nullptr) return SF_OK;
  return check_hip(hipEventDestroy((hipEvent_t)event), "hipEventDestroy");
}

int sf_event_record(void* event, void* stream) {
  if (event == nullptr) return fail(SF_ERR_INVALID_ARG, "sf_event_record: null event");
  return check_hip(hipEventRecord((hipEvent_t)event, (hipStream_t)stream), "hipEventRecord");
}

int sf_event_synchronize(void* event) {
  if (event == nullptr) return fail(SF_ERR_INVALID_ARG, "sf_event_synchronize: null event");
  return check_hip(hipEventSynchronize((hipEvent_t)event), "hipEventSynchronize");
}

int sf_stream_wait_event(void* stream, void* event) {
  if (event == nullptr) return fail(SF_ERR_INVALID_ARG, "sf_stream_wait_event: null event");
  return check_hip(hipStreamWaitEvent((hipStream_t)stream, (hipEvent_t)event, 0), "hipStreamWaitEvent");
}

int sf_event_elapsed_ms(float* ms, void* start, void* end) {
  if (ms == nullptr || start == nullptr || end == nullptr)
    return fail(SF_ERR_INVALID_ARG, "sf_event_elapsed_ms: null pointer");
  return check_hip(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end), "hipEventElapsedTime");
}

}  // extern "C"
