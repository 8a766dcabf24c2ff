// sf_internal.hpp — host-side declarations shared by the translation units
// of libsfgemm (launchers, error reporting).  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>

#include "gemm16.hpp"
#include "sf_common.hpp"

namespace sf {

// Records a formatted message as this thread's last error; returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Maps a pending launch error (hipGetLastError) to SF_ERR_HIP with context.
int check_launch(const char* what);
// Maps a HIP status to SF_OK / SF_ERR_HIP with context.
int check_hip(hipError_t e, const char* what);

// Test hooks, set only through sf_set_test_hooks (never read from the
// environment): they force plans the planner would not pick, and every one
// of them must leave results unchanged.
//   xcd_shift   1..7: each part of a persistent split tile expects the XCD
//               this many places from its own (the agent-scope fallback);
//   split_spins >= 0: caps a split part's wait for the others (0: the last
//               part sums every slice); < 0: the built-in bound;
//   attn_parts  2..16: every attention work item split into this many key
//               ranges; 0: the automatic plan.
struct TestHooks {
  std::atomic<int> xcd_shift{0};
  std::atomic<int> split_spins{-1};
  std::atomic<int> attn_parts{0};
};
extern TestHooks g_test_hooks;

// Tile shapes of the 16-bit and fp32 GEMM kernels.
enum TileCfg {
  TILE_256x256 = 0,  // 512 threads, waves 2x4 of 128x64
  TILE_256x128 = 1,  // 512 threads, waves 4x2 of 64x64
  TILE_128x128 = 2,  // 256 threads, waves 2x2 of 64x64
  TILE_256x64 = 3,   // 256 threads, waves 4x1 of 64x64 (narrow N, e.g. P.V)
  TILE_64x64 = 4,    // 256 threads, waves 2x2 of 32x32
  TILE_GENERIC = 5,  // 64x64, element-wise bounds-checked loads (any layout)
  TILE_SKINNY = 6,   // M <= 16 stream kernel
  TILE_NT_BIG = 7,   // 256x256 NT, 8-wave ping-pong, direct-to-LDS (gemm16nt_pp.hpp)
  TILE_SKINNY_LINE = 8,  // M <= 16, K in {2048, 4096, 8192}: row-segment stream (skinny16l)
  // fp32 only:
  TILE32_SMALL1 = 9,     // 16x16 blocks, 4 waves splitting k (gemm32small.hpp)
  TILE32_SMALL2 = 10,    // 16x32 blocks, 8 waves splitting k
  TILE32_DMA = 11,       // 64x64, direct-to-LDS ring, two 4-wave k-groups (gemm32dma.hpp)
  TILE32_DMA_SPLIT = 12,  // 64x64, direct-to-LDS ring, one k-group, split-K capable
  // 16-bit again:
  TILE_NT_K64 = 13  // 128x128 NT with K == 64, four workgroups per CU (gemm16nt_k64.hpp)
};
const char* tile_name(int cfg);

// One GEMM launch: batch entries [0, batch) of p, grid.y <= 65535 per call.
int launch_gemm16(sf_dtype in, sf_dtype out, bool a_kmajor, bool b_kmajor, int cfg, const GemmParams& p,
                  int64_t batch, hipStream_t st);
int launch_gemm16_bf16(sf_dtype out, bool a_kmajor, bool b_kmajor, int cfg, const GemmParams& p, unsigned gx,
                       unsigned gy, hipStream_t st);
int launch_gemm16_f16(sf_dtype out, bool a_kmajor, bool b_kmajor, int cfg, const GemmParams& p, unsigned gx,
                      unsigned gy, hipStream_t st);
int launch_gemm32(bool a_kmajor, bool b_kmajor, int cfg, const GemmParams& p, int64_t batch, hipStream_t st);

// Tile edge of a config (BM, BN).
void tile_dims(int cfg, bool fp32, int& bm, int& bn);

// A validated GEMM launch: the kernel config and its parameters (abi.hip).
struct GemmPlan {
  GemmParams p;
  int cfg;
  bool fp32;
  bool a_kmajor;
  bool b_kmajor;
  bool noop;  // an empty problem: nothing to launch
};
// Validates sf_gemm's arguments (R: residual of sf_gemm_add or NULL;
// need_c: C must be non-NULL) and fills `plan`; no HIP call.
int gemm_prepare(int transA, int transB, int64_t M, int64_t N, int64_t K, int64_t batch, const void* A,
                 int64_t lda, int64_t strideA, const void* B, int64_t ldb, int64_t strideB, void* C, int64_t ldc,
                 int64_t strideC, sf_dtype ab_dtype, sf_dtype c_dtype, float alpha, const void* bias,
                 sf_epilogue epi, const void* R, int64_t ldr, int64_t strideR, bool need_c, GemmPlan& plan);
// The split plan's workspace: fp32 partials (*part_bytes, 0 without a
// split) followed by *counters ints that must be zero at launch.
void gemm_split_needs(const GemmPlan& plan, size_t* part_bytes, int* counters);
// Launches a plan whose workspace pointers (plan.p.ws, plan.p.counters)
// are set when it splits.
int gemm_launch_plan(const GemmPlan& plan, int64_t batch, sf_dtype ab_dtype, sf_dtype c_dtype, hipStream_t st);

// Operands of one fused attention call (element strides): pair (b, h)
// reads Q + b sQ + h hQ (rows of ldq), likewise K, V, and writes O.
struct AttnShape {
  const void* Q;
  const void* K;
  const void* V;
  void* O;
  int64_t ldq, ldk, ldv, ldo;
  int64_t sQ, sK, sV, sO;
  int64_t hQ, hK, hV, hO;
  int64_t batch, heads, Sq, Sk;
  int64_t D;  // head size: a multiple of 8, at most 64
};
// Work items of one attention call: (batch, head) pairs x blocks of 256
// query rows.  Items [0, full) run whole; each later one is split into
// `parts` key ranges (0: no split), whose fp32 partials take
// kAttnPartBytes each in `ws` ((items - full) * parts of them).
struct AttnSplit {
  int64_t items;
  int64_t full;
  int parts;
};
constexpr size_t kAttnPartBytes = 73728;
AttnSplit attn_split_plan(const AttnShape& a, int cus);
int launch_attention(const AttnShape& a, float scale, sf_dtype dt, const AttnSplit& sp, float* ws, hipStream_t st);
// Layer norm (rms = false: centred, gamma and beta, optional per-group
// modulation y = h (1 + scale) + shift) or RMS norm (rms = true: gamma
// only) over `rows` contiguous rows of `cols` elements.
struct NormArgs {
  const void* x;
  void* y;
  const void* gamma;
  const void* beta;
  const void* mscale;
  const void* mshift;
  float* mean_out;
  float* rstd_out;
  int64_t rows, cols, mld, group_rows;
  float eps;
  bool rms;
};
int launch_norm(const NormArgs& a, sf_dtype dt, hipStream_t st);
int launch_add(const void* a, const void* b, void* y, int64_t n, sf_dtype dt, hipStream_t st);
int launch_softmax(const void* x, void* y, int64_t rows, int64_t cols, sf_dtype in, sf_dtype out,
                   float scale, hipStream_t st);
// Additive mask of a masked softmax (see sf_softmax_rows_masked).
struct MaskArgs {
  const void* m;
  int64_t per, inner, souter, sinner, srow;
  int scol;  // 0 or 1
};
// dt: scores in and probabilities out; mask_dt is dt or F32.
int launch_softmax_masked(const void* x, void* y, int64_t rows, int64_t cols, sf_dtype dt, float scale,
                          const MaskArgs& ma, sf_dtype mask_dt, hipStream_t st);
int launch_unary(int op, const void* x, void* y, int64_t n, sf_dtype dt, float s, hipStream_t st);
int launch_dropout(const void* x, void* y, void* mask, int64_t n, sf_dtype dt, float p, uint64_t seed,
                   uint64_t offset, hipStream_t st);
int launch_bias_rows(void* C, const void* bias, int64_t M, int64_t N, sf_dtype dt, hipStream_t st);
int launch_cast(const void* x, sf_dtype in, void* y, sf_dtype out, int64_t n, hipStream_t st);
int launch_zero(void* p, size_t nbytes, hipStream_t st);
// Sum over the middle axis of [outer, D, inner]; S parts (sum_dim_parts)
// with an fp32 workspace of S * outer * inner floats when S > 1.
int sum_dim_parts(int64_t outer, int64_t D, int64_t inner, int cus);
int launch_sum_dim(const void* x, void* y, int64_t outer, int64_t D, int64_t inner, sf_dtype in, sf_dtype out,
                   float* ws, int S, hipStream_t st);

}  // namespace sf
