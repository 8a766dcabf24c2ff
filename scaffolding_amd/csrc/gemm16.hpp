// gemm16.hpp — 16-bit (bf16 / fp16) GEMM on gfx950 MFMA with fp32
// accumulation and a register-fused epilogue.
//
//   C[b] = epi(alpha * A[b] . op(B[b]) (+ bias))      row-major
//
// A is M x K (K-contiguous) or, with A_KMAJOR = false, stored K x M
// (M-contiguous: the product uses its transpose, "TN" / "TT": dW = dY^T X).
// B is either N x K (K-contiguous, "NT": x . W^T, QK^T) or K x N
// (N-contiguous, "NN": A . B, P . V).
//
// Work decomposition
//   * one workgroup per BM x BN output tile, grid.y = batch;
//   * WAVES_M x WAVES_N waves, each owning a WM x WN sub-tile computed as
//     (WN/16) x (WM/16) blocks of v_mfma_f32_16x16x32_{bf16,f16};
//   * K walked in BK = 64 slices, double-buffered in LDS: while the MFMAs
//     consume slice k from one buffer, the 16-byte global loads of slice k+1
//     are in flight into registers and land in the other buffer after the
//     MFMAs, so one barrier per slice suffices.
//
// MFMA operand roles.  The MFMA computes D = X . Y with X lane l holding
// row (l%16) and Y lane l holding column (l%16); lane l receives
// D[4*(l/16)+q][l%16], q = 0..3.  This kernel feeds X from the B tile
// (rows = output columns n) and Y from the A tile (columns = output rows m),
// so lane l ends with C[m = l%16][n = 4*(l/16) + 0..3]: four consecutive
// output columns, i.e. one 8-byte (16-bit out) or 16-byte (fp32 out) store
// and one vector bias load per fragment.
//
// LDS layout.  Both tiles are stored K-contiguous, 64 elements (128 bytes)
// per row, as eight 16-byte chunks; chunk c of row r sits at slot
// c ^ (r & 7).  An MFMA operand read (16 lanes on 16 consecutive rows, same
// chunk) therefore touches 8 distinct slots per 8 lanes — no bank conflicts
// for ds_read_b128 — and the 16-byte global->LDS stores of a row are a
// permutation of the row's slots.  An N-contiguous B tile (and an
// M-contiguous A tile) is transposed on its way into LDS (each 16-byte
// global load of 8 consecutive n scatters into 8 rows); the lane->k
// assignment makes each ds_write_b16 instruction cover 64 distinct 2-byte
// slots of one 128-byte row group.
#pragma once

#include "sf_common.hpp"

namespace sf {

// Most k-parts of an fp32 split-K tile (the kernels keep every part's
// partial-sum loads in flight at once).
constexpr int kMaxSplit32 = 8;

struct GemmParams {
  const void* A;
  const void* B;
  void* C;
  const void* bias;
  int64_t lda, ldb, ldc;
  int64_t sA, sB, sC;  // batch strides, elements (0 = broadcast)
  int M, N, K;
  float alpha;
  int epi;  // sf_epilogue
  int tiles_m, tiles_n;
  int rows_per;  // skinny line kernel: W rows per workgroup
  // Split tail of the 256 x 256 NT kernel (batch 1): tiles [0, full_tiles)
  // run whole; each later tile is split over k into `split` parts whose
  // fp32 partial tiles go to `ws` (256 KB each) and are summed, in part
  // order, by the part that finishes last (`counters`: one per split tile,
  // zero between launches).  split == 0: no tail split.
  // fp32 kernels: every tile split into `split` parts (at most kMaxSplit32),
  // one workgroup each, summed the same way.
  int full_tiles, split;
  float* ws;
  int* counters;
  // Residual added after the activation, R[b] M x N of the output dtype
  // (row stride ldr, batch stride sR; NULL: none).  R may be C itself
  // (same pointer and ldc): every element is read before it is written.
  const void* res;
  int64_t ldr, sR;
  // 256 x 256 NT kernel, batch 1: > 0 runs the persistent variant on this
  // many workgroups (one per CU, a multiple of 8); 0: one workgroup per
  // tile (or split part).
  int persist;
  // Added to the XCD a persistent split part expects to run on (0 in
  // production).  A test sets it to make every part see itself off its XCD
  // and take the agent-scope fallback of split_arrive_xcd.
  int xcd_shift;
  // Most polls a part of a shared split sum waits for the other parts
  // (kSplitArriveSpins in production).  A test sets 0 so that every part
  // but the last gives up at once and the last sums every slice.
  int arrive_spins;
  // 256 x 256 NT kernel, one workgroup per tile and no split: 1 runs the
  // one-wave-per-SIMD variant (gemm16nt_4w.hpp), bit-identical results.
  int wave4;
};

// Split-tile arrival, called by one thread of a workgroup after every
// thread's partial stores (plain global stores) completed: s_waitcnt
// vmcnt(0), then a workgroup barrier.  Returns how many of the `parts`
// parts of the tile arrived before this one.
//
// The XCDs' L2 caches are not coherent with each other, so the increment
// is bracketed by agent-scope fences: release (L2 write-back), an explicit
// wait for that write-back (the compiler leaves none between the
// write-back and the atomic), and, for the last part only (the one that
// reads the others' partials, with plain loads), acquire (L2
// invalidate).  A
// relaxed counter with sc0 sc1 (write-through / coherent) stores and loads
// instead was measured wrong: a 2-way split of 1024^3 fp32 on 64 x 64
// tiles, two workgroups per CU, read stale partials in about 0.1 % of
// outputs, with or without these fences around the counter.  Consistent
// with every measurement, though not proven: a write-through store counts
// as complete before it reaches memory, and the L2 write-back waits only
// for dirty lines, not for write-throughs already in flight; plain stores
// leave the partial dirty in L2, where the write-back moves it and waits.
__device__ __forceinline__ int split_arrive(int* counter, int parts) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __builtin_amdgcn_s_waitcnt(0);
  const int before = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (before == parts - 1) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  return before;
}

// Split-tile arrival for parts that the launch places on one XCD (so they
// share its L2): called by one thread after every thread's partial stores
// completed (s_waitcnt vmcnt(0), workgroup barrier).  The stores are then
// in the XCD's L2, where the last part reads them, so no L2 write-back or
// invalidate is needed.  Each part checks that it really runs on the XCD
// the launch intended (hardware register XCC_ID against `xcd`); one that
// does not releases at agent scope (L2 write-back) and flags its arrival
// (bit 16 and up), and the last part then acquires at agent scope before
// reading.  Returns how many parts arrived before this one.
__device__ __forceinline__ int split_arrive_xcd(int* counter, int parts, int xcd) {
  const int xcc = __builtin_amdgcn_s_getreg((3 << 11) | 20) & 15;  // HW_REG_XCC_ID[3:0]
  const bool off = xcc != xcd;
  if (off) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __builtin_amdgcn_s_waitcnt(0);
  }
  const int before = __hip_atomic_fetch_add(counter, off ? 0x10001 : 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if ((before & 0xffff) == parts - 1 && ((before >> 16) != 0 || off)) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  return before & 0xffff;
}

// Bounded waits of the shared split hand-off, in polls of the arrival word
// (an agent-scope load plus s_sleep 1, about a microsecond each): how long a
// part waits for the other parts to arrive, and how long the last part waits
// for the others to claim their slices before it takes what is unclaimed.
constexpr int kSplitArriveSpins = 256;
constexpr int kSplitClaimSpins = 32;

// Split hand-off with the final sum shared among the parts, for launches
// whose parts of one tile are all resident at once (the persistent grid, one
// workgroup per CU).  Called by one thread of each part after every thread's
// partial stores completed (s_waitcnt vmcnt(0), workgroup barrier).  Three
// words per split tile, all zero between launches:
//   w[0] arrivals: bits 0-3 parts arrived, bits 4-7 those of them that ran
//        off the XCD the launch intended (they release at agent scope, and
//        the readers then acquire at agent scope, as in split_arrive_xcd);
//   w[1] claimed slices: bit q set once some part has taken slice q;
//   w[2] parts done with w[0] and w[1]; the part that completes it clears
//        all three for the next launch (every other part has made its last
//        access to them by then).
// Slice q is the part's share of the final sum (the kernel maps it to rows).
// A part waits for all arrivals (at most arrive_spins polls), then claims
// its own slice; the last part to arrive waits (bounded) for the other
// parts' claims and takes every slice still unclaimed, so a part whose wait
// ran out loses nothing and every slice is summed by exactly one part.  Returns the bitmask of
// slices this part sums (0: none).
__device__ __forceinline__ int split_handoff_shared(int* w, int parts, int part, int xcd, int arrive_spins) {
  const int xcc = __builtin_amdgcn_s_getreg((3 << 11) | 20) & 15;  // HW_REG_XCC_ID[3:0]
  const bool off = xcc != xcd;
  if (off) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __builtin_amdgcn_s_waitcnt(0);
  }
  const int inc = off ? 0x11 : 0x01;
  int v = __hip_atomic_fetch_add(&w[0], inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + inc;
  const bool last = (v & 15) == parts;
  bool seen = last;
#pragma nounroll
  for (int it = 0; !seen && it < arrive_spins; ++it) {
    __builtin_amdgcn_s_sleep(1);
    v = __hip_atomic_load(&w[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    seen = (v & 15) == parts;
  }
  int mine = 0;
  if (seen) {
    if (((v >> 4) & 15) != 0 || off) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    const int full = (1 << parts) - 1;
    if (!last) {
      const int old = __hip_atomic_fetch_or(&w[1], 1 << part, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      mine = ((old >> part) & 1) ? 0 : 1 << part;
    } else {
#pragma nounroll
      for (int it = 0; it < kSplitClaimSpins; ++it) {
        if ((__hip_atomic_load(&w[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) | (1 << part)) == full) break;
        __builtin_amdgcn_s_sleep(1);
      }
      const int old = __hip_atomic_fetch_or(&w[1], full, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      mine = full & ~old;
    }
  }
  // Every access above must have returned its value before this increment
  // issues: a claim landing after the last part cleared w[1] would leave a
  // stale bit for the next launch.  The w[2] increment has no data
  // dependence on those accesses, so the order is enforced here: a compiler
  // fence keeps the atomics in program order and the wait drains them.
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  if (__hip_atomic_fetch_add(&w[2], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == parts - 1) {
    __hip_atomic_store(&w[0], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&w[1], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&w[2], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  return mine;
}

template <typename T> struct Mfma16;
template <> struct Mfma16<BF16> {
  __device__ __forceinline__ static f32x4 run(u32x4 x, u32x4 y, f32x4 acc) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, x),
                                                   __builtin_bit_cast(bf16x8, y), acc, 0, 0, 0);
  }
};
template <> struct Mfma16<F16> {
  __device__ __forceinline__ static f32x4 run(u32x4 x, u32x4 y, f32x4 acc) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, x),
                                                  __builtin_bit_cast(f16x8, y), acc, 0, 0, 0);
  }
};

// Byte offset of (row, 16-byte chunk) inside a swizzled 128-byte-row tile.
__device__ __forceinline__ int swz(int row, int chunk) {
  return (row << 7) + (((chunk ^ (row & 7))) << 4);
}

// Store four fp32 results (already through the epilogue) to C[m][n..n+3].
template <typename TOut> struct Store4 {  // 16-bit outputs
  __device__ __forceinline__ static void run(uint16_t* crow, int n, int N, bool vec_ok,
                                             const float v[4]) {
    if (vec_ok && n + 3 < N) {
      *reinterpret_cast<u32x2*>(crow + n) = u32x2{pack2<TOut>(v[0], v[1]), pack2<TOut>(v[2], v[3])};
    } else {
      uint16_t h[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) h[q] = Elem<TOut>::from_f32(v[q]);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (n + q < N) crow[n + q] = h[q];
    }
  }
};
template <> struct Store4<float> {
  __device__ __forceinline__ static void run(float* crow, int n, int N, bool vec_ok,
                                             const float v[4]) {
    if (vec_ok && n + 3 < N) {
      f32x4 o = {v[0], v[1], v[2], v[3]};
      *reinterpret_cast<f32x4*>(crow + n) = o;
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (n + q < N) crow[n + q] = v[q];
    }
  }
};

// Bias values for columns n..n+3 (bias dtype = input dtype TIn), fp32.
template <typename TIn>
__device__ __forceinline__ void load_bias4(const void* bias, int n, int N, float b[4]) {
  const uint16_t* bp = static_cast<const uint16_t*>(bias);
#pragma unroll
  for (int q = 0; q < 4; ++q) b[q] = (n + q < N) ? Elem<TIn>::to_f32(bp[n + q]) : 0.0f;
}

// Residual values R[m][n..n+3] (dtype = output dtype TOut) as fp32, zeros
// past N; `vec`: 8-byte (16-bit) / 16-byte (fp32) aligned rows.
template <typename TOut> struct Res4 {  // 16-bit outputs
  __device__ __forceinline__ static void load(const void* R, int64_t row_off, int n, int N, bool vec,
                                              float r[4]) {
    const uint16_t* rrow = static_cast<const uint16_t*>(R) + row_off;
    if (vec && n + 3 < N) {
      const u32x2 w = *reinterpret_cast<const u32x2*>(rrow + n);
#pragma unroll
      for (int q = 0; q < 4; ++q) r[q] = Elem<TOut>::to_f32(static_cast<uint16_t>(w[q >> 1] >> ((q & 1) * 16)));
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) r[q] = (n + q < N) ? Elem<TOut>::to_f32(rrow[n + q]) : 0.0f;
    }
  }
};
template <> struct Res4<float> {
  __device__ __forceinline__ static void load(const void* R, int64_t row_off, int n, int N, bool vec,
                                              float r[4]) {
    const float* rrow = static_cast<const float*>(R) + row_off;
    if (vec && n + 3 < N) {
      const f32x4 w = *reinterpret_cast<const f32x4*>(rrow + n);
#pragma unroll
      for (int q = 0; q < 4; ++q) r[q] = w[q];
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) r[q] = (n + q < N) ? rrow[n + q] : 0.0f;
    }
  }
};
// Whether Res4 may use vector loads on R (rows aligned for 4 elements).
template <typename TOut>
__device__ __forceinline__ bool res_vec_ok(const void* R, int64_t ldr) {
  constexpr int E = sizeof(typename Elem<TOut>::storage);
  return ((ldr & 3) == 0) && ((reinterpret_cast<uintptr_t>(R) & (4 * E - 1)) == 0);
}

template <typename TIn, typename TOut, int BM, int BN, int WAVES_M, int WAVES_N, bool B_KMAJOR,
          bool VEC, bool A_KMAJOR = true>
__global__ __launch_bounds__(WAVES_M* WAVES_N * 64) void gemm16_kernel(GemmParams p) {
  constexpr int NT = WAVES_M * WAVES_N * 64;
  constexpr int BK = 64;
  constexpr int CH = BK / 8;  // 16-byte chunks per tile row
  constexpr int WM = BM / WAVES_M;
  constexpr int WN = BN / WAVES_N;
  constexpr int FM = WM / 16;
  constexpr int FN = WN / 16;
  constexpr int A_BYTES = BM * BK * 2;
  constexpr int B_BYTES = BN * BK * 2;
  constexpr int STAGE = A_BYTES + B_BYTES;
  static_assert(WM % 16 == 0 && WN % 16 == 0, "wave tile must be 16-aligned");
  static_assert((BM * CH) % NT == 0, "A tile loads must divide evenly");
  static_assert((BN * CH) % NT == 0, "B tile loads must divide evenly");
  constexpr int A_LD = BM * CH / NT;
  constexpr int B_LD = BN * CH / NT;

  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WAVES_N;
  const int wn = wave % WAVES_N;

  int tm, tn;
  {
    int pid = xcd_remap(blockIdx.x, gridDim.x);
    group_tile(pid, p.tiles_m, p.tiles_n, 8, tm, tn);
  }
  const int m0 = tm * BM;
  const int n0 = tn * BN;
  const int64_t b = blockIdx.y;
  const uint16_t* __restrict__ A = static_cast<const uint16_t*>(p.A) + b * p.sA;
  const uint16_t* __restrict__ B = static_cast<const uint16_t*>(p.B) + b * p.sB;
  const int M = p.M, N = p.N, K = p.K;
  const int64_t lda = p.lda, ldb = p.ldb;

  f32x4 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  u32x4 ra[A_LD];
  u32x4 rb[B_LD];

  // ---- global -> registers ------------------------------------------------
  auto load_tiles = [&](int k0) {
    if constexpr (!A_KMAJOR) {
      // A is K x M: thread -> (k = idx % BK, 8-wide m chunk = idx / BK).
#pragma unroll
      for (int i = 0; i < A_LD; ++i) {
        int idx = tid + i * NT;
        int k = idx % BK, mc = idx / BK;
        int gk = k0 + k, gm = m0 + mc * 8;
        if constexpr (VEC) {
          ra[i] = (gk < K && gm < M)
                      ? *reinterpret_cast<const u32x4*>(A + (int64_t)gk * lda + gm)
                      : u32x4{0u, 0u, 0u, 0u};
        } else {
          uint16_t e[8];
#pragma unroll
          for (int q = 0; q < 8; ++q)
            e[q] = (gk < K && gm + q < M) ? A[(int64_t)gk * lda + gm + q] : (uint16_t)0;
          ra[i] = u32x4{e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16),
                        e[4] | ((uint32_t)e[5] << 16), e[6] | ((uint32_t)e[7] << 16)};
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < A_LD; ++i) {
        int idx = tid + i * NT;
        int row = idx / CH, ch = idx % CH;
        int gm = m0 + row, gk = k0 + ch * 8;
        if constexpr (VEC) {
          const u32x4* pa = reinterpret_cast<const u32x4*>(A + (int64_t)gm * lda + gk);
          // The 256 x 64 tile serves N <= 64 (one tile column): every A row
          // panel is read exactly once, so it streams past the caches.
          if constexpr (BM == 256 && BN == 64)
            ra[i] = (gm < M && gk < K) ? __builtin_nontemporal_load(pa) : u32x4{0u, 0u, 0u, 0u};
          else
            ra[i] = (gm < M && gk < K) ? *pa : u32x4{0u, 0u, 0u, 0u};
        } else {
          uint16_t e[8];
#pragma unroll
          for (int q = 0; q < 8; ++q)
            e[q] = (gm < M && gk + q < K) ? A[(int64_t)gm * lda + gk + q] : (uint16_t)0;
          ra[i] = u32x4{e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16),
                        e[4] | ((uint32_t)e[5] << 16), e[6] | ((uint32_t)e[7] << 16)};
        }
      }
    }
    if constexpr (B_KMAJOR) {
#pragma unroll
      for (int i = 0; i < B_LD; ++i) {
        int idx = tid + i * NT;
        int row = idx / CH, ch = idx % CH;
        int gn = n0 + row, gk = k0 + ch * 8;
        if constexpr (VEC) {
          rb[i] = (gn < N && gk < K)
                      ? *reinterpret_cast<const u32x4*>(B + (int64_t)gn * ldb + gk)
                      : u32x4{0u, 0u, 0u, 0u};
        } else {
          uint16_t e[8];
#pragma unroll
          for (int q = 0; q < 8; ++q)
            e[q] = (gn < N && gk + q < K) ? B[(int64_t)gn * ldb + gk + q] : (uint16_t)0;
          rb[i] = u32x4{e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16),
                        e[4] | ((uint32_t)e[5] << 16), e[6] | ((uint32_t)e[7] << 16)};
        }
      }
    } else {
      // B is K x N: thread -> (k = idx % BK, 8-wide n chunk = idx / BK).
#pragma unroll
      for (int i = 0; i < B_LD; ++i) {
        int idx = tid + i * NT;
        int k = idx % BK, nc = idx / BK;
        int gk = k0 + k, gn = n0 + nc * 8;
        if constexpr (VEC) {
          rb[i] = (gk < K && gn < N)
                      ? *reinterpret_cast<const u32x4*>(B + (int64_t)gk * ldb + gn)
                      : u32x4{0u, 0u, 0u, 0u};
        } else {
          uint16_t e[8];
#pragma unroll
          for (int q = 0; q < 8; ++q)
            e[q] = (gk < K && gn + q < N) ? B[(int64_t)gk * ldb + gn + q] : (uint16_t)0;
          rb[i] = u32x4{e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16),
                        e[4] | ((uint32_t)e[5] << 16), e[6] | ((uint32_t)e[7] << 16)};
        }
      }
    }
  };

  // ---- registers -> LDS stage ----------------------------------------------
  auto store_tiles = [&](int stage) {
    uint8_t* As = smem + stage * STAGE;
    uint8_t* Bs = As + A_BYTES;
    if constexpr (A_KMAJOR) {
#pragma unroll
      for (int i = 0; i < A_LD; ++i) {
        int idx = tid + i * NT;
        int row = idx / CH, ch = idx % CH;
        *reinterpret_cast<u32x4*>(As + swz(row, ch)) = ra[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < A_LD; ++i) {
        int idx = tid + i * NT;
        int k = idx % BK, mc = idx / BK;
        uint32_t w[4] = {ra[i][0], ra[i][1], ra[i][2], ra[i][3]};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          int m = mc * 8 + e;
          uint16_t v = static_cast<uint16_t>(w[e >> 1] >> ((e & 1) * 16));
          *reinterpret_cast<uint16_t*>(As + swz(m, k >> 3) + ((k & 7) << 1)) = v;
        }
      }
    }
    if constexpr (B_KMAJOR) {
#pragma unroll
      for (int i = 0; i < B_LD; ++i) {
        int idx = tid + i * NT;
        int row = idx / CH, ch = idx % CH;
        *reinterpret_cast<u32x4*>(Bs + swz(row, ch)) = rb[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < B_LD; ++i) {
        int idx = tid + i * NT;
        int k = idx % BK, nc = idx / BK;
        uint32_t w[4] = {rb[i][0], rb[i][1], rb[i][2], rb[i][3]};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          int n = nc * 8 + e;
          uint16_t v = static_cast<uint16_t>(w[e >> 1] >> ((e & 1) * 16));
          *reinterpret_cast<uint16_t*>(Bs + swz(n, k >> 3) + ((k & 7) << 1)) = v;
        }
      }
    }
  };

  // ---- LDS -> MFMA ---------------------------------------------------------
  auto compute = [&](int stage) {
    const uint8_t* As = smem + stage * STAGE;
    const uint8_t* Bs = As + A_BYTES;
#pragma unroll
    for (int s = 0; s < BK / 32; ++s) {
      const int ch = s * 4 + (lane >> 4);
      u32x4 ya[FM], xb[FN];
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        int row = wm * WM + j * 16 + (lane & 15);
        ya[j] = *reinterpret_cast<const u32x4*>(As + swz(row, ch));
      }
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        int row = wn * WN + i * 16 + (lane & 15);
        xb[i] = *reinterpret_cast<const u32x4*>(Bs + swz(row, ch));
      }
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = Mfma16<TIn>::run(xb[i], ya[j], acc[i][j]);
    }
  };

  const int KT = (K + BK - 1) / BK;
  if (KT > 0) {
    load_tiles(0);
    store_tiles(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
      const bool more = kt + 1 < KT;
      if (more) load_tiles((kt + 1) * BK);
      compute(kt & 1);
      if (more) store_tiles((kt + 1) & 1);
      __syncthreads();
    }
  }

  // ---- epilogue ------------------------------------------------------------
  typedef typename Elem<TOut>::storage OutS;
  OutS* C = static_cast<OutS*>(p.C) + b * p.sC;
  const bool has_bias = epi_has_bias(p.epi);
  const int act = epi_act(p.epi);
  const float alpha = p.alpha;
  const bool vec_ok = ((p.ldc & 3) == 0) && ((reinterpret_cast<uintptr_t>(C) & 15) == 0);
  const void* R = p.res != nullptr ? static_cast<const OutS*>(p.res) + b * p.sR : nullptr;
  const bool rvec = R != nullptr && res_vec_ok<TOut>(R, p.ldr);
  with_act(act, [&](auto act_c) {
    constexpr int ACT = decltype(act_c)::value;
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      const int n = n0 + wn * WN + i * 16 + 4 * (lane >> 4);
      float bv[4] = {0.f, 0.f, 0.f, 0.f};
      if (has_bias) load_bias4<TIn>(p.bias, n, N, bv);
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const int m = m0 + wm * WM + j * 16 + (lane & 15);
        if (m < M && n < N) {
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] = act_t<ACT>(acc[i][j][q] * alpha + bv[q]);
          if (R != nullptr) {
            float r[4];
            Res4<TOut>::load(R, (int64_t)m * p.ldr, n, N, rvec, r);
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] += r[q];
          }
          Store4<TOut>::run(C + (int64_t)m * p.ldc, n, N, vec_ok, v);
        }
      }
    }
  });
}

}  // namespace sf
