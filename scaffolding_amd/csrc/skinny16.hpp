// skinny16.hpp — bandwidth-bound 16-bit GEMM for M <= 16 ("decode"
// shapes): C[M,N] = epi(alpha * x[M,K] . W[N,K]^T (+ bias)).
//
// At M <= 16 the weight W (N x K) is the only large operand and is read
// exactly once, so the kernel is an HBM stream:
//   * a workgroup owns NB consecutive 16-row blocks of W (16*NB output
//     columns) and KSPLIT waves; wave w walks its 1/KSPLIT share of K;
//   * each step, a lane loads one 16-byte chunk (8 k-values) of W per row
//     block and the matching chunk of x, and one v_mfma_f32_16x16x32 per
//     row block folds 32 k of a 16(n) x 16(m) block: X = W rows, Y = x^T.
//     The MFMA is ~10x faster than the stream, so padding M up to 16 rows
//     costs nothing while keeping VALU work off the critical path;
//   * loads are issued UNROLL steps ahead of their MFMAs so each wave keeps
//     UNROLL*(NB+1) 1 KB requests in flight;
//   * partial 16x16 blocks of the KSPLIT waves are summed through LDS and
//     wave 0 applies alpha, bias, activation, and stores: lane l holds
//     C[m = l%16][n0 + 4*(l/16) + 0..3].
// Requires K % 8 == 0, 16-byte aligned rows (lda, ldb multiples of 8).
#pragma once

#include "gemm16.hpp"

namespace sf {

template <typename TIn, typename TOut, int KSPLIT, int NB, int UNROLL>
__global__ __launch_bounds__(KSPLIT * 64) void skinny16_kernel(GemmParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t b = blockIdx.y;
  const int n0 = blockIdx.x * (16 * NB);
  const uint16_t* __restrict__ X = static_cast<const uint16_t*>(p.A) + b * p.sA;
  const uint16_t* __restrict__ W = static_cast<const uint16_t*>(p.B) + b * p.sB;
  const int M = p.M, N = p.N, K = p.K;

  const int ksteps = (K + 31) / 32;
  const int per = (ksteps + KSPLIT - 1) / KSPLIT;
  const int s_begin = wave * per;
  int s_end = s_begin + per;
  if (s_end > ksteps) s_end = ksteps;

  const int r = lane & 15;         // row inside a 16-block (n for W, m for x)
  const int kc = (lane >> 4) * 8;  // k offset of this lane's chunk in a step
  const bool xrow_ok = r < M;
  const uint16_t* xrow = X + (int64_t)(xrow_ok ? r : 0) * p.lda + kc;
  const uint16_t* wrow[NB];
  bool wrow_ok[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    int n = n0 + j * 16 + r;
    wrow_ok[j] = n < N;
    wrow[j] = W + (int64_t)(wrow_ok[j] ? n : 0) * p.ldb + kc;
  }

  f32x4 acc[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int s0 = s_begin; s0 < s_end; s0 += UNROLL) {
    u32x4 wv[UNROLL][NB];
    u32x4 xv[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int s = s0 + u;
      const int k = s * 32 + kc;
      const bool kin = (s < s_end) && (k < K);
#pragma unroll
      for (int j = 0; j < NB; ++j)
        wv[u][j] = (kin && wrow_ok[j])
                       ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[j] + s * 32))
                       : u32x4{0u, 0u, 0u, 0u};
      xv[u] = (kin && xrow_ok) ? *reinterpret_cast<const u32x4*>(xrow + s * 32)
                               : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
#pragma unroll
      for (int j = 0; j < NB; ++j) acc[j] = Mfma16<TIn>::run(wv[u][j], xv[u], acc[j]);
  }

  // Cross-wave reduction of the KSPLIT partial blocks.
  __shared__ f32x4 red[KSPLIT > 1 ? KSPLIT - 1 : 1][NB][64];
  if (KSPLIT > 1) {
    if (wave > 0) {
#pragma unroll
      for (int j = 0; j < NB; ++j) red[wave - 1][j][lane] = acc[j];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 0; w < KSPLIT - 1; ++w)
#pragma unroll
      for (int j = 0; j < NB; ++j) acc[j] += red[w][j][lane];
  }

  typedef typename Elem<TOut>::storage OutS;
  OutS* C = static_cast<OutS*>(p.C) + b * p.sC;
  const bool has_bias = epi_has_bias(p.epi);
  const int act = epi_act(p.epi);
  const bool vec_ok = ((p.ldc & 3) == 0) && ((reinterpret_cast<uintptr_t>(C) & 15) == 0);
  const int m = lane & 15;
  if (m >= M) return;
  with_act(act, [&](auto act_c) {
    constexpr int ACT = decltype(act_c)::value;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int n = n0 + j * 16 + 4 * (lane >> 4);
      if (n >= N) continue;
      float bv[4] = {0.f, 0.f, 0.f, 0.f};
      if (has_bias) load_bias4<TIn>(p.bias, n, N, bv);
      float v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = act_t<ACT>(acc[j][q] * p.alpha + bv[q]);
      Store4<TOut>::run(C + (int64_t)m * p.ldc, n, N, vec_ok, v);
    }
  });
}

}  // namespace sf
