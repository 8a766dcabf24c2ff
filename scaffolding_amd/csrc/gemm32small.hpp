// gemm32small.hpp — fp32 GEMM for outputs too small to fill the GPU with
// 64 x 64 tiles (a 64-row nn.Linear, a 64 x 512 projection):
//
//   C[b] = epi(alpha * A[b] . op(B[b]) (+ bias)) (+ R[b])     row-major, fp32
//
// A is M x K (K-contiguous); B is N x K (K-contiguous) or K x N
// (N-contiguous).  K % 4 == 0, rows 16-byte aligned.
//
// Why.  Such a GEMM is latency-bound: with 64 x 64 tiles it runs a few
// dozen workgroups, each walking a long k range slice after slice, and
// splitting k across workgroups adds a round trip through memory for the
// partial sums.  Here a workgroup computes a 16 x 16 FS block of C with KW
// waves, wave w taking the w-th KW-th of the k range, so the grid holds
// (M / 16) (N / 16 FS) KW waves, each short.  The operands go straight from
// global memory into the MFMA registers (no LDS staging: a wave shares no
// operand with another), four 16-k steps in flight per wave; the KW partial
// blocks are summed through LDS in wave order (a fixed order, so results do
// not depend on timing).
//
// MFMA roles as gemm32.hpp: X from B, Y from A; over the four MFMAs of 16 k
// lane group g = l / 16 supplies k = 4 g + s at step s, so a K-contiguous
// operand is one float4 per lane per 16 k.  Lane l ends with C[m0 + l % 16]
// [n0 + 16 i + 4 g + q] in acc[i][q].
#pragma once

#include "gemm32.hpp"

namespace sf {

template <int FS, bool B_KMAJOR, int KW>
__global__ __launch_bounds__(KW * 64) void gemm32small_kernel(GemmParams p) {
  constexpr int U = 4;  // 16-k steps per batch of loads
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, r = lane & 15;

  const int tm = (int)(blockIdx.x / (unsigned)p.tiles_n), tn = (int)(blockIdx.x % (unsigned)p.tiles_n);
  const int m0 = tm * 16, n0 = tn * 16 * FS;
  const int64_t b = blockIdx.y;
  const float* A = static_cast<const float*>(p.A) + b * p.sA;
  const float* B = static_cast<const float*>(p.B) + b * p.sB;
  const int M = p.M, N = p.N, K = p.K;

  // Rows past M (N) are clamped to the last one: their products reach no
  // stored output.
  const float* arow = A + (int64_t)(m0 + r < M ? m0 + r : M - 1) * p.lda;
  const float* bptr[FS];
#pragma unroll
  for (int i = 0; i < FS; ++i) {
    const int n = n0 + 16 * i + r < N ? n0 + 16 * i + r : N - 1;
    bptr[i] = B_KMAJOR ? B + (int64_t)n * p.ldb : B + n;
  }

  const int S = (K + 15) / 16;
  const int s0 = wave * S / KW, s1 = (wave + 1) * S / KW;

  // One batch: U steps from step st; steps past s1 or k past K load zeros
  // (K % 4 == 0, so a lane group's 4 k are all in range or all out).
  auto load = [&](int st, f32x4 (&a)[U], f32x4 (&x)[U][FS]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = (st + u) * 16 + 4 * g;
      const bool ok = st + u < s1 && k < K;
      a[u] = ok ? *reinterpret_cast<const f32x4*>(arow + k) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < FS; ++i) {
        if constexpr (B_KMAJOR) {
          x[u][i] = ok ? *reinterpret_cast<const f32x4*>(bptr[i] + k) : f32x4{0.f, 0.f, 0.f, 0.f};
        } else {
#pragma unroll
          for (int s = 0; s < 4; ++s) x[u][i][s] = ok ? bptr[i][(int64_t)(k + s) * p.ldb] : 0.f;
        }
      }
    }
  };

  f32x4 acc[FS];
#pragma unroll
  for (int i = 0; i < FS; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (s1 > s0) {
    f32x4 a[U], x[U][FS], an[U], xn[U][FS];
    load(s0, a, x);
    for (int st = s0; st < s1; st += U) {
      const bool more = st + U < s1;  // wave-uniform
      if (more) load(st + U, an, xn);
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int i = 0; i < FS; ++i)
            acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[u][i][s], a[u][s], acc[i], 0, 0, 0);
      if (more) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          a[u] = an[u];
#pragma unroll
          for (int i = 0; i < FS; ++i) x[u][i] = xn[u][i];
        }
      }
    }
  }

  // Sum the KW partial blocks in wave order; fragment i is summed and
  // stored by wave i % KW.
  __shared__ f32x4 red[KW][FS][64];
#pragma unroll
  for (int i = 0; i < FS; ++i) red[wave][i][lane] = acc[i];
  __syncthreads();

  float* C = static_cast<float*>(p.C) + b * p.sC;
  const bool has_bias = epi_has_bias(p.epi);
  const int act = epi_act(p.epi);
  const float alpha = p.alpha;
  const bool vec_ok = ((p.ldc & 3) == 0) && ((reinterpret_cast<uintptr_t>(C) & 15) == 0);
  const float* bias = static_cast<const float*>(p.bias);
  const void* R = p.res != nullptr ? static_cast<const float*>(p.res) + b * p.sR : nullptr;
  const bool rvec = R != nullptr && res_vec_ok<float>(R, p.ldr);
  const int m = m0 + r;
  with_act(act, [&](auto act_c) {
    constexpr int ACT = decltype(act_c)::value;
#pragma unroll
    for (int i = 0; i < FS; ++i) {
      if (i % KW != wave) continue;  // wave-uniform
      f32x4 sum = red[0][i][lane];
#pragma unroll
      for (int w = 1; w < KW; ++w) sum += red[w][i][lane];
      const int n = n0 + 16 * i + 4 * g;
      if (m < M && n < N) {
        float bv[4] = {0.f, 0.f, 0.f, 0.f};
        if (has_bias) {
#pragma unroll
          for (int q = 0; q < 4; ++q) bv[q] = (n + q < N) ? bias[n + q] : 0.f;
        }
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = act_t<ACT>(sum[q] * alpha + bv[q]);
        if (R != nullptr) {
          float rr[4];
          Res4<float>::load(R, (int64_t)m * p.ldr, n, N, rvec, rr);
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] += rr[q];
        }
        Store4<float>::run(C + (int64_t)m * p.ldc, n, N, vec_ok, v);
      }
    }
  });
}

}  // namespace sf
