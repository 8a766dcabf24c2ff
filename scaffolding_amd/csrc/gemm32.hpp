// gemm32.hpp — fp32 GEMM on gfx950's fp32 MFMA (v_mfma_f32_16x16x4_f32),
// true fp32 products and accumulation (no reduced-precision shortcut).
//
//   C[b] = epi(alpha * A[b] . op(B[b]) (+ bias))      row-major, fp32
//
// Same decomposition and operand roles as gemm16.hpp (X from the B tile,
// Y from the A tile, lane l ends with C[m = l%16][n = 4*(l/16) + 0..3]),
// with BK = 32 fp32 per slice.
//
// k assignment.  One 16x16x4 MFMA consumes 4 k: lane group g = l/16
// supplies one k.  Over four consecutive MFMAs (16 k) this kernel gives
// group g the k values 4g, 4g+1, 4g+2, 4g+3 (step j uses 4g+j).  The sum
// over k is order-free, and A and B use the same assignment, so the
// product is exact; it lets a K-contiguous tile be read as one float4 per
// lane for four MFMAs.
//
// LDS layout (floats):
//   A            [BM][BK + 4]   K-contiguous; a float4 read by 16 lanes on
//                               16 rows hits 16 distinct 16-byte bank groups
//                               (row pitch 144 B = 9 slots, 9 odd).
//   B, K-major   [BN][BK + 4]   as A.
//   B, N-major   [BK][BN + 4]   N-contiguous; the X operand is a scalar per
//                               lane per step (16 consecutive n per group,
//                               groups 4 rows = 16 banks apart).
//   A, M-major   [BK][BM + 4]   A stored K x M (the product uses A^T); the
//                               Y operand is read like the N-major B.
#pragma once

#include "gemm16.hpp"

namespace sf {

// Split-K hand-off of an fp32 tile held as NF fragments per thread (flat
// f32x4 array, fragment f of thread tid parked at ((f * NT) + tid) * 4 of
// the part's slab): park this part's fragments, count the arrival, and in
// the last part to arrive sum every part's fragments, this one's included,
// in part order (the same additions whichever part is last).  Returns false
// in every other part, which then has nothing left to do.  At most
// kMaxSplit32 parts: each thread keeps all parts' loads of four fragments
// in flight at once, so the sum costs one round trip per four fragments.
template <int NF, int NT>
__device__ __forceinline__ bool split32_handoff(f32x4* acc, const GemmParams& p, int tile_id, int part, int tid) {
  static_assert(NF % 4 == 0, "partials move four fragments at a time");
  float* mine = p.ws + (size_t)(tile_id * p.split + part) * (NF * NT * 4);
#pragma unroll
  for (int f = 0; f < NF; ++f) *reinterpret_cast<f32x4*>(mine + (size_t)(f * NT + tid) * 4) = acc[f];
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  __shared__ int arrived;
  if (tid == 0) arrived = split_arrive(&p.counters[tile_id], p.split);
  __syncthreads();
  if (arrived != p.split - 1) return false;  // workgroup-uniform
  const float* all = p.ws + (size_t)tile_id * p.split * (NF * NT * 4);
#pragma unroll
  for (int c = 0; c < NF / 4; ++c) {
    f32x4 v[kMaxSplit32][4];
#pragma unroll
    for (int q = 0; q < kMaxSplit32; ++q) {
      if (q < p.split) {
        const float* src = all + ((size_t)q * NF + 4 * c) * NT * 4 + (size_t)tid * 4;
#pragma unroll
        for (int u = 0; u < 4; ++u) v[q][u] = *reinterpret_cast<const f32x4*>(src + (size_t)u * NT * 4);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[4 * c + u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < kMaxSplit32; ++q) {
      if (q < p.split) {
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[4 * c + u] += v[q][u];
      }
    }
  }
  if (tid == 0) __hip_atomic_store(&p.counters[tile_id], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

template <int BM, int BN, int WAVES_M, int WAVES_N, bool B_KMAJOR, bool VEC, bool A_KMAJOR = true>
__global__ __launch_bounds__(WAVES_M* WAVES_N * 64) void gemm32_kernel(GemmParams p) {
  constexpr int NT = WAVES_M * WAVES_N * 64;
  constexpr int BK = 32;
  constexpr int CH = BK / 4;  // float4 chunks per K-contiguous row
  constexpr int AP = BK + 4;  // A / K-major-B row pitch (floats)
  constexpr int BP = BN + 4;  // N-major-B row pitch (floats)
  constexpr int MP = BM + 4;  // M-major-A row pitch (floats)
  constexpr int WM = BM / WAVES_M;
  constexpr int WN = BN / WAVES_N;
  constexpr int FM = WM / 16;
  constexpr int FN = WN / 16;
  constexpr int A_FLOATS = A_KMAJOR ? BM * AP : BK * MP;
  constexpr int B_FLOATS = B_KMAJOR ? BN * AP : BK * BP;
  constexpr int STAGE = A_FLOATS + B_FLOATS;
  static_assert((BM * CH) % NT == 0 && (BN * CH) % NT == 0, "tile loads must divide evenly");
  constexpr int A_LD = BM * CH / NT;
  constexpr int B_LD = BN * CH / NT;  // BK*BN/4 == BN*CH as well

  __shared__ __attribute__((aligned(16))) float smem[2 * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WAVES_N;
  const int wn = wave % WAVES_N;
  const int g = lane >> 4;

  // Split-K (p.split > 0, batch 1): workgroup x is part x % split of tile
  // x / split; part q covers k-slices [KT q / split, KT (q + 1) / split).
  const int part = p.split > 0 ? (int)(blockIdx.x % (unsigned)p.split) : -1;
  const int tile_id = p.split > 0 ? (int)(blockIdx.x / (unsigned)p.split) : 0;
  int tm, tn;
  {
    int pid = p.split > 0 ? tile_id : xcd_remap(blockIdx.x, gridDim.x);
    group_tile(pid, p.tiles_m, p.tiles_n, 8, tm, tn);
  }
  const int m0 = tm * BM;
  const int n0 = tn * BN;
  const int64_t b = blockIdx.y;
  const float* __restrict__ A = static_cast<const float*>(p.A) + b * p.sA;
  const float* __restrict__ B = static_cast<const float*>(p.B) + b * p.sB;
  const int M = p.M, N = p.N, K = p.K;
  const int64_t lda = p.lda, ldb = p.ldb;

  f32x4 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  f32x4 ra[A_LD], rb[B_LD];

  auto load4 = [&](const float* base, int64_t ld, int r, int c, int rmax, int cmax) -> f32x4 {
    if constexpr (VEC) {
      return (r < rmax && c < cmax) ? *reinterpret_cast<const f32x4*>(base + (int64_t)r * ld + c)
                                    : f32x4{0.f, 0.f, 0.f, 0.f};
    } else {
      f32x4 v;
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = (r < rmax && c + q < cmax) ? base[(int64_t)r * ld + c + q] : 0.f;
      return v;
    }
  };

  auto load_tiles = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      int idx = tid + i * NT;
      if constexpr (A_KMAJOR) {
        ra[i] = load4(A, lda, m0 + idx / CH, k0 + (idx % CH) * 4, M, K);
      } else {
        constexpr int MC = BM / 4;
        ra[i] = load4(A, lda, k0 + idx / MC, m0 + (idx % MC) * 4, K, M);
      }
    }
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      int idx = tid + i * NT;
      if constexpr (B_KMAJOR) {
        rb[i] = load4(B, ldb, n0 + idx / CH, k0 + (idx % CH) * 4, N, K);
      } else {
        constexpr int NC = BN / 4;
        rb[i] = load4(B, ldb, k0 + idx / NC, n0 + (idx % NC) * 4, K, N);
      }
    }
  };

  auto store_tiles = [&](int stage) {
    float* As = smem + stage * STAGE;
    float* Bs = As + A_FLOATS;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      int idx = tid + i * NT;
      if constexpr (A_KMAJOR) {
        *reinterpret_cast<f32x4*>(As + (idx / CH) * AP + (idx % CH) * 4) = ra[i];
      } else {
        constexpr int MC = BM / 4;
        *reinterpret_cast<f32x4*>(As + (idx / MC) * MP + (idx % MC) * 4) = ra[i];
      }
    }
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      int idx = tid + i * NT;
      if constexpr (B_KMAJOR) {
        *reinterpret_cast<f32x4*>(Bs + (idx / CH) * AP + (idx % CH) * 4) = rb[i];
      } else {
        constexpr int NC = BN / 4;
        *reinterpret_cast<f32x4*>(Bs + (idx / NC) * BP + (idx % NC) * 4) = rb[i];
      }
    }
  };

  auto compute = [&](int stage) {
    const float* As = smem + stage * STAGE;
    const float* Bs = As + A_FLOATS;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      // K-major tiles: one float4 per fragment covers the four steps.
      f32x4 ya4[FM], xb4[FN];
      if constexpr (A_KMAJOR) {
#pragma unroll
        for (int j = 0; j < FM; ++j) {
          int row = wm * WM + j * 16 + (lane & 15);
          ya4[j] = *reinterpret_cast<const f32x4*>(As + row * AP + kk * 16 + 4 * g);
        }
      }
      if constexpr (B_KMAJOR) {
#pragma unroll
        for (int i = 0; i < FN; ++i) {
          int row = wn * WN + i * 16 + (lane & 15);
          xb4[i] = *reinterpret_cast<const f32x4*>(Bs + row * AP + kk * 16 + 4 * g);
        }
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int k = kk * 16 + 4 * g + s;
        float ys[FM], xs[FN];
#pragma unroll
        for (int j = 0; j < FM; ++j)
          ys[j] = A_KMAJOR ? ya4[j][s] : As[k * MP + wm * WM + j * 16 + (lane & 15)];
#pragma unroll
        for (int i = 0; i < FN; ++i)
          xs[i] = B_KMAJOR ? xb4[i][s] : Bs[k * BP + wn * WN + i * 16 + (lane & 15)];
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
          for (int j = 0; j < FM; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(xs[i], ys[j], acc[i][j], 0, 0, 0);
      }
    }
  };

  const int KTall = (K + BK - 1) / BK;
  const int kt0 = part >= 0 ? KTall * part / p.split : 0;
  const int kt1 = part >= 0 ? KTall * (part + 1) / p.split : KTall;
  if (kt1 > kt0) {
    load_tiles(kt0 * BK);
    store_tiles(0);
    __syncthreads();
    for (int kt = kt0; kt < kt1; ++kt) {
      const bool more = kt + 1 < kt1;
      if (more) load_tiles((kt + 1) * BK);
      compute((kt - kt0) & 1);
      if (more) store_tiles((kt - kt0 + 1) & 1);
      __syncthreads();
    }
  }

  // ---- split-K: park the partial, the last part sums all of them in part
  // order (the same protocol as the 16-bit LDS-DMA kernel's split tail:
  // plain stores, the counter bumped by split_arrive, plain loads).
  if (part >= 0 && !split32_handoff<FN * FM, NT>(&acc[0][0], p, tile_id, part, tid)) return;

  float* C = static_cast<float*>(p.C) + b * p.sC;
  const bool has_bias = epi_has_bias(p.epi);
  const int act = epi_act(p.epi);
  const float alpha = p.alpha;
  const bool vec_ok = ((p.ldc & 3) == 0) && ((reinterpret_cast<uintptr_t>(C) & 15) == 0);
  const float* bias = static_cast<const float*>(p.bias);
  const void* R = p.res != nullptr ? static_cast<const float*>(p.res) + b * p.sR : nullptr;
  const bool rvec = R != nullptr && res_vec_ok<float>(R, p.ldr);
  with_act(act, [&](auto act_c) {
    constexpr int ACT = decltype(act_c)::value;
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      const int n = n0 + wn * WN + i * 16 + 4 * g;
      float bv[4] = {0.f, 0.f, 0.f, 0.f};
      if (has_bias) {
#pragma unroll
        for (int q = 0; q < 4; ++q) bv[q] = (n + q < N) ? bias[n + q] : 0.f;
      }
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const int m = m0 + wm * WM + j * 16 + (lane & 15);
        if (m < M && n < N) {
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] = act_t<ACT>(acc[i][j][q] * alpha + bv[q]);
          if (R != nullptr) {
            float r[4];
            Res4<float>::load(R, (int64_t)m * p.ldr, n, N, rvec, r);
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] += r[q];
          }
          Store4<float>::run(C + (int64_t)m * p.ldc, n, N, vec_ok, v);
        }
      }
    }
  });
}

}  // namespace sf
