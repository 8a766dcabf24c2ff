// gemm32dma.hpp — fp32 GEMM on fp32 MFMA (v_mfma_f32_16x16x4_f32) with
// direct-to-LDS loads into a multi-stage ring:
//
//   C[b] = epi(alpha * A[b] . op(B[b]) (+ bias)) (+ R[b])     row-major, fp32
//
// A is M x K (K-contiguous); B is N x K (K-contiguous, "NT": x . W^T) or
// K x N (N-contiguous, "NN": A . B).  K % 32 == 0, rows 16-byte aligned.
//
// Why.  An fp32 MFMA slice (32 k) of a 64 x 64 tile is 32 MFMAs per wave,
// about 1000 cycles, shorter than a global-load round trip under load; the
// register-staged kernel (gemm32.hpp) has one slice in flight and waits for
// every one.  Here buffer_load_dwordx4 ... lds moves each slice straight
// into LDS (no VGPRs, no ds_write) NSTG - 1 slices ahead of the one the
// MFMAs consume.
//
// Work decomposition: 256 threads, waves 2 x 2 of (BM/2) x (BN/2), MFMA X
// operand from B, Y from A; lane l ends with fragment rows 4 (l / 16) + q of
// column l % 16 (C[m][n] with m from the column, n from the row).  Over the
// four MFMAs of 16 k, lane group g = l / 16 supplies k = 4 g + s at step s
// (A and B alike, so the sum is exact).
//
// LDS layouts (no padding, XOR swizzles instead, since a direct load writes
// lane l's 16 bytes at the instruction's base + 16 l):
//   K-contiguous operand: line r = row r's 32 floats (128 bytes), 16-byte
//     chunk c at slot c ^ (r & 7).  A fragment read (16 lanes on 16 rows,
//     one chunk) covers 8 distinct slots per 8 rows: conflict-free float4
//     reads, which hold k = 4 g .. 4 g + 3, one per step.  A direct load
//     fills 8 rows (lane l: row l >> 3, slot l & 7, chunk (l & 7) ^ (l >> 3)).
//     Fragment i of a wave holds rows (columns of C) wn WN + 16 i + r.
//   N-contiguous B: k-row k = BN floats.  Fragment i of a wave's X operand
//     holds columns n = wn WN + FN r + i (r = fragment row), so at step s
//     lane l reads the FN consecutive floats B[k][wn WN + FN (l & 15) + i]
//     of k-row k = 4 g + s in one ds_read (b128 at FN = 4, b64 at FN = 2)
//     that feeds all FN fragments, and the epilogue stores 4 FN consecutive
//     columns per lane.  At FN = 2 the k-rows with (k >> 2) odd hold their
//     16-byte chunks c at slot c ^ 8 (row halves swapped), so lane groups 0
//     and 1 of a read use different banks.  A direct load fills 1024 / (4 BN)
//     k-rows.
// The ring has NSTG slots of one slice each; slice t sits in slot t % NSTG.
// Per slice each wave waits for its own loads of slice t (the later ones
// stay in flight), the workgroup barrier makes everyone's complete, then the
// slot of slice t - 1 (read by every wave before the barrier) is refilled
// with slice t + NSTG - 1.  Fill number u past the last slice re-loads the
// last slice into slot u % NSTG, which no slice still to be read occupies
// (u - NSTG + 1 > last), so every wait counts the same number of loads.
//
// Split-K (p.split > 0, batch 1): split32_handoff (parts of a tile park
// partials, the last arriver sums them in part order).
#pragma once

#include "gemm32.hpp"
#include "gemm16nt_pp.hpp"

namespace sf {

// ds_read_b64 as inline assembly (see ds_read16 for why and how it is
// ordered).  The result is a 64-bit integer: with a two-element vector
// result this compiler reads element 1 from element 0's register.
template <int OFF>
__device__ __forceinline__ uint64_t ds_read8(uint32_t addr) {
  uint64_t v;
  asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}

// Waits for this wave's LDS reads.  The reads are inline assembly, whose
// results the compiler takes as ready at once, so scheduling barriers keep
// their consumers (MFMAs, which touch no memory and would otherwise move
// freely) behind the wait.
__device__ __forceinline__ void lds_wait_all() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
  __builtin_amdgcn_sched_barrier(0);
}

template <int BM, int BN, bool B_KMAJOR, int NSTG, int KG = 1>
__global__ __launch_bounds__(256 * KG) void gemm32dma_kernel(GemmParams p) {
  constexpr int NT = 256;  // threads of one k-group
  constexpr int BK = 32;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int FM = WM / 16, FN = WN / 16;
  constexpr int A_BYTES = BM * BK * 4;
  constexpr int B_BYTES = BN * BK * 4;
  constexpr int SLOT = A_BYTES + B_BYTES;
  constexpr int LA = A_BYTES / 1024 / 4;  // direct loads per wave per slice, A
  constexpr int LB = B_BYTES / 1024 / 4;  // and B
  constexpr int L = LA + LB;
  static_assert(LA >= 1 && LB >= 1, "each wave loads part of both operands");
  static_assert(B_KMAJOR || FN == 2 || FN == 4, "N-contiguous B reads 2 or 4 columns per lane");
  static_assert(NSTG >= 2 && L * (NSTG - 2) < 64, "vmcnt holds at most 63");
  static_assert(KG == 1 || KG == 2, "one or two k-groups");
  static_assert(KG == 1 || FN * FM * 4 * 1024 <= NSTG * SLOT, "group 1's partial block fits in its ring");
  __shared__ __attribute__((aligned(1024))) uint8_t ring_all[KG * NSTG * SLOT];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int kg = KG == 1 ? 0 : __builtin_amdgcn_readfirstlane(tid >> 8);
  const int wave = __builtin_amdgcn_readfirstlane((tid >> 6) & 3);  // within the k-group
  const int wm = wave >> 1, wn = wave & 1;
  const int g = lane >> 4;
  uint8_t* const ring = ring_all + kg * (NSTG * SLOT);

  // Two k-groups never split across workgroups (the host passes split 0).
  const int part = (KG == 1 && p.split > 0) ? (int)(blockIdx.x % (unsigned)p.split) : -1;
  const int tile_id = p.split > 0 ? (int)(blockIdx.x / (unsigned)p.split) : 0;
  int tm, tn;
  group_tile(p.split > 0 ? tile_id : xcd_remap(blockIdx.x, gridDim.x), p.tiles_m, p.tiles_n, 8, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int64_t b = blockIdx.y;
  const float* A = static_cast<const float*>(p.A) + b * p.sA;
  const float* B = static_cast<const float*>(p.B) + b * p.sB;
  const int M = p.M, N = p.N, K = p.K;

  // This k-group's slices [kt0, kt1): with two groups the host keeps the
  // slice count even, so both run the same number of iterations (and
  // workgroup barriers).
  const int KTall = K / BK;
  const int kt0 = part >= 0 ? KTall * part / p.split : kg * (KTall / KG);
  const int kt1 = part >= 0 ? KTall * (part + 1) / p.split : kt0 + KTall / KG;
  const int last = kt1 - 1;

  // Buffer resources over this batch entry's rows (the host keeps them
  // under 2^31 bytes).  Rows past M (N) are clamped to the last row (their
  // products reach no stored output); for an N-contiguous B, columns past N
  // read the next row or, past the buffer, zeros (likewise unstored).
  const __amdgpu_buffer_rsrc_t rA =
      __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, (int)((uint32_t)M * (uint32_t)p.lda * 4u), 0x00020000);
  const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc(
      (void*)B, (short)0, (int)((uint32_t)(B_KMAJOR ? N : K) * (uint32_t)p.ldb * 4u), 0x00020000);
  uint32_t voa[LA], vob[LB];
#pragma unroll
  for (int i = 0; i < LA; ++i) {
    const int r = (wave * LA + i) * 8 + (lane >> 3);
    const int gm = m0 + r < M ? m0 + r : M - 1;
    voa[i] = (uint32_t)gm * (uint32_t)p.lda * 4u + (uint32_t)(((lane & 7) ^ (r & 7)) * 16);
  }
#pragma unroll
  for (int i = 0; i < LB; ++i) {
    if constexpr (B_KMAJOR) {
      const int r = (wave * LB + i) * 8 + (lane >> 3);
      const int gn = n0 + r < N ? n0 + r : N - 1;
      vob[i] = (uint32_t)gn * (uint32_t)p.ldb * 4u + (uint32_t)(((lane & 7) ^ (r & 7)) * 16);
    } else {
      // k-rows of BN floats: RPL k-rows per load, lane l on k-row l / CPR,
      // slot l % CPR.
      constexpr int CPR = BN / 4;    // 16-byte chunks per k-row
      constexpr int RPL = 64 / CPR;  // k-rows per load
      const int kr = (wave * LB + i) * RPL + lane / CPR;
      const int slot = lane % CPR;
      const int chunk = FN == 2 ? slot ^ (8 * ((kr >> 2) & 1)) : slot;
      vob[i] = (uint32_t)kr * (uint32_t)p.ldb * 4u + (uint32_t)(n0 * 4 + chunk * 16);
    }
  }
  // Fill u: slice min(u, last) into slot u % NSTG (the k offset of a
  // K-contiguous operand goes in the scalar offset; an N-contiguous B moves
  // by 32 k-rows).
  // (The lane offsets come in as pointer arguments: a lambda that captures
  // an array whose length depends on the template parameters leaves the
  // kernel's host stub undefined with this compiler.)
  auto issue = [&](int u, const uint32_t* va, const uint32_t* vb) {
    const int s = u % NSTG;
    const int t = u < last ? u : last;
    uint8_t* sa = ring + s * SLOT;
    uint8_t* sb = sa + A_BYTES;
#pragma unroll
    for (int i = 0; i < LA; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lds_ptr_t)(sa + (wave * LA + i) * 1024), 16, va[i], t * BK * 4,
                                               0, 0);
#pragma unroll
    for (int i = 0; i < LB; ++i) {
      if constexpr (B_KMAJOR)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, (lds_ptr_t)(sb + (wave * LB + i) * 1024), 16, vb[i],
                                                 t * BK * 4, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, (lds_ptr_t)(sb + (wave * LB + i) * 1024), 16,
                                                 vb[i] + (uint32_t)(t * BK) * (uint32_t)p.ldb * 4u, 0, 0, 0);
    }
  };

  f32x4 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Per-lane fragment addresses inside a slot.  K-contiguous: row r, chunk
  // kk*4 + g at slot (kk*4 + g) ^ (r & 7), and r & 7 = lane & 7 for every
  // fragment.  N-contiguous B: k-row 4g (+ kk*16 + s), columns
  // wn*WN + FN (l & 15), row halves swapped at FN = 2 when g is odd
  // ((k >> 2) & 1 = g & 1).
  const uint32_t ring_l = lds_addr(ring);
  const uint32_t fa = (uint32_t)((wm * WM + (lane & 15)) * 128);
  const uint32_t fb = (uint32_t)((wn * WN + (lane & 15)) * 128);
  const int sw = lane & 7;
  const uint32_t xcol = (uint32_t)((wn * WN + FN * (lane & 15)) * 4);
  const uint32_t xrow = (uint32_t)(4 * g * BN * 4) + (FN == 2 ? (xcol ^ (uint32_t)(128 * (g & 1))) : xcol);

  // Fragments of one 16-k step pair (kk): Y from A, X from B by step s.
  struct Frags {
    f32x4 y[FM];
    float x[4][FN];
  };
  constexpr int NR = FM + (B_KMAJOR ? FN : 4);  // LDS reads per kk
  auto read = [&](uint32_t sa, uint32_t sb, int kk, Frags& f) {
    const uint32_t cs = (uint32_t)(((kk * 4 + g) ^ sw) << 4);
    static_for<FM>([&](auto j_c) {
      constexpr int J = decltype(j_c)::value;
      f.y[J] = __builtin_bit_cast(f32x4, ds_read16<J * 16 * 128>(sa + fa + cs));
    });
    if constexpr (B_KMAJOR) {
      static_for<FN>([&](auto i_c) {
        constexpr int I = decltype(i_c)::value;
        const f32x4 v = __builtin_bit_cast(f32x4, ds_read16<I * 16 * 128>(sb + fb + cs));
#pragma unroll
        for (int s = 0; s < 4; ++s) f.x[s][I] = v[s];
      });
    } else {
      // Step s: B[k = kk*16 + 4g + s][wn*WN + FN (l & 15) + i], all i.
      const uint32_t xa = sb + xrow + (uint32_t)(kk * 16 * BN * 4);
      static_for<4>([&](auto s_c) {
        constexpr int S = decltype(s_c)::value;
        if constexpr (FN == 4) {
          const f32x4 v = __builtin_bit_cast(f32x4, ds_read16<S * BN * 4>(xa));
#pragma unroll
          for (int i = 0; i < 4; ++i) f.x[S][i] = v[i];
        } else {
          const uint64_t v = ds_read8<S * BN * 4>(xa);
          f.x[S][0] = __builtin_bit_cast(float, (uint32_t)v);
          f.x[S][1] = __builtin_bit_cast(float, (uint32_t)(v >> 32));
        }
      });
    }
  };
  auto mma = [&](const Frags& f) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(f.x[s][i], f.y[j][s], acc[i][j], 0, 0, 0);
  };
  // Both step pairs' reads go out first; the first pair's MFMAs wait only
  // for its own reads (LDS reads of a wave complete in order).
  auto compute = [&](uint32_t sbase) {
    static_assert(BK == 32 && NR <= 15, "two step pairs per slice, lgkmcnt holds at most 15");
    const uint32_t sa = sbase, sb = sbase + A_BYTES;
    Frags f0, f1;
    read(sa, sb, 0, f0);
    read(sa, sb, 1, f1);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, NR));
    __builtin_amdgcn_sched_barrier(0);
    mma(f0);
    lds_wait_all();
    mma(f1);
  };

  if (kt1 > kt0) {
#pragma unroll
    for (int q = 0; q < NSTG - 1; ++q) issue(kt0 + q, voa, vob);
    for (int t = kt0; t < kt1; ++t) {
      // This wave's loads of slice t are complete when at most the loads of
      // the NSTG - 2 later fills are in flight.
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(L * (NSTG - 2), 63));
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      issue(t + NSTG - 1, voa, vob);
      compute(ring_l + (uint32_t)((t % NSTG) * SLOT));
    }
    // Refills may still be landing in the ring: wait for them before the
    // workgroup's LDS is reused or goes to another workgroup.
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 63));
  }

  if constexpr (KG == 2) {
    // Group 1 parks its partial block in its own ring (every ring read and
    // refill of both groups is over after the barrier); group 0 adds it to
    // its own (group 0 + group 1, a fixed order) and runs the epilogue.
    constexpr int NF = FN * FM;
    __syncthreads();
    f32x4* park = reinterpret_cast<f32x4*>(ring_all + NSTG * SLOT) + wave * NF * 64 + lane;
    if (kg == 1) {
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) park[(i * FM + j) * 64] = acc[i][j];
    }
    __syncthreads();
    if (kg == 1) return;
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j) acc[i][j] += park[(i * FM + j) * 64];
  }

  if (part >= 0 && !split32_handoff<FN * FM, NT>(&acc[0][0], p, tile_id, part, tid)) return;

  // Epilogue, in runs of 4 consecutive columns per lane: K-contiguous B,
  // run c = fragment c's rows 4g..4g+3; N-contiguous B, run c = columns
  // wn*WN + 4 FN g + 4c + e, element e of run c from fragment (4c+e) % FN,
  // row (4c+e) / FN.
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
    for (int c = 0; c < FN; ++c) {
      const int n = B_KMAJOR ? n0 + wn * WN + c * 16 + 4 * g : n0 + wn * WN + 4 * FN * g + 4 * c;
      float bv[4] = {0.f, 0.f, 0.f, 0.f};
      if (has_bias) {
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[e] = (n + e < N) ? bias[n + e] : 0.f;
      }
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const int m = m0 + wm * WM + j * 16 + (lane & 15);
        if (m < M && n < N) {
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float a = B_KMAJOR ? acc[c][j][e] : acc[(4 * c + e) % FN][j][(4 * c + e) / FN];
            v[e] = act_t<ACT>(a * alpha + bv[e]);
          }
          if (R != nullptr) {
            float r[4];
            Res4<float>::load(R, (int64_t)m * p.ldr, n, N, rvec, r);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] += r[e];
          }
          Store4<float>::run(C + (int64_t)m * p.ldc, n, N, vec_ok, v);
        }
      }
    }
  });
}

}  // namespace sf
