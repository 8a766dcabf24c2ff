// gemm16nt_k64.hpp — 16-bit NT GEMM with K = 64 exactly:
//
//   C[b] = epi(alpha * A[b] . B[b]^T (+ bias) (+ R[b])),  A M x 64, B N x 64,
//
// the attention scores Q K^T at head size 64 (C4: 60 x 4096 x 4096, 2 GB of
// 16-bit scores written for 62 MB read).  Such a product is bound by its
// stores, so the kernel is built to keep stores in flight: one 256-thread
// workgroup per 128 x 128 tile, four waves of 64 x 64 (64 fp32
// accumulators), at most 128 VGPRs and 32 KB of LDS, so four workgroups
// share a CU and one's epilogue stores overlap the others' loads and MFMAs.
// (The 8-wave 256 x 256 kernel ran this shape at one workgroup per CU: 220
// VGPRs. Measured on one box, C4's scores: 0.4227 -> 0.3808 ms, 4.76 ->
// 5.29 TB/s written, bit-identical; one 64-row epilogue pass or four
// 16-row passes instead of two 32-row passes: within 0.5 %.)
//
// Per workgroup: the A and B tiles (128 rows x 128 bytes each, the 8-wave
// kernel's line layout: 16-byte chunk h of a row at slot h ^ (row & 7))
// arrive by direct-to-LDS loads, 8 whole rows per instruction, rows past M
// or N clamped to the last row (their outputs are not stored); each wave
// then reads its fragments of k 0-31, runs 16 v_mfma_f32_16x16x32, reads
// those of k 32-63 and runs 16 more.  The epilogue (alpha, bias, activation
// as a template parameter, residual, one rounding) stages each wave's
// results through LDS in two 32-row passes (144-byte pitch, conflict-free)
// into non-temporal 16-byte stores of 128-byte row segments.  Every output
// accumulates in the 8-wave kernel's order, so results match it bit for bit.
#pragma once

#include "gemm16nt_pp.hpp"

namespace sf {

template <typename TIn, typename TOut, int ACT>
__global__ __launch_bounds__(256, 4) void gemm16nt_k64_kernel(GemmParams p) {
  constexpr int BM = 128, BN = 128;
  constexpr int FM = 4, FN = 4;       // 16-row (A) and 16-column (B) blocks per wave
  constexpr int PITCH = 64 * 2 + 16;  // staged row: 64 outputs + 16 bytes
  constexpr int ROWS_S = 32;          // rows per epilogue pass
  static_assert(4 * ROWS_S * PITCH <= (BM + BN) * 128, "the staging fits in the operand lines");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[(BM + BN) * 128];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int M = p.M, N = p.N;
  int tm, tn;
  group_tile(xcd_remap(blockIdx.x, gridDim.x), p.tiles_m, p.tiles_n, 8, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int64_t b = blockIdx.y;
  const uint16_t* __restrict__ A = static_cast<const uint16_t*>(p.A) + b * p.sA;
  const uint16_t* __restrict__ Bm = static_cast<const uint16_t*>(p.B) + b * p.sB;

  // Direct loads: 256 lines of 128 bytes (A rows 0-127, then B rows 0-127);
  // wave w moves lines 64 w .. 64 w + 63, 8 per instruction; lane l writes
  // slot l & 7 of line + (l >> 3), i.e. chunk (l & 7) ^ (l >> 3).  Rows past
  // M or N load the last row (their outputs are not stored).
  {
    const int dl = lane >> 3;
    const uint32_t dch = (uint32_t)(((lane & 7) ^ dl) * 16);
    const bool is_b = wave >= 2;
    const int rows = is_b ? N : M;
    const int base = (is_b ? n0 : m0) + (wave & 1) * 64;
    const int64_t ld = is_b ? p.ldb : p.lda;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(is_b ? Bm : A), (short)0, (int)((uint32_t)rows * (uint32_t)ld * 2u), 0x00020000);
    static_for<8>([&](auto i_c) {
      constexpr int I = decltype(i_c)::value;
      const int g = base + I * 8 + dl;
      const uint32_t vo = (uint32_t)(g < rows ? g : rows - 1) * (uint32_t)ld * 2u + dch;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)(smem + wave * 8192 + I * 1024), 16, vo, 0, 0, 0);
    });
  }

  // Fragment offsets (the 8-wave kernel's): A block j = rows wm 64 + 16 j +
  // (l & 15), B block i = rows wn 64 + 16 i + (l & 15), chunk l >> 4 of the
  // first 32 k, 4 + (l >> 4) of the second (address bit 6 flipped).
  const uint32_t fo = (uint32_t)((lane & 15) * 128 + (((lane >> 4) ^ (lane & 7)) << 4));
  const uint32_t la = lds_addr(smem) + (uint32_t)(wm * 64 * 128) + fo;
  const uint32_t lb = lds_addr(smem) + (uint32_t)(BM * 128 + wn * 64 * 128) + fo;

  __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);

  f32x4 acc[FN][FM];
  static_for<2>([&](auto s_c) {
    constexpr int SL = decltype(s_c)::value;
    constexpr uint32_t X = SL ? 64u : 0u;
    u32x4 fa[FM], fb[FN];
    static_for<FM>([&](auto j_c) {
      constexpr int J = decltype(j_c)::value;
      fa[J] = ds_read16<0>((la + J * 2048) ^ X);
    });
    static_for<FN>([&](auto i_c) {
      constexpr int I = decltype(i_c)::value;
      fb[I] = ds_read16<0>((lb + I * 2048) ^ X);
    });
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j)
        acc[i][j] = Mfma16<TIn>::run(fb[i], fa[j], SL ? acc[i][j] : f32x4{0.f, 0.f, 0.f, 0.f});
    __builtin_amdgcn_sched_barrier(0);
  });

  // ---- epilogue: alpha, bias, activation, residual; staged through LDS ----
  const int elane = lane_id_fresh();
  const bool has_bias = epi_has_bias(p.epi);
  const float alpha = p.alpha;
  float bv[FN][4];
#pragma unroll
  for (int i = 0; i < FN; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) bv[i][q] = 0.f;
    if (has_bias) load_bias4<TIn>(p.bias, n0 + wn * 64 + i * 16 + 4 * (elane >> 4), N, bv[i]);
  }
  uint8_t* stage = smem + wave * (ROWS_S * PITCH);
  uint16_t* C = static_cast<uint16_t*>(p.C) + b * p.sC;
  const bool vec_ok = ((p.ldc & 7) == 0) && ((reinterpret_cast<uintptr_t>(C) & 15) == 0);
  const void* R = p.res != nullptr ? static_cast<const uint16_t*>(p.res) + b * p.sR : nullptr;
  const bool rvec = R != nullptr && res_vec_ok<TOut>(R, p.ldr);
#pragma unroll
  for (int ps = 0; ps < 64 / ROWS_S; ++ps) {
    // the first pass waits for every wave's fragment reads (the staging
    // area covers the operand lines); later passes only order this wave's
    if (ps == 0)
      __syncthreads();
    else
      wave_lds_sync();
#pragma unroll
    for (int jj = 0; jj < ROWS_S / 16; ++jj) {
      const int j = ps * (ROWS_S / 16) + jj;
      const int r = jj * 16 + (elane & 15);
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = act_t<ACT>(acc[i][j][q] * alpha + bv[i][q]);
        if (R != nullptr) {
          const int gm = m0 + wm * 64 + j * 16 + (elane & 15);
          if (gm < M) {
            float rr[4];
            Res4<TOut>::load(R, (int64_t)gm * p.ldr, n0 + wn * 64 + i * 16 + 4 * (elane >> 4), N, rvec, rr);
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] += rr[q];
          }
        }
        const uint32_t lo = pack2<TOut>(v[0], v[1]);
        const uint32_t hi = pack2<TOut>(v[2], v[3]);
        *reinterpret_cast<u32x2*>(stage + r * PITCH + (i * 16 + 4 * (elane >> 4)) * 2) = u32x2{lo, hi};
      }
    }
    wave_lds_sync();
    // 8 lanes a 128-byte row segment, 8 rows a store
    u32x4 vals[ROWS_S / 8];
    const int cl = elane & 7;
#pragma unroll
    for (int rr = 0; rr < ROWS_S / 8; ++rr)
      vals[rr] = *reinterpret_cast<const u32x4*>(stage + (rr * 8 + (elane >> 3)) * PITCH + cl * 16);
#pragma unroll
    for (int rr = 0; rr < ROWS_S / 8; ++rr) {
      const int gm = m0 + wm * 64 + ps * ROWS_S + rr * 8 + (elane >> 3);
      const int gn = n0 + wn * 64 + cl * 8;
      if (gm < M) {
        uint16_t* crow = C + (int64_t)gm * p.ldc;
        if (vec_ok && gn + 8 <= N) {
          __builtin_nontemporal_store(vals[rr], reinterpret_cast<u32x4*>(crow + gn));
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (gn + e < N) crow[gn + e] = static_cast<uint16_t>(vals[rr][e >> 1] >> ((e & 1) * 16));
        }
      }
    }
  }
}

}  // namespace sf
