// gemm16nt_4w.hpp — large-problem 16-bit NT GEMM, one wave per SIMD:
//
//   C[b] = epi(alpha * A[b] . B[b]^T (+ bias) (+ R[b])),  A M x K and B N x K
//   both K-contiguous (the forward linear x . W^T), 16-bit in and out, fp32
//   accumulation.
//
// One 256-thread workgroup per 256 x 256 output tile: four waves in a 2 x 2
// grid, each owning a 128 x 128 sub-tile = 8 x 8 blocks of
// v_mfma_f32_16x16x32 (256 fp32 accumulators, which the compiler keeps in
// the accumulation registers).  Against the 8-wave kernel of
// gemm16nt_pp.hpp (128 x 64 per wave) a wave reads 8 + 8 fragments per
// 32-deep k-slice for 64 MFMAs instead of 8 + 4 for 32: a third less LDS
// read traffic for the same work, which on this power-capped part buys
// clock (measured: dropping a third of the 8-wave kernel's fragment reads,
// in a timing-only copy, raised the clock 2 % and cut the time 3 %).
//
// With one wave per SIMD nothing else covers a wave's LDS latency, so the
// wave software-pipelines itself: while the MFMAs of slice t run, it reads
// the fragments of slice t + 1 into the other half of a double-buffered
// fragment set (64 VGPRs each) and issues its share of the direct-to-LDS
// loads of the pair two pairs ahead, fenced so that issue order is program
// order.  A pair's 64 loads per workgroup are spread over a slice and a
// half: issued in one half slice they back the vector memory path up into
// the MFMA issue (measured: 102.1 -> 99.4 us at 4096^3).
//
// LDS: two stages, each a pair of 32-deep k-slices of the 256-row A and B
// tiles (64 KB per stage), in the 8-wave kernel's layout: a 128-byte line
// is one row's 64 k values with 16-byte chunk h at slot h ^ (row & 7), so
// fragment reads are conflict-free; direct loads move whole 128-byte rows
// (wave w fills lines 64 w .. 64 w + 63 of each operand, 8 per
// instruction).  Rows past M or N load a copy of the last row; their
// products only reach unstored outputs.  K % 64 == 0 and K >= 192.
//
// Schedule per pair p (stage p % 2), per wave:
//   slice 2p     MFMAs on fragments [0], reads of slice 2p + 1 -> [1];
//                wait for the reads, workgroup barrier (every wave is done
//                with stage p % 2), the first 4 loads of pair p + 2 into
//                it; wait for this wave's loads of pair p + 1, workgroup
//                barrier (every load of pair p + 1 has landed);
//   slice 2p + 1 MFMAs on [1], reads of slice 2p + 2 (stage (p + 1) % 2)
//                -> [0] and the other 12 loads of pair p + 2; wait for the
//                reads.
// Two barriers per 128 MFMAs of each wave.  A fragment register is
// rewritten only after the MFMAs that read it were issued (in-order issue:
// an MFMA reads its sources at issue).
//
// Pair 0 is peeled so that its first slice's MFMAs start from a zero C
// operand (no clearing of 256 accumulators before the loop), and the last
// two pairs, which load nothing, are peeled after it.
//
// Epilogue: alpha, bias (moved into LDS beside the first k-pair), the
// activation (a template parameter: one epilogue per kernel keeps the
// accumulators in place until they are read) and the residual in
// registers, each wave staging its 128 x 128 result through LDS (64-row
// passes, 272-byte pitch) into non-temporal 16-byte row stores of 256-byte
// row segments.  With one tile per CU every tile's stores leave at once:
// the epilogue runs at the chip's write bandwidth (about 6 us at 4096^3).
#pragma once

#include "gemm16nt_pp.hpp"

namespace sf {

// One accumulator value moved to an ordinary register where the epilogue
// uses it: as an explicit read, the accumulators stay in the accumulation
// registers until then instead of all 256 moving out at the end of the
// loop (more than the ordinary registers hold beside the epilogue's own).
__device__ __forceinline__ float acc_read(float a) {
  float v;
  asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
  return v;
}

template <typename TIn, typename TOut, int ACT>
__global__ __launch_bounds__(256, 1) void gemm16nt_4w_kernel(GemmParams p) {
  constexpr int BM = 256, BN = 256;
  constexpr int FM = 8, FN = 8;            // 16-row (A) and 16-column (B) blocks per wave
  constexpr int OP_BYTES = 256 * 128;      // one operand's pair stage: 256 lines of 128 B
  constexpr int DMA_I = 8;                 // direct loads per operand per wave per pair
  __shared__ __attribute__((aligned(1024))) uint8_t sA[2][OP_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t sB[2][OP_BYTES];
  __shared__ __attribute__((aligned(16))) uint16_t sBias[BN];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int M = p.M, N = p.N, K = p.K;
  int tm, tn;
  group_tile(xcd_remap(blockIdx.x, gridDim.x), p.tiles_m, p.tiles_n, 8, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int64_t b = blockIdx.y;
  const uint16_t* __restrict__ A = static_cast<const uint16_t*>(p.A) + b * p.sA;
  const uint16_t* __restrict__ Bm = static_cast<const uint16_t*>(p.B) + b * p.sB;
  const int NP = K / 64;  // k-slice pairs

  // Direct loads: instruction i of wave w fills lines 64 w + 8 i .. + 7; lane
  // l writes slot l & 7 of line + (l >> 3), i.e. chunk (l & 7) ^ (l >> 3).
  // A per-lane offset per instruction, its row clamped to the last row of
  // the operand (rows past M or N load a copy of that row; their products
  // only reach unstored outputs); the pair's k offset goes in the scalar
  // offset.
  const int nrA = (int)((uint32_t)M * (uint32_t)p.lda * 2u), nrB = (int)((uint32_t)N * (uint32_t)p.ldb * 2u);
  const int dl = lane >> 3;
  const uint32_t dch = (uint32_t)(((lane & 7) ^ dl) * 16);
  uint32_t voa[DMA_I], vob[DMA_I];
#pragma unroll
  for (int i = 0; i < DMA_I; ++i) {
    const int ga = m0 + wave * 64 + i * 8 + dl, gb = n0 + wave * 64 + i * 8 + dl;
    voa[i] = (uint32_t)(ga < M ? ga : M - 1) * (uint32_t)p.lda * 2u + dch;
    vob[i] = (uint32_t)(gb < N ? gb : N - 1) * (uint32_t)p.ldb * 2u + dch;
  }
  auto rsrc = [&](const uint16_t* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, bytes, 0x00020000);
  };
  auto dma_a = [&](__amdgpu_buffer_rsrc_t r, int s, int kk, auto i_c) {
    constexpr int I = decltype(i_c)::value;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)(&sA[s][0] + wave * 8192 + I * 1024), 16, voa[I],
                                             kk * 2, 0, 0);
  };
  auto dma_b = [&](__amdgpu_buffer_rsrc_t r, int s, int kk, auto i_c) {
    constexpr int I = decltype(i_c)::value;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)(&sB[s][0] + wave * 8192 + I * 1024), 16, vob[I],
                                             kk * 2, 0, 0);
  };
  auto dma_pair = [&](int s, int kk) {
    const __amdgpu_buffer_rsrc_t ra = rsrc(A, nrA), rb = rsrc(Bm, nrB);
    static_for<DMA_I>([&](auto i_c) { dma_a(ra, s, kk, i_c); });
    static_for<DMA_I>([&](auto i_c) { dma_b(rb, s, kk, i_c); });
  };
  // Bias (as the 8-wave kernel): waves 0 and 1 move 128 values each into
  // LDS beside pair 0; an odd N loads it in the epilogue instead.
  const bool bias_lds = epi_has_bias(p.epi) && (N & 1) == 0;
  if (bias_lds && wave < 2) {
    const __amdgpu_buffer_rsrc_t rBias = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(p.bias), (short)0, (int)((uint32_t)N * 2u), 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rBias, (lds_ptr_t)(reinterpret_cast<uint8_t*>(&sBias[0]) + wave * 256), 4,
                                             (uint32_t)(n0 + wave * 128) * 2u + (uint32_t)lane * 4u, 0, 0, 0);
  }

  // Fragment offsets: A block j = rows wm 128 + 16 j + (l & 15), B block i =
  // rows wn 128 + 16 i + (l & 15), chunk l >> 4 (even slice) or 4 + (l >> 4)
  // (odd slice: slot bit 2 flipped, byte bit 6).
  const uint32_t fo = (uint32_t)((lane & 15) * 128 + (((lane >> 4) ^ (lane & 7)) << 4));
  const uint32_t la0 = lds_addr(&sA[0][0]) + (uint32_t)(wm * 128 * 128) + fo;
  const uint32_t lb0 = lds_addr(&sB[0][0]) + (uint32_t)(wn * 128 * 128) + fo;

  f32x4 acc[FN][FM];  // first written by slice 0's MFMAs, which add to zero
  u32x4 fa[2][FM], fb[2][FN];

  // Fragment q of slice t (A blocks 0-7, then B blocks 0-7) into set BUF:
  // slice t lies in stage (t / 2) % 2, half t % 2.
  auto read_slice_frag = [&](auto q_c, int t, auto buf_c) {
    constexpr int Q = decltype(q_c)::value;
    constexpr int BUF = decltype(buf_c)::value;
    const uint32_t st = (uint32_t)(((t >> 1) & 1) * OP_BYTES);
    if constexpr (Q < FM) {
      const uint32_t a = (la0 + st) ^ ((t & 1) ? 64u : 0u);
      fa[BUF][Q] = ds_read16<Q * 2048>(a);
    } else {
      const uint32_t a = (lb0 + st) ^ ((t & 1) ? 64u : 0u);
      fb[BUF][Q - FM] = ds_read16<(Q - FM) * 2048>(a);
    }
  };
  // 64 MFMAs on fragment set BUF in 32 groups of two, with (READS) the 16
  // reads of slice tnext into the other set after groups 0-15 and (LOADS)
  // part of the direct loads of the pair at kk into stage sn.  FIRST marks
  // the pair's first slice: there LOADS first waits for this wave's reads
  // and crosses a workgroup barrier (after group 19: every wave is then done
  // with stage sn), then issues loads 0-3 after groups 20, 23, 26, 29; the
  // second slice issues loads 4-15 after the odd groups 1 .. 23.  Spreading
  // a pair's 64 loads per workgroup over a slice and a half keeps the
  // vector memory path from backing up into the MFMA issue.  All choices
  // are compile-time: the loop body has no branch, so the accumulators stay
  // in the accumulation registers across it.
  auto compute = [&](auto buf_c, auto reads_c, auto loads_c, auto first_c, int tnext, int sn, int kk,
                     __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb, auto zero_c) {
    constexpr int BUF = decltype(buf_c)::value;
    constexpr int NB = 1 - BUF;
    constexpr bool READS = decltype(reads_c)::value;
    constexpr bool LOADS = decltype(loads_c)::value;
    constexpr bool FIRST = decltype(first_c)::value;
    constexpr bool ZERO = decltype(zero_c)::value;  // slice 0: C operand zero
    static_for<32>([&](auto g_c) {
      constexpr int G = decltype(g_c)::value;
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int mm = G * 2 + u;  // MFMA index: i = mm / 8, j = mm % 8
        acc[mm / FM][mm % FM] = Mfma16<TIn>::run(fb[BUF][mm / FM], fa[BUF][mm % FM],
                                                 ZERO ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[mm / FM][mm % FM]);
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (READS && G < 16) read_slice_frag(std::integral_constant<int, G>{}, tnext, std::integral_constant<int, NB>{});
      if constexpr (LOADS) {
        // load index after group G (-1: none)
        constexpr int L = FIRST ? (G >= 20 && (G - 20) % 3 == 0 ? (G - 20) / 3 : -1)
                                : ((G & 1) && G <= 23 ? 4 + (G >> 1) : -1);
        if constexpr (FIRST && G == 19) {
          __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
          __builtin_amdgcn_s_barrier();
          __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (L >= 0 && L < DMA_I)
          dma_a(ra, sn, kk, std::integral_constant<int, L>{});
        else if constexpr (L >= DMA_I)
          dma_b(rb, sn, kk, std::integral_constant<int, L - DMA_I>{});
      }
    });
    __builtin_amdgcn_sched_barrier(0);
  };
  constexpr std::true_type yes{};
  constexpr std::false_type no{};
  constexpr std::integral_constant<int, 0> set0{};
  constexpr std::integral_constant<int, 1> set1{};
  // End of a pair's first slice: this wave's reads done and its loads of the
  // next pair landed (only the NEWER loads, already issued for the pair
  // after it, may still be in flight); then every wave is done reading and
  // every load of the next pair has landed.
  auto pair_sync = [&](auto newer_c) {
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(decltype(newer_c)::value, 0));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  };
  auto reads_done = [&]() {
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
    __builtin_amdgcn_sched_barrier(0);
  };
  constexpr std::integral_constant<int, 4> first_loads{};  // loads issued in a pair's first slice

  // Prologue: pairs 0 and 1 in flight, slice 0's fragments read.
  dma_pair(0, 0);
  dma_pair(1, 64);
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(2 * DMA_I, 0));  // pair 0 (and the bias) landed
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  static_for<16>([&](auto q_c) { read_slice_frag(q_c, 0, set0); });
  reads_done();

  // Pairs 0 .. NP - 3: slice 2 pp on set 0 (reads of slice 2 pp + 1 into set
  // 1, then the first loads of pair pp + 2 into this pair's stage), slice
  // 2 pp + 1 on set 1 (reads of slice 2 pp + 2 into set 0, the rest of the
  // loads).  Pair 0 is peeled: its first slice's MFMAs take a zero C
  // operand instead of 256 accumulators cleared beforehand.
  {
    const __amdgpu_buffer_rsrc_t ra = rsrc(A, nrA), rb = rsrc(Bm, nrB);
    compute(set0, yes, yes, yes, 1, 0, 128, ra, rb, yes);
    pair_sync(first_loads);
    compute(set1, yes, yes, no, 2, 0, 128, ra, rb, no);
    reads_done();
    for (int pp = 1; pp < NP - 2; ++pp) {
      const int sn = pp & 1, kk = (pp + 2) * 64;
      compute(set0, yes, yes, yes, 2 * pp + 1, sn, kk, ra, rb, no);
      pair_sync(first_loads);
      compute(set1, yes, yes, no, 2 * pp + 2, sn, kk, ra, rb, no);
      reads_done();
    }
  }
  // The last two pairs load nothing more; the very last slice reads nothing.
  {
    const __amdgpu_buffer_rsrc_t r0 = rsrc(A, 0);
    compute(set0, yes, no, yes, 2 * NP - 3, 0, 0, r0, r0, no);
    pair_sync(std::integral_constant<int, 0>{});
    compute(set1, yes, no, no, 2 * NP - 2, 0, 0, r0, r0, no);
    reads_done();
    compute(set0, yes, no, yes, 2 * NP - 1, 0, 0, r0, r0, no);
    reads_done();
    compute(set1, no, no, no, 0, 0, 0, r0, r0, no);
  }

  // ---- epilogue ------------------------------------------------------------
  const int elane = lane_id_fresh();
  const bool has_bias = epi_has_bias(p.epi);
  const float alpha = p.alpha;
  float bv[FN][4];
  if (bias_lds) {
    const uint32_t ba = lds_addr(&sBias[0]) + (uint32_t)(wn * 128 + 4 * (elane >> 4)) * 2u;
    u32x2 bw[FN];
    static_for<FN>([&](auto i_c) {
      constexpr int I = decltype(i_c)::value;
      bw[I] = ds_read8v<I * 32>(ba);
    });
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      bv[i][0] = Elem<TIn>::to_f32(static_cast<uint16_t>(bw[i][0]));
      bv[i][1] = Elem<TIn>::to_f32(static_cast<uint16_t>(bw[i][0] >> 16));
      bv[i][2] = Elem<TIn>::to_f32(static_cast<uint16_t>(bw[i][1]));
      bv[i][3] = Elem<TIn>::to_f32(static_cast<uint16_t>(bw[i][1] >> 16));
    }
  } else {
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) bv[i][q] = 0.f;
      if (has_bias) load_bias4<TIn>(p.bias, n0 + wn * 128 + i * 16 + 4 * (elane >> 4), N, bv[i]);
    }
  }
  constexpr int WN = 128, WM = 128;
  constexpr int PITCH = WN * 2 + 16;  // 272 bytes
  constexpr int ROWS_S = 64;          // rows per pass: 17408 bytes per wave
  uint8_t* stage = (wave < 2 ? &sA[0][0] : &sB[0][0]) + (wave & 1) * (ROWS_S * PITCH);
  constexpr int LANES_ROW = WN * 2 / 16;  // 16 lanes store one 256-byte row segment
  constexpr int ROWS_I = 64 / LANES_ROW;  // 4 rows per store instruction
  uint16_t* C = static_cast<uint16_t*>(p.C) + b * p.sC;
  const bool vec_ok = ((p.ldc & 7) == 0) && ((reinterpret_cast<uintptr_t>(C) & 15) == 0);
  // Residual: the wave's whole 128 x 128 block of R is loaded before the
  // epilogue's first barrier (raw 16-bit pairs in the accumulator layout,
  // 128 registers that the main loop's fragments have freed), so its
  // latency is paid once per tile, not once per pass (R may alias C, which
  // keeps the compiler from hoisting the loads itself).  R may be C: every
  // element is read here, before any store.  Rows past M read row M - 1
  // (not stored), columns past N read as zero.
  const uint16_t* R = p.res != nullptr ? static_cast<const uint16_t*>(p.res) + b * p.sR : nullptr;
  const bool rvec = R != nullptr && res_vec_ok<TOut>(R, p.ldr);
  u32x2 rall[WM / 16][FN];
  if (R != nullptr) {
#pragma unroll
    for (int j = 0; j < WM / 16; ++j) {
      const int gm = m0 + wm * WM + j * 16 + (elane & 15);
      const uint16_t* rrow = R + (int64_t)(gm < M ? gm : M - 1) * p.ldr;
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        const int n = n0 + wn * WN + i * 16 + 4 * (elane >> 4);
        if (rvec && n + 3 < N) {
          rall[j][i] = *reinterpret_cast<const u32x2*>(rrow + n);
        } else {
          uint32_t h[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) h[q] = n + q < N ? rrow[n + q] : 0u;
          rall[j][i] = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
        }
      }
    }
  }
  {
#pragma unroll
    for (int ps = 0; ps < WM / ROWS_S; ++ps) {
      // the first pass waits for every wave's last fragment reads of the
      // stage arrays; later passes only order this wave's own accesses
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
          for (int q = 0; q < 4; ++q) v[q] = act_t<ACT>(acc_read(acc[i][j][q]) * alpha + bv[i][q]);
          if (R != nullptr) {
            const u32x2 rw = rall[j][i];
#pragma unroll
            for (int q = 0; q < 4; ++q)
              v[q] += Elem<TOut>::to_f32(static_cast<uint16_t>(rw[q >> 1] >> ((q & 1) * 16)));
          }
          const uint32_t lo = pack2<TOut>(v[0], v[1]);
          const uint32_t hi = pack2<TOut>(v[2], v[3]);
          *reinterpret_cast<u32x2*>(stage + r * PITCH + (i * 16 + 4 * (elane >> 4)) * 2) = u32x2{lo, hi};
        }
      }
      wave_lds_sync();
      u32x4 vals[ROWS_S / ROWS_I];
      const int cl = elane % LANES_ROW;
#pragma unroll
      for (int rr = 0; rr < ROWS_S / ROWS_I; ++rr)
        vals[rr] = *reinterpret_cast<const u32x4*>(stage + (rr * ROWS_I + elane / LANES_ROW) * PITCH + cl * 16);
#pragma unroll
      for (int rr = 0; rr < ROWS_S / ROWS_I; ++rr) {
        const int r = rr * ROWS_I + elane / LANES_ROW;
        const int gm = m0 + wm * WM + ps * ROWS_S + r;
        const int gn = n0 + wn * WN + cl * 8;
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
}

}  // namespace sf
