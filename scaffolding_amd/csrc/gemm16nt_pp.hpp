// gemm16nt_pp.hpp — large-problem 16-bit NT GEMM with an 8-wave ping-pong
// schedule:
//
//   C[b] = epi(alpha * A[b] . B[b]^T (+ bias)),  A M x K, B N x K, both
//   K-contiguous, 16-bit in and out, fp32 accumulation.
//
// One 512-thread workgroup per 256 x 256 output tile; eight waves in a
// 2 x 4 grid, each owning a 128 x 64 sub-tile = 4 x 8 blocks of
// v_mfma_f32_16x16x32 (128 fp32 accumulators), so two waves fit on every
// SIMD.  A wave alternates a memory phase (ds_read its fragments of one
// 32-deep k-slice, issue its share of the direct-to-LDS loads of a later
// slice) and a compute phase (32 MFMAs on those fragments).
//
// Ping-pong.  Waves 0-3 (group 0) and 4-7 (group 1) sit one per SIMD each.
// Group 1 passes one extra workgroup barrier at the start (group 0 one at
// the end), which offsets the groups by half a step: between consecutive
// barriers one group computes while the other loads, so each SIMD's MFMA
// pipe is fed by one wave while its sibling's LDS traffic is in flight.
// Per wave the loop is  memory(t); barrier; compute(t); barrier.
//
// LDS: four stages of the 256 x 32 A and B slices (separate __shared__
// arrays, so the compiler's wait-count logic can tell a direct load into
// one stage from ds_reads of another; the loop is unrolled by four so stage
// references are static).  Operand tiles reach LDS through gfx950's
// direct-to-LDS load (global_load_lds_dwordx4: lane l's 16 bytes land at
// base + 16 l), so no VGPRs or ds_write instructions carry them.  A slice
// row is 32 elements = 64 bytes = four 16-byte chunks.  The 16 KB stage is
// laid out as 128 lines of 128 bytes: line q holds rows q and q + 128, and
// logical chunk h = 4 * (row >> 7) + c sits at slot h ^ (q & 7).  An MFMA
// fragment (16 consecutive rows, one chunk) then reads 16 lines at 128-byte
// stride with the slot rotated by the line, which ds_read_b128 serves
// without bank conflicts (measured: 64-byte-row layouts conflict whatever
// the chunk swizzle).  A direct-load instruction fills 8 lines slot by
// slot, so lane l fetches logical chunk (l & 7) ^ (l >> 3) of line l >> 3.
// Rows past M or N are clamped to
// the last valid row (their products only reach unstored outputs);
// K % 128 == 0 is required.  Slice t is read by
// group 0 between barriers 2t and 2t+1 and by group 1 between 2t+1 and
// 2t+2, so every wave finishes its own loads of slice t before barrier 2t
// (group 0 at the end of compute(t-1), group 1 at the end of memory(t-1)),
// and the loads of slice t+3 (issued in memory(t)) only start after the
// last reads of slice t-1, which sat in the same stage.  Each memory phase
// ends with its ds_reads complete (lgkmcnt 0) for the same reason.
//
// Epilogue: alpha, bias and activation in registers, each wave stages its
// 128 x 64 result through its own LDS array (64-row passes, 144-byte
// pitch) and stores 128-byte row segments with 16-byte lanes.
#pragma once

#include "gemm16.hpp"

namespace sf {

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef const __attribute__((address_space(1))) void* gbl_ptr_t;

// Direct global -> LDS load of 16 bytes per lane (global_load_lds_dwordx4):
// lane l's bytes land at LDS address `lds` + 16 l; `lds` is wave-uniform.
__device__ __forceinline__ void dma16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds((gbl_ptr_t)g, (lds_ptr_t)lds, 16, 0, 0);
}

// ds_read_b128 of 16 bytes at LDS byte address `addr` + OFF, issued as inline
// assembly.  The compiler cannot tell which LDS array a direct load writes,
// so for an ordinary LDS load it waits for every direct load in flight
// (vmcnt(0)), which would drain the prefetch queue each k-step; this form
// carries no such wait.  The caller orders it with explicit s_waitcnt:
// lgkmcnt before the data is used, and the vmcnt + barrier protocol below
// before the bytes it reads are valid.
template <int OFF>
__device__ __forceinline__ u32x4 ds_read16(uint32_t addr) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] |
// lgkmcnt[11:8] | vmcnt[5:4] << 14); counts not being waited on are at max.
constexpr int waitcnt_imm(int vm, int lgkm) {
  return (vm & 15) | (7 << 4) | ((lgkm & 15) << 8) | (((vm >> 4) & 3) << 14);
}

template <typename TIn, typename TOut>
__global__ __launch_bounds__(512) void gemm16nt_pp_kernel(GemmParams p) {
  constexpr int BM = 256, BN = 256, BK = 32;
  constexpr int WM = 128, WN = 64, FM = WM / 16, FN = WN / 16;
  constexpr int OP_BYTES = BM * BK * 2;  // 16 KB per operand per stage
  constexpr int DMA_I = 2;               // per operand per wave per slice (32 rows)
  constexpr int DPT = 2 * DMA_I;         // direct loads per wave per slice
  __shared__ __attribute__((aligned(1024))) uint8_t sA0[OP_BYTES], sB0[OP_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t sA1[OP_BYTES], sB1[OP_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t sA2[OP_BYTES], sB2[OP_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t sA3[OP_BYTES], sB3[OP_BYTES];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2;
  const int wm = wave >> 2;
  const int wn = wave & 3;

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
  const int KT = K / BK;  // multiple of 4

  // Direct loads: instruction i of this wave fills lines wave*16 + 8 i .. +7;
  // lane l takes line + (l >> 3), logical chunk h = (l & 7) ^ (l >> 3), i.e.
  // row line + 128 (h >> 2), chunk h & 3.
  const int dh = (lane & 7) ^ (lane >> 3);
  const uint32_t dchunk_b = (uint32_t)((dh & 3) * 16);
  const int drow = wave * 16 + (lane >> 3) + (dh >> 2) * 128;
  const int ra0 = m0 + drow;
  const int rb0 = n0 + drow;
  const uint32_t lda_b = (uint32_t)p.lda * 2u, ldb_b = (uint32_t)p.ldb * 2u;
  const char* Ab = reinterpret_cast<const char*>(A);
  const char* Bb = reinterpret_cast<const char*>(B);
  auto dma = [&](uint8_t* sA, uint8_t* sB, int k0) {
    const char* ak = Ab + (size_t)k0 * 2;
    const char* bk = Bb + (size_t)k0 * 2;
#pragma unroll
    for (int i = 0; i < DMA_I; ++i) {
      const int ga = ra0 + i * 8, gb = rb0 + i * 8;
      const uint32_t oa = (uint32_t)(ga < M ? ga : M - 1) * lda_b + dchunk_b;
      const uint32_t ob = (uint32_t)(gb < N ? gb : N - 1) * ldb_b + dchunk_b;
      dma16(ak + oa, sA + (wave * 16 + i * 8) * 128);
      dma16(bk + ob, sB + (wave * 16 + i * 8) * 128);
    }
  };

  f32x4 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  u32x4 ya[FM], xb[FN];

  // Fragment byte offsets: A block j reads rows wm*128 + 16 j + (l & 15),
  // i.e. lines 16 j + (l & 15), logical chunk 4 wm + (l >> 4); B block i
  // reads rows wn*64 + 16 i + (l & 15), i.e. lines 64 (wn & 1) + 16 i +
  // (l & 15), logical chunk 4 (wn >> 1) + (l >> 4).  Blocks are 2 KB apart.
  const int fa = (lane & 15) * 128 + (((wm * 4 + (lane >> 4)) ^ (lane & 7)) << 4);
  const int fb = ((wn & 1) * 64 + (lane & 15)) * 128 + ((((wn >> 1) * 4 + (lane >> 4)) ^ (lane & 7)) << 4);

  // Waits: own direct loads of slice t+1 landed; slices after it that this
  // wave already issued (at most two) may still be in flight.
  auto wait_next = [&](int t) {
    const int pend = KT - 2 - t;  // slices t+2 .. min(t+3, KT-1) issued
    if (pend >= 2)
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(2 * DPT, 0));
    else if (pend == 1)
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(DPT, 0));
    else
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
  };

  auto step = [&](int t, const uint8_t* sA, const uint8_t* sB, uint8_t* nA, uint8_t* nB) {
    // memory phase
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t la = lds_addr(sA) + fa, lb = lds_addr(sB) + fb;
    ya[0] = ds_read16<0 * 2048>(la);
    ya[1] = ds_read16<1 * 2048>(la);
    ya[2] = ds_read16<2 * 2048>(la);
    ya[3] = ds_read16<3 * 2048>(la);
    ya[4] = ds_read16<4 * 2048>(la);
    ya[5] = ds_read16<5 * 2048>(la);
    ya[6] = ds_read16<6 * 2048>(la);
    ya[7] = ds_read16<7 * 2048>(la);
    xb[0] = ds_read16<0 * 2048>(lb);
    xb[1] = ds_read16<1 * 2048>(lb);
    xb[2] = ds_read16<2 * 2048>(lb);
    xb[3] = ds_read16<3 * 2048>(lb);
    if (t + 3 < KT) dma(nA, nB, (t + 3) * BK);
    if (grp == 1)
      wait_next(t);
    else
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // compute phase
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j) acc[i][j] = Mfma16<TIn>::run(xb[i], ya[j], acc[i][j]);
    __builtin_amdgcn_sched_barrier(0);
    if (grp == 0) wait_next(t);
    __builtin_amdgcn_s_barrier();
  };

  dma(sA0, sB0, 0);
  dma(sA1, sB1, BK);
  dma(sA2, sB2, 2 * BK);
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(2 * DPT, 0));  // own part of slice 0
  __builtin_amdgcn_s_barrier();
  if (grp == 1) __builtin_amdgcn_s_barrier();
  for (int t = 0; t < KT; t += 4) {
    step(t + 0, sA0, sB0, sA3, sB3);
    step(t + 1, sA1, sB1, sA0, sB0);
    step(t + 2, sA2, sB2, sA1, sB1);
    step(t + 3, sA3, sB3, sA2, sB2);
  }
  if (grp == 0) __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);

  // ---- epilogue ------------------------------------------------------------
  const bool has_bias = epi_has_bias(p.epi);
  const int act = epi_act(p.epi);
  const float alpha = p.alpha;
  float bv[FN][4];
#pragma unroll
  for (int i = 0; i < FN; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) bv[i][q] = 0.f;
    if (has_bias) load_bias4<TIn>(p.bias, n0 + wn * WN + i * 16 + 4 * (lane >> 4), N, bv[i]);
  }
  uint8_t* stage;
  switch (wave) {
    case 0: stage = sA0; break;
    case 1: stage = sB0; break;
    case 2: stage = sA1; break;
    case 3: stage = sB1; break;
    case 4: stage = sA2; break;
    case 5: stage = sB2; break;
    case 6: stage = sA3; break;
    default: stage = sB3; break;
  }
  constexpr int PITCH = WN * 2 + 16;  // 144 bytes
  constexpr int ROWS_S = 64;          // 64 x 144 = 9216 B per pass
  constexpr int LANES_ROW = WN * 2 / 16;
  constexpr int ROWS_I = 64 / LANES_ROW;
  uint16_t* C = static_cast<uint16_t*>(p.C) + b * p.sC;
  const bool vec_ok = ((p.ldc & 7) == 0) && ((reinterpret_cast<uintptr_t>(C) & 15) == 0);
  with_act(act, [&](auto act_c) {
  constexpr int ACT = decltype(act_c)::value;
#pragma unroll
  for (int ps = 0; ps < WM / ROWS_S; ++ps) {
    __syncthreads();
#pragma unroll
    for (int jj = 0; jj < ROWS_S / 16; ++jj) {
      const int j = ps * (ROWS_S / 16) + jj;
      const int r = jj * 16 + (lane & 15);
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = act_t<ACT>(acc[i][j][q] * alpha + bv[i][q]);
        const uint32_t lo = Elem<TOut>::from_f32(v[0]) | ((uint32_t)Elem<TOut>::from_f32(v[1]) << 16);
        const uint32_t hi = Elem<TOut>::from_f32(v[2]) | ((uint32_t)Elem<TOut>::from_f32(v[3]) << 16);
        *reinterpret_cast<u32x2*>(stage + r * PITCH + (i * 16 + 4 * (lane >> 4)) * 2) = u32x2{lo, hi};
      }
    }
    __syncthreads();
#pragma unroll
    for (int rr = 0; rr < ROWS_S / ROWS_I; ++rr) {
      const int r = rr * ROWS_I + lane / LANES_ROW;
      const int cl = lane % LANES_ROW;
      const int gm = m0 + wm * WM + ps * ROWS_S + r;
      const int gn = n0 + wn * WN + cl * 8;
      const u32x4 val = *reinterpret_cast<const u32x4*>(stage + r * PITCH + cl * 16);
      if (gm < M) {
        uint16_t* crow = C + (int64_t)gm * p.ldc;
        if (vec_ok && gn + 8 <= N) {
          *reinterpret_cast<u32x4*>(crow + gn) = val;
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (gn + e < N) crow[gn + e] = static_cast<uint16_t>(val[e >> 1] >> ((e & 1) * 16));
        }
      }
    }
  }
  });
}

}  // namespace sf
