// gemm16nt_pp.hpp — large-problem 16-bit GEMM with an 8-wave ping-pong
// schedule:
//
//   C[b] = epi(alpha * op(A[b]) . op(B[b]) (+ bias)),  16-bit in and out,
//   fp32 accumulation.  Each operand is K-contiguous (A M x K, B N x K: the
//   forward "NT" product x . W^T) or M/N-contiguous (A stored K x M, B stored
//   K x N: the backward products dY . W and dY^T . X) — template flags
//   A_KM / B_KM.
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
// LDS: two stages, each holding a pair of 32-deep k-slices of the 256-row A
// and B tiles (64 KB per stage, 128 KB in all).  A stage line is one row's
// 64 k values (128 bytes); its 16-byte chunk h sits at slot h ^ (row & 7),
// so the 16 rows of an MFMA fragment (one chunk each) fall on 16 distinct
// bank groups and ds_read_b128 runs without conflicts (measured; layouts of
// 64-byte rows conflict whatever the swizzle).  Operands move global -> LDS
// through gfx950's buffer_load_dwordx4 ... lds (lane l's 16 bytes land at
// the instruction's LDS base + 16 l; no VGPRs or ds_writes), each
// instruction fetching 8 whole 128-byte rows: full cache lines, twice the
// useful bytes per request of 64-byte row halves.  Rows past M or N are
// clamped to the last valid row (their products only reach unstored
// outputs); K % 128 == 0 is required.
//
// M/N-contiguous operands.  The stage (same 32 KB per operand) holds four
// blocks of 64 m (or n); block b is 64 k-rows of 128 bytes (64 m of one k),
// 16-byte chunk c of row k at slot c ^ fmn(k), fmn(k) = 2 ((k >> 1) & 1) +
// 4 ((k >> 3) & 1).  Direct-load instruction i of wave w fills rows
// 8w .. 8w+7 of block i (whole 128-byte rows again).  Fragments come from
// gfx950's transposing read ds_read_b64_tr_b16: two reads (k 0-3 and 4-7 of
// the lane group's 8) give a lane the same 8 k of its m that a ds_read_b128
// gives from a K-contiguous tile, and the swizzle spreads the 16 rows each
// read touches over distinct banks (0 SQ_LDS_BANK_CONFLICT, measured).
// Columns past M or N read neighbouring data or, past the buffer's end,
// zeros; their products only reach unstored outputs.  With both operands
// M/N-contiguous, K may be any multiple of 8: k-rows past K lie beyond both
// buffers' bounds and read as zeros, so they add nothing.
//
// Schedule per slice t (group 0 between barriers 2t and 2t+1, group 1 one
// barrier later): at even t each wave issues its loads of pair t/2 + 1 into
// the other stage, whose last slice (t-1) both groups finished reading before
// barrier 2t; before the barrier that precedes slice t+2, every wave waits
// for its own loads of that pair (vmcnt(0): nothing newer is in flight).
// Fragment reads are inline-asm ds_read_b128 (see ds_read16), ordered by
// these explicit waits.
//
// Epilogue: alpha, bias and activation in registers, each wave stages its
// 128 x 64 result through its own 16 KB of the stage arrays (64-row passes,
// 144-byte pitch) and stores 128-byte row segments with 16-byte lanes.
//
// Persistent tiles (PERSIST, K-contiguous A, B either way, batch 1): one
// workgroup per CU walks a list of jobs — whole tiles in rounds of
// gridDim.x, then at most one part of a split tail tile.  The k-pair stream
// runs on across jobs: in the last pair of a job, the even step loads the
// next job's first pair into the stage that pair KP - 2 has left (the same
// rule as inside a job), so that load's latency hides under the job's last
// two slices and its epilogue.  The epilogue stages through stage 1 only
// (32-row passes) while stage 0 receives the next job's first pair; a
// workgroup barrier after it frees stage 1 for the next job's second pair.
// The split tail places every part of a tile on one XCD (tail tile t on XCD
// t % 8, parts on consecutive workgroups of that XCD), so the partial-sum
// hand-off goes through that XCD's L2 without write-back or invalidate.  The
// parts of a tile are resident together, so they share the final sum: each
// sums and stores its own slice of the tile's rows (split_handoff_shared)
// instead of one part reading every partial through one CU.
#pragma once

#include "gemm16.hpp"

namespace sf {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

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

// ds_read_b64 of 8 bytes at LDS byte address `addr` + OFF (as ds_read16).
template <int OFF>
__device__ __forceinline__ u32x2 ds_read8v(uint32_t addr) {
  u32x2 v;
  asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}

// ds_write_b128 of a lane's 16 bytes at LDS byte address `addr` + OFF, as
// inline assembly, so it stays in program order with the ds_read16 reads
// (LDS runs one wave's accesses in issue order).
template <int OFF>
__device__ __forceinline__ void ds_write16(uint32_t addr, u32x4 v) {
  asm volatile("ds_write_b128 %0, %1 offset:%2" : : "v"(addr), "v"(v), "i"(OFF));
}

// ds_read_b64_tr_b16 as inline assembly (as ds_read16): within each 16-lane
// group, lane 4a + b receives element b of the 8-byte rows addressed by
// lanes a, 4 + a, 8 + a and 12 + a (measured lane layout).
template <int OFF>
__device__ __forceinline__ u32x2 ds_read_tr16(uint32_t addr) {
  u32x2 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}

// Orders a wave's LDS writes before its later LDS reads of other lanes'
// data (and the reads before later writes).  A wave's LDS instructions
// execute in issue order, so this only has to stop the compiler from
// moving accesses across it; no workgroup barrier is needed for data that
// never leaves the wave.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] |
// lgkmcnt[11:8] | vmcnt[5:4] << 14); counts not being waited on are at max.
constexpr int waitcnt_imm(int vm, int lgkm) {
  return (vm & 15) | (7 << 4) | ((lgkm & 15) << 8) | (((vm >> 4) & 3) << 14);
}

// NSTAGE = 2, the pipelined kernel above: K % 128 == 0.  (K == 64 runs
// gemm16nt_k64_kernel, which holds four workgroups per CU.)
template <typename TIn, typename TOut, int NSTAGE = 2, bool A_KM = true, bool B_KM = true, bool PERSIST = false,
          bool SHARED = false>
__global__ __launch_bounds__(512) void gemm16nt_pp_kernel(GemmParams p) {
  static_assert(NSTAGE == 2, "two pair stages (K == 64 runs gemm16nt_k64_kernel)");
  static_assert(!PERSIST || A_KM, "persistent tiles: K-contiguous A");
  static_assert(!SHARED || PERSIST, "a shared split sum needs the persistent grid");
  constexpr int BM = 256, BN = 256, BK = 32;
  constexpr int WM = 128, WN = 64, FM = WM / 16, FN = WN / 16;
  constexpr int OP_BYTES = BM * 2 * BK * 2;  // 32 KB: one operand, two slices
  constexpr int DMA_I = 4;                   // per operand per wave per slice pair
  __shared__ __attribute__((aligned(1024))) uint8_t sA0[OP_BYTES], sB0[OP_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t sA1[OP_BYTES], sB1[OP_BYTES];
  // The tile's 256 bias values, loaded with its first k-pair (two areas:
  // the persistent kernel loads the next job's while this one's is in use).
  __shared__ __attribute__((aligned(16))) uint16_t sBias[2][BN];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2;
  const int wm = wave >> 2;
  const int wn = wave & 3;

  const int M = p.M, N = p.N, K = p.K;
  // With two M/N-contiguous operands K need not be a multiple of 128: the
  // loop runs to the next multiple and the k-rows past K read as zeros
  // through both buffers' bounds.
  const int KU = (K + 4 * BK - 1) / (4 * BK);  // 128-k units
  // A job: one output tile (pid), its k slices [t_begin, t_begin + KT) and,
  // in a split tile, its part index (-1: whole tile) and split tile index.
  struct Job {
    int m0, n0, t_begin, KT, part, split_tile;
  };
  const int xcd = blockIdx.x % kNumXcd, xo = blockIdx.x / kNumXcd;
  auto make_job = [&](int pid, int q, int st, Job& jb) {
    int tm, tn;
    group_tile(pid, p.tiles_m, p.tiles_n, 8, tm, tn);
    jb.m0 = tm * BM;
    jb.n0 = tn * BN;
    jb.part = q;
    jb.split_tile = st;
    if (q >= 0) {
      const int u0 = q * KU / p.split, u1 = (q + 1) * KU / p.split;
      jb.t_begin = 4 * u0;
      jb.KT = 4 * (u1 - u0);
    } else {
      jb.t_begin = 0;
      jb.KT = 4 * KU;
    }
  };
  // Job k of this workgroup; false when it has fewer jobs.
  //  PERSIST: the grid is one workgroup per CU (a multiple of 8).  Round r
  //   of the whole tiles is tile r * grid + slot (each XCD a contiguous
  //   range of 32 tile ids per round).  With a split tail, the R leftover
  //   tiles follow: tail tile t runs on XCD t % 8, as split parts on
  //   consecutive workgroups of that XCD, so every part of a tile shares one
  //   L2 (the partial-sum hand-off then needs no L2 write-back).
  //  otherwise: one job per workgroup; split tails as before (whole tiles
  //   first, then each XCD's share of the parts).
  const int n_tiles = p.tiles_m * p.tiles_n;
  auto job_at = [&](int k, Job& jb) -> bool {
    if constexpr (PERSIST) {
      const int G = (int)gridDim.x;
      const int slot = xcd * (G / kNumXcd) + xo;
      const int whole = p.split > 0 ? p.full_tiles : n_tiles;
      const int nr = (whole + G - 1) / G;
      if (k < nr) {
        const int pid = k * G + slot;
        if (pid >= whole) return false;
        make_job(pid, -1, 0, jb);
        return true;
      }
      if (p.split <= 0 || k > nr) return false;
      const int t = (xo / p.split) * kNumXcd + xcd;
      if (t >= n_tiles - p.full_tiles) return false;
      make_job(p.full_tiles + t, xo % p.split, t, jb);
      return true;
    } else {
      if (k > 0) return false;
      if (p.split > 0) {
        // Every XCD gets the same share of whole tiles (a contiguous range,
        // as xcd_remap gives) followed by its share of split parts, so the
        // XCDs finish together; within an XCD the long jobs come first.
        const int fx = p.full_tiles / kNumXcd;  // full_tiles is a multiple of the CU count
        const int P = (n_tiles - p.full_tiles) * p.split;
        if (xo < fx) {
          make_job(xcd * fx + xo, -1, 0, jb);
        } else {
          const int spid = xcd * (P / kNumXcd) + (xcd < P % kNumXcd ? xcd : P % kNumXcd) + (xo - fx);
          make_job(p.full_tiles + spid / p.split, spid % p.split, spid / p.split, jb);
        }
      } else {
        make_job(xcd_remap(blockIdx.x, gridDim.x), -1, 0, jb);
      }
      return true;
    }
  };
  Job cur, nxt;
  if (!job_at(0, cur)) return;  // workgroup-uniform: no work at all
  int jk = 0;
  bool has_next = job_at(1, nxt);
  int m0 = cur.m0, n0 = cur.n0;
  int t_begin = cur.t_begin, KT = cur.KT, part = cur.part, split_tile = cur.split_tile;
  const int64_t b = blockIdx.y;
  const uint16_t* __restrict__ A = static_cast<const uint16_t*>(p.A) + b * p.sA;
  const uint16_t* __restrict__ B = static_cast<const uint16_t*>(p.B) + b * p.sB;
  int KP = KT / 2;  // slice pairs (KT a multiple of 4)

  // A pair stage holds 64 k-columns: line r (128 B) is row r's 64 k values,
  // logical 16-byte chunk h (k = 8h .. 8h+7) at slot h ^ (r & 7).  Slice 2s
  // of the pair is chunks 0-3, slice 2s+1 chunks 4-7.  Direct loads fetch
  // whole 128-byte rows: instruction i of this wave fills lines wave*32 +
  // 8 i .. +7, lane l line + (l >> 3), slot l & 7, i.e. chunk (l&7)^(l>>3).
  // An M/N-contiguous operand: instruction i fills rows 8 wave .. +7 of
  // block i (stage bytes i * 8192 + wave * 1024 ..), lane l row
  // 8 wave + (l >> 3), slot l & 7, i.e. chunk (l & 7) ^ fmn(8 wave + (l >> 3)).
  const int dh = (lane & 7) ^ (lane >> 3);
  const uint32_t dchunk_b = (uint32_t)(dh * 16);
  const int drow = wave * 32 + (lane >> 3);
  const int mrow = wave * 8 + (lane >> 3);  // k-row of an M/N-contiguous operand
  const int mch = (lane & 7) ^ (2 * ((mrow >> 1) & 1) + 4 * ((mrow >> 3) & 1));
  // Buffer resources over A's and B's rows of this batch; per-lane 32-bit
  // row offsets (rows past M / N clamped to the last row: their products
  // only reach unstored outputs) are fixed for the whole loop, the k offset
  // goes in the scalar offset.  Every byte read lies below rows * ld * 2.
  const uint32_t a_rows = A_KM ? (uint32_t)M : (uint32_t)K;
  const uint32_t b_rows = B_KM ? (uint32_t)N : (uint32_t)K;
  const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(
      (void*)A, (short)0, (int)(a_rows * (uint32_t)p.lda * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc(
      (void*)B, (short)0, (int)(b_rows * (uint32_t)p.ldb * 2u), 0x00020000);
  // Bias: waves 0 and 1 each move 128 values (lane l: one dword, two
  // values) straight into the job's bias area beside its first k-pair, so
  // the epilogue reads them from LDS instead of waiting on global loads
  // after the main loop (1.6 us at 4096^3, measured).  The buffer's bound is
  // N values: columns past N read zero (their outputs are not stored).  An
  // even N keeps every dword either inside or outside that bound; an odd N
  // loads the bias in the epilogue as before, and so does the NN layout
  // (dX = dY W has no bias; the persistent NN kernel has no registers to
  // spare for the next job's bias area).
  const bool bias_lds = B_KM && epi_has_bias(p.epi) && (N & 1) == 0;
  const __amdgpu_buffer_rsrc_t rBias = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(p.bias), (short)0, (int)((uint32_t)N * 2u), 0x00020000);
  auto bias_dma = [&](int bn0, int area) {
    if (bias_lds && wave < 2)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rBias, (lds_ptr_t)(reinterpret_cast<uint8_t*>(&sBias[area][0]) + wave * 256),
                                               4, (uint32_t)(bn0 + wave * 128) * 2u + (uint32_t)lane_id_fresh() * 4u, 0,
                                               0, 0);
  };
  // An M/N-contiguous operand needs one per-lane offset: instruction i
  // reads 64 columns (128 bytes) further, through the instruction's
  // immediate offset.  That offset also moves the LDS destination, so the
  // LDS base handed to the instruction is lowered by the same amount.
  uint32_t voa[A_KM ? DMA_I : 1], vob[B_KM ? DMA_I : 1];
  if constexpr (A_KM) {
#pragma unroll
    for (int i = 0; i < DMA_I; ++i) {
      const int ga = m0 + drow + i * 8;
      voa[i] = (uint32_t)(ga < M ? ga : M - 1) * (uint32_t)p.lda * 2u + dchunk_b;
    }
  } else {
    voa[0] = ((uint32_t)mrow * (uint32_t)p.lda + (uint32_t)(m0 + mch * 8)) * 2u;
  }
  if constexpr (B_KM) {
#pragma unroll
    for (int i = 0; i < DMA_I; ++i) {
      const int gb = n0 + drow + i * 8;
      vob[i] = (uint32_t)(gb < N ? gb : N - 1) * (uint32_t)p.ldb * 2u + dchunk_b;
    }
  } else {
    vob[0] = ((uint32_t)mrow * (uint32_t)p.ldb + (uint32_t)(n0 + mch * 8)) * 2u;
  }
  // The next job's offsets (persistent kernel: K-contiguous A; B either
  // way).  Only the persistent kernel re-points the offsets; the one-job
  // kernels keep the straight-line set-up above (written through this
  // lambda, the both-M/N-contiguous kernel spilled two offsets to scratch).
  // The lane's row and chunk indices are recomputed from a fresh lane id
  // here, not kept live across the main loop (with an M/N-contiguous B
  // they would spill).
  auto set_offsets = [&](int am0, int bn0) {
    if constexpr (PERSIST) {
      const int fl = lane_id_fresh();
      const int frow = wave * 32 + (fl >> 3);
      const uint32_t fch = (uint32_t)(((fl & 7) ^ (fl >> 3)) * 16);
#pragma unroll
      for (int i = 0; i < DMA_I; ++i) {
        const int ga = am0 + frow + i * 8;
        voa[i] = (uint32_t)(ga < M ? ga : M - 1) * (uint32_t)p.lda * 2u + fch;
      }
      if constexpr (B_KM) {
#pragma unroll
        for (int i = 0; i < DMA_I; ++i) {
          const int gb = bn0 + frow + i * 8;
          vob[i] = (uint32_t)(gb < N ? gb : N - 1) * (uint32_t)p.ldb * 2u + fch;
        }
      } else {
        const int fmrow = wave * 8 + (fl >> 3);
        const int fmch = (fl & 7) ^ (2 * ((fmrow >> 1) & 1) + 4 * ((fmrow >> 3) & 1));
        vob[0] = ((uint32_t)fmrow * (uint32_t)p.ldb + (uint32_t)(bn0 + fmch * 8)) * 2u;
      }
    }
  };
  // With an M/N-contiguous operand beside it, a K-contiguous operand keeps
  // only its first row offset live and adds the 8-row steps at issue time
  // (the empty asm hides the value's invariance from loop hoisting): the
  // kernel then fits in 256 VGPRs without spills.
  constexpr bool LEAN = !(A_KM && B_KM) || PERSIST;
  auto dma_op = [&](auto km_c, const __amdgpu_buffer_rsrc_t& rs, uint8_t* st, uint32_t* vo, int so, uint32_t step8) {
    constexpr bool KMJ = decltype(km_c)::value;
    if constexpr (KMJ && LEAN) asm volatile("" : "+v"(vo[0]));
    static_for<DMA_I>([&](auto i_c) {
      constexpr int I = decltype(i_c)::value;
      if constexpr (KMJ && LEAN)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(st + wave * 4096 + I * 1024), 16,
                                                 vo[0] + (uint32_t)I * step8, so, 0, 0);
      else if constexpr (KMJ)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(st + wave * 4096 + I * 1024), 16, vo[I], so, 0, 0);
      else  // the k-row offset goes in the lane offset, so the buffer's bound
            // check covers it: columns past the last row's end read zeros.
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(st + wave * 1024 + I * (8192 - 128)), 16,
                                                 vo[0] + (uint32_t)so, 0, I * 128, 0);
    });
  };
  auto dma_at = [&](uint8_t* sA, uint8_t* sB, int kk) {  // kk: first k of the pair
    dma_op(std::integral_constant<bool, A_KM>{}, rA, sA, voa, A_KM ? kk * 2 : kk * (int)p.lda * 2,
           (uint32_t)p.lda * 16u);
    dma_op(std::integral_constant<bool, B_KM>{}, rB, sB, vob, B_KM ? kk * 2 : kk * (int)p.ldb * 2,
           (uint32_t)p.ldb * 16u);
  };
  auto dma = [&](uint8_t* sA, uint8_t* sB, int k0) { dma_at(sA, sB, t_begin * BK + k0); };

  f32x4 acc[FN][FM];
  u32x4 ya[FM], xb[FN];

  // Fragment byte offsets for slice half 0 of a K-contiguous operand: A
  // block j reads lines wm*128 + 16 j + (l & 15), chunk l >> 4; B block i
  // lines wn*64 + 16 i + (l & 15).  Half 1 reads chunk 4 + (l >> 4): its
  // slot differs in bit 2 (byte bit 6).
  const int fa = (wm * 128 + (lane & 15)) * 128 + (((lane >> 4) ^ (lane & 7)) << 4);
  const int fb = (wn * 64 + (lane & 15)) * 128 + (((lane >> 4) ^ (lane & 7)) << 4);
  // M/N-contiguous operand, lane l = 16 g + 4 e + a: the transposing read
  // of 8 bytes at k-row 8 g + e (+ 4 for k 4-7, + 32 for the second slice),
  // columns 16 j + 4 a .. + 3, i.e. chunk 2 j + (a >> 1) at slot
  // (2 j + (a >> 1)) ^ fmn(k); fmn of these rows is 2 ((e >> 1) & 1) +
  // 4 (g & 1) for every half and slice, so fragment j' = j % 4 is the base
  // address with (j' << 5) xor-ed in, and j / 4 selects the 8 KB block.
  const int mn_g = lane >> 4, mn_e = (lane >> 2) & 3, mn_a = lane & 3;
  const int mn_f = 2 * ((mn_e >> 1) & 1) + 4 * (mn_g & 1);
  const int fmn = (8 * mn_g + mn_e) * 128 + ((mn_f | (mn_a >> 1)) << 4) + (mn_a & 1) * 8;
  const int fa_mn = (2 * wm) * 8192 + fmn;  // A: blocks 2 wm, 2 wm + 1
  const int fb_mn = wn * 8192 + fmn;        // B: block wn

  // One fragment of a K-contiguous operand (one ds_read_b128) or of an
  // M/N-contiguous one (two transposing reads, k 0-3 then 4-7).
  auto frag_km = [&](auto j_c, uint32_t base) -> u32x4 {
    constexpr int J = decltype(j_c)::value;
    return ds_read16<J * 2048>(base);
  };
  auto frag_mn = [&](auto j_c, uint32_t base) -> u32x4 {
    constexpr int J = decltype(j_c)::value;
    const uint32_t ad = base ^ (uint32_t)((J & 3) << 5);
    const u32x2 lo = ds_read_tr16<(J >> 2) * 8192>(ad);
    const u32x2 hi = ds_read_tr16<(J >> 2) * 8192 + 512>(ad);
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  };

  auto step = [&](int t, const uint8_t* sA, const uint8_t* sB, uint8_t* nA, uint8_t* nB, auto nxt_c) {
    constexpr bool NXT = decltype(nxt_c)::value;  // load the next tile's first pair
    const bool odd = t & 1;  // static after unrolling
    // memory phase
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t la = A_KM ? lds_addr(sA) + (odd ? (fa ^ 64) : fa) : lds_addr(sA) + fa_mn + (odd ? 4096 : 0);
    const uint32_t lb = B_KM ? lds_addr(sB) + (odd ? (fb ^ 64) : fb) : lds_addr(sB) + fb_mn + (odd ? 4096 : 0);
    static_for<FM>([&](auto j_c) {
      if constexpr (A_KM) ya[decltype(j_c)::value] = frag_km(j_c, la);
      else ya[decltype(j_c)::value] = frag_mn(j_c, la);
    });
    static_for<FN>([&](auto i_c) {
      if constexpr (B_KM) xb[decltype(i_c)::value] = frag_km(i_c, lb);
      else xb[decltype(i_c)::value] = frag_mn(i_c, lb);
    });
    // Even t: the other pair stage was last read in step t-1, which both
    // groups finished before this phase; fill it with pair t/2 + 1.
    if constexpr (NXT) {
      // last pair of this tile: the next tile's first pair goes into the
      // stage whose slices (pair KP - 2) every wave has finished reading
      set_offsets(nxt.m0, nxt.n0);
      dma_at(nA, nB, nxt.t_begin * BK);
      bias_dma(nxt.n0, (jk + 1) & 1);
    } else {
      if (!odd && t / 2 + 1 < KP) dma(nA, nB, (t + 2) * BK);
    }
    // Before step t+1 may read: if t+1 starts a new pair, this wave's loads of
    // that pair (issued in step t-1, nothing later yet) have landed.
    if (grp == 1 && odd)
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
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
    if (grp == 0 && odd) __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 63));
    __builtin_amdgcn_s_barrier();
  };

  dma(sA0, sB0, 0);
  bias_dma(n0, 0);
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
  __builtin_amdgcn_s_barrier();
  for (;;) {
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (grp == 1) __builtin_amdgcn_s_barrier();
  constexpr std::false_type no_c{};
  {
    if (PERSIST && has_next) {
      for (int t = 0; t < KT - 4; t += 4) {
        step(t + 0, sA0, sB0, sA1, sB1, no_c);
        step(t + 1, sA0, sB0, sA1, sB1, no_c);
        step(t + 2, sA1, sB1, sA0, sB0, no_c);
        step(t + 3, sA1, sB1, sA0, sB0, no_c);
      }
      step(KT - 4, sA0, sB0, sA1, sB1, no_c);
      step(KT - 3, sA0, sB0, sA1, sB1, no_c);
      step(KT - 2, sA1, sB1, sA0, sB0, std::true_type{});
      step(KT - 1, sA1, sB1, sA0, sB0, no_c);
    } else {
      for (int t = 0; t < KT; t += 4) {
        step(t + 0, sA0, sB0, sA1, sB1, no_c);
        step(t + 1, sA0, sB0, sA1, sB1, no_c);
        step(t + 2, sA1, sB1, sA0, sB0, no_c);
        step(t + 3, sA1, sB1, sA0, sB0, no_c);
      }
    }
  }
  if (grp == 0) __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);

  // The lane index is recomputed here rather than kept live across the
  // main loop: with two M/N-contiguous operands the loop needs every
  // register, and a value held across it would be spilled to scratch.
  const int elane = lane_id_fresh();

  // ---- split tile: park the partial, then sum the parts ----------------------
  // Partials move with plain 16-byte stores and loads.  Each thread waits
  // for its own stores (vmcnt 0) before the workgroup barrier.
  // One workgroup per tile: the counter increment after the barrier is an
  // agent-scope release and acquire (split_arrive), so the part that sees
  // count split - 1 reads every other part's data as written, and sums all
  // of them.
  // Persistent with SHARED: all parts of a tile are resident together, so
  // the final sum is shared (split_handoff_shared): slice q is the 16-row
  // blocks j with j % split == q of every wave, each summed and stored by
  // one part.  `own` holds the row blocks this part sums and stores.
  // Persistent without SHARED: the last part sums all (split_arrive_xcd).
  int own = (1 << FM) - 1;
  if constexpr (SHARED) {
    if (part >= 0) {
      const int tid = wave * 64 + elane;
      float* mine = p.ws + (size_t)(split_tile * p.split + part) * (FN * FM * 512 * 4);
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
          *reinterpret_cast<f32x4*>(mine + (size_t)((i * FM + j) * 512 + tid) * 4) = acc[i][j];
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      __shared__ int slices;
      if (tid == 0)
        slices = split_handoff_shared(p.counters + 3 * split_tile, p.split, part, (xcd + p.xcd_shift) & (kNumXcd - 1),
                                      p.arrive_spins);
      __syncthreads();
      const int sl = slices;  // workgroup-uniform
      if (sl == 0) return;
      own = 0;
#pragma unroll
      for (int j = 0; j < FM; ++j)
        if ((sl >> (j % p.split)) & 1) own |= 1 << j;
      // Sum each owned block over the parts in part order (the same bits
      // whichever part sums it), every part read back from the workspace.
      // Blocks of other slices are zeroed: staged by the epilogue, never
      // stored, and no accumulator stays live across the sums.
      const float* all = p.ws + (size_t)split_tile * p.split * (FN * FM * 512 * 4) + (size_t)tid * 4;
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        if ((own >> j) & 1) {
          f32x4 sum[FN];
#pragma unroll
          for (int i = 0; i < FN; ++i) sum[i] = f32x4{0.f, 0.f, 0.f, 0.f};
          for (int q = 0; q < p.split; ++q) {
            f32x4 v[FN];
#pragma unroll
            for (int i = 0; i < FN; ++i)
              v[i] = *reinterpret_cast<const f32x4*>(all + ((size_t)(q * FN + i) * FM + j) * 512 * 4);
#pragma unroll
            for (int i = 0; i < FN; ++i) sum[i] += v[i];
          }
#pragma unroll
          for (int i = 0; i < FN; ++i) acc[i][j] = sum[i];
        } else {
#pragma unroll
          for (int i = 0; i < FN; ++i) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
  } else if (part >= 0) {
    const int tid = wave * 64 + elane;
    float* mine = p.ws + (size_t)(split_tile * p.split + part) * (FN * FM * 512 * 4);
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j)
        *reinterpret_cast<f32x4*>(mine + (size_t)((i * FM + j) * 512 + tid) * 4) = acc[i][j];
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    __shared__ int arrived;
    if (tid == 0)
      arrived = PERSIST ? split_arrive_xcd(&p.counters[split_tile], p.split, (xcd + p.xcd_shift) & (kNumXcd - 1))
                        : split_arrive(&p.counters[split_tile], p.split);
    __syncthreads();
    if (arrived != p.split - 1) return;  // workgroup-uniform
    // Sum the parts in part order (the same bits whichever part is last),
    // one B block (8 fragments, 8 16-byte loads in flight) per round trip.
    const float* all = p.ws + (size_t)split_tile * p.split * (FN * FM * 512 * 4);
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      f32x4 sum[FM];
#pragma unroll
      for (int j = 0; j < FM; ++j) sum[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      // Every part, this one included, is read back from the workspace: one
      // straight-line loop, the same additions whichever part is last.
      for (int q = 0; q < p.split; ++q) {
        const float* src = all + ((size_t)q * (FN * FM) + i * FM) * 512 * 4 + (size_t)tid * 4;
        f32x4 v[FM];
#pragma unroll
        for (int j = 0; j < FM; ++j) v[j] = *reinterpret_cast<const f32x4*>(src + (size_t)j * 512 * 4);
#pragma unroll
        for (int j = 0; j < FM; ++j) sum[j] += v[j];
      }
#pragma unroll
      for (int j = 0; j < FM; ++j) acc[i][j] = sum[j];
    }
    if (tid == 0) __hip_atomic_store(&p.counters[split_tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
  }

  // ---- epilogue ------------------------------------------------------------
  const bool has_bias = epi_has_bias(p.epi);
  const int act = epi_act(p.epi);
  const float alpha = p.alpha;
  float bv[FN][4];
  if (bias_lds) {
    // every wave passed a vmcnt(0) wait after the job's first pair (and its
    // bias) was issued; an inline-asm read carries no wait for the next
    // job's loads in flight
    const uint32_t ba = lds_addr(&sBias[jk & 1][0]) + (uint32_t)(wn * WN + 4 * (elane >> 4)) * 2u;
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
      if (has_bias) load_bias4<TIn>(p.bias, n0 + wn * WN + i * 16 + 4 * (elane >> 4), N, bv[i]);
    }
  }
  constexpr int PITCH = WN * 2 + 16;             // 144 bytes
  constexpr int ROWS_S = !PERSIST ? 64 : 32;  // 9216 / 4608 B per pass and wave
  uint8_t* stage;
  if constexpr (PERSIST) {
    // stage 0 is receiving the next tile's first pair: stage 1 only
    stage = ((wave >> 2) ? sB1 : sA1) + (wave & 3) * (ROWS_S * PITCH);
  } else {
    switch (wave >> 1) {
      case 0: stage = sA0; break;
      case 1: stage = sB0; break;
      case 2: stage = sA1; break;
      default: stage = sB1; break;
    }
    stage += (wave & 1) * (OP_BYTES / 2);
  }
  constexpr int LANES_ROW = WN * 2 / 16;
  constexpr int ROWS_I = 64 / LANES_ROW;
  static_assert(16 % ROWS_I == 0, "a store's rows lie in one 16-row block");
  uint16_t* C = static_cast<uint16_t*>(p.C) + b * p.sC;
  const bool vec_ok = ((p.ldc & 7) == 0) && ((reinterpret_cast<uintptr_t>(C) & 15) == 0);
  // Residual: read in the accumulator layout (4 consecutive columns of one
  // row per lane, as raw 16-bit pairs) and added before the single
  // rounding.  With a K-contiguous B (the forward products, where the
  // residual is used) each pass's residual is loaded one pass ahead, the
  // first pass's before the epilogue's first barrier, so only that one
  // load's latency is exposed per tile instead of one per pass (R may alias
  // C, which keeps the compiler from hoisting them itself; measured on
  // 17776 x 1920 x 1920 bf16: the residual cost 22 us of 146 loaded in
  // each pass).  With a k-major B the registers are not there, and each
  // pass loads its own.  R may be C: the passes cover disjoint rows, so
  // every element of R is still read before the pass that stores it.
  const uint16_t* R = p.res != nullptr ? static_cast<const uint16_t*>(p.res) + b * p.sR : nullptr;
  const bool rvec = R != nullptr && res_vec_ok<TOut>(R, p.ldr);
  constexpr int NPASS = WM / ROWS_S;
  constexpr int RB = ROWS_S / 16;  // row blocks per pass
  constexpr bool RES_AHEAD = B_KM;
  // Rows past M read row M - 1 (their sums are not stored), columns past N
  // read as zero.
  auto rload = [&](int ps, u32x2 (&rw)[RB][FN]) {
#pragma unroll
    for (int jj = 0; jj < RB; ++jj) {
      const int gm = m0 + wm * WM + (ps * RB + jj) * 16 + (elane & 15);
      const uint16_t* rrow = R + (int64_t)(gm < M ? gm : M - 1) * p.ldr;
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        const int n = n0 + wn * WN + i * 16 + 4 * (elane >> 4);
        if (rvec && n + 3 < N) {
          rw[jj][i] = *reinterpret_cast<const u32x2*>(rrow + n);
        } else {
          uint32_t h[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) h[q] = n + q < N ? rrow[n + q] : 0u;
          rw[jj][i] = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
        }
      }
    }
  };
  // MASKED: a part of a shared split sum, which stores only its own row
  // blocks; whole tiles compile without that test.
  auto epilogue = [&](auto masked_c) {
  constexpr bool MASKED = decltype(masked_c)::value;
  with_act(act, [&](auto act_c) {
  constexpr int ACT = decltype(act_c)::value;
  u32x2 rcur[RB][FN];
  if constexpr (RES_AHEAD)
    if (R != nullptr) rload(0, rcur);
#pragma unroll
  for (int ps = 0; ps < NPASS; ++ps) {
    u32x2 rnext[RB][FN];
    if constexpr (RES_AHEAD)
      if (R != nullptr && ps + 1 < NPASS) rload(ps + 1, rnext);
    // A part of a shared split sum skips passes without a row block of its
    // own (workgroup-uniform); a workgroup barrier has already followed the
    // main loop there.
    if constexpr (MASKED)
      if (((own >> (ps * (ROWS_S / 16))) & ((1 << (ROWS_S / 16)) - 1)) == 0) {
        if constexpr (RES_AHEAD)
#pragma unroll
          for (int jj = 0; jj < RB; ++jj)
#pragma unroll
            for (int i = 0; i < FN; ++i) rcur[jj][i] = rnext[jj][i];
        continue;
      }
    // The staging region is private to this wave: only the first pass
    // waits for the other waves (their last fragment reads of the main loop
    // may touch it); later passes order this wave's own LDS accesses.
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
          if constexpr (RES_AHEAD) {
            const u32x2 rw = rcur[jj][i];
#pragma unroll
            for (int q = 0; q < 4; ++q)
              v[q] += Elem<TOut>::to_f32(static_cast<uint16_t>(rw[q >> 1] >> ((q & 1) * 16)));
          } else {
            const int gm = m0 + wm * WM + j * 16 + (elane & 15);
            if (gm < M) {
              float rr[4];
              Res4<TOut>::load(R, (int64_t)gm * p.ldr, n0 + wn * WN + i * 16 + 4 * (elane >> 4), N, rvec, rr);
#pragma unroll
              for (int q = 0; q < 4; ++q) v[q] += rr[q];
            }
          }
        }
        const uint32_t lo = pack2<TOut>(v[0], v[1]);
        const uint32_t hi = pack2<TOut>(v[2], v[3]);
        *reinterpret_cast<u32x2*>(stage + r * PITCH + (i * 16 + 4 * (elane >> 4)) * 2) = u32x2{lo, hi};
      }
    }
    wave_lds_sync();
    // All of this pass's staged row segments are read first (one LDS wait),
    // then stored.
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
      const u32x4 val = vals[rr];
      // row block of this store, the same for every lane: ROWS_I divides 16
      const bool own_blk = !MASKED || ((own >> ((ps * ROWS_S + rr * ROWS_I) >> 4)) & 1);
      if (own_blk && gm < M) {
        uint16_t* crow = C + (int64_t)gm * p.ldc;
        if (vec_ok && gn + 8 <= N) {
          __builtin_nontemporal_store(val, reinterpret_cast<u32x4*>(crow + gn));
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (gn + e < N) crow[gn + e] = static_cast<uint16_t>(val[e >> 1] >> ((e & 1) * 16));
        }
      }
    }
    if constexpr (RES_AHEAD)
#pragma unroll
      for (int jj = 0; jj < RB; ++jj)
#pragma unroll
        for (int i = 0; i < FN; ++i) rcur[jj][i] = rnext[jj][i];
  }
  });
  };
  if constexpr (SHARED) {
    if (part >= 0)
      epilogue(std::true_type{});
    else
      epilogue(std::false_type{});
  } else {
    epilogue(std::false_type{});
  }
  if (!has_next) break;
  // every wave is done with the staging area (stage 1) before the next
  // tile's second pair is loaded into it; then group 1 drops half a step
  __syncthreads();
  cur = nxt;
  ++jk;
  has_next = job_at(jk + 1, nxt);
  m0 = cur.m0;
  n0 = cur.n0;
  t_begin = cur.t_begin;
  KT = cur.KT;
  KP = KT / 2;
  part = cur.part;
  split_tile = cur.split_tile;
  }
}

}  // namespace sf
