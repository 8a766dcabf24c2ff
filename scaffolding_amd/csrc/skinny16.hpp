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
#include "gemm16nt_pp.hpp"

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
  const void* R = p.res != nullptr ? static_cast<const OutS*>(p.res) + b * p.sR : nullptr;
  const bool rvec = R != nullptr && res_vec_ok<TOut>(R, p.ldr);
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
      if (R != nullptr) {
        float r[4];
        Res4<TOut>::load(R, (int64_t)m * p.ldr, n, N, rvec, r);
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] += r[q];
      }
      Store4<TOut>::run(C + (int64_t)m * p.ldc, n, N, vec_ok, v);
    }
  });
}


// 16-byte global load issued as inline assembly at byte offset OFF, with no
// wait: the caller orders it with an explicit s_waitcnt and then tie2.
template <int OFF>
__device__ __forceinline__ u32x4 gload16_nowait(const void* p) {
  u32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, off offset:%2" : "=v"(v) : "v"(p), "i"(OFF) : "memory");
  return v;
}
// Marks both registers as written here, so no use moves above this point.
__device__ __forceinline__ void tie2(u32x4& a, u32x4& b) { asm volatile("" : "+v"(a), "+v"(b)); }

// skinny16l_kernel — the M <= 16 stream for K = 512 * NW (NW waves), reading
// W in whole 128-byte row segments.
//
//   * Workgroup g owns W rows [g * rows_per, min(N, (g + 1) * rows_per)),
//     rows_per <= 64, in up to four 16-row blocks; wave w owns k in
//     [512 w, 512 w + 512) of every one of those rows.
//   * A tile is 16 rows x 64 k (16 x 128 bytes).  Its two loads
//     (buffer_load_dwordx4 ... lds, rows 0-7 and 8-15) each fetch 8 whole
//     128-byte row segments straight into the wave's private R-tile LDS
//     ring, line r = row r with 16-byte chunk h at slot h ^ (r & 7); rows
//     past the workgroup's last row fall outside the buffer resource and
//     read as zero without touching memory.  R - 1 tiles stay in flight
//     behind the one being folded.
//   * Each tile is two conflict-free ds_read_b128 fragments (k halves) and
//     two v_mfma_f32_16x16x32 with X = W rows, Y = x rows; x's fragments
//     for the wave's 512 k are loaded once into 64 VGPRs.
//   * The NW partial 16x16 blocks are summed through LDS by waves 0..nblk-1,
//     which apply alpha, bias and activation and store their block: lane l
//     holds C[m = l % 16][n = 4 (l / 16) + 0..3].
// Every wave waits only for its own loads (vmcnt) and reads only its own
// ring, so the loop has no barrier.  Requires 16-byte aligned rows.
template <typename TIn, typename TOut, int NW, int R = 4, bool XLINE = true>
__global__ __launch_bounds__(NW * 64) void skinny16l_kernel(GemmParams p) {
  static_assert(R == 4 || R == 8, "the ring depth divides the 8 tiles of a row block");
  constexpr int TILE = 2048;  // 16 rows x 128 bytes
  constexpr int MAXB = 4;     // 16-row blocks per workgroup
  __shared__ __attribute__((aligned(1024))) uint8_t ring[NW][R * TILE];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t b = blockIdx.y;
  const int M = p.M, N = p.N;
  const int r0 = blockIdx.x * p.rows_per;
  const int nrows = (N - r0) < p.rows_per ? (N - r0) : p.rows_per;
  const int nblk = (nrows + 15) >> 4;
  const uint16_t* __restrict__ X = static_cast<const uint16_t*>(p.A) + b * p.sA;
  const uint16_t* W = static_cast<const uint16_t*>(p.B) + b * p.sB + (int64_t)r0 * p.ldb;
  const uint32_t ldb_b = (uint32_t)p.ldb * 2u;
  const __amdgpu_buffer_rsrc_t rW =
      __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, (int)((uint32_t)nrows * ldb_b), 0x00020000);
  const int kw = wave * 512;
  uint8_t* myring = &ring[wave][0];

  // W is read once: non-temporal loads (cache-policy bit "nt") stream it
  // past the caches, measured 6.2-6.3 TB/s against 5.5-5.6 without.
  constexpr int kNonTemporal = 2;
  // Load lane mapping: load ih of a tile fills tile rows 8 ih + (l >> 3),
  // slot l & 7, i.e. chunk (l & 7) ^ (l >> 3) of that row.  The 128-byte
  // line step goes in the scalar offset: an instruction offset would also
  // move the LDS destination.
  const uint32_t vrow = (uint32_t)(lane >> 3) * ldb_b + (uint32_t)kw * 2u +
                        (uint32_t)(((lane & 7) ^ (lane >> 3)) * 16);
  auto issue = [&](int blk, auto Lc) {
    constexpr int L = decltype(Lc)::value;
    uint8_t* dst = myring + (L % R) * TILE;
    const uint32_t v0 = vrow + (uint32_t)(blk * 16) * ldb_b;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rW, (lds_ptr_t)dst, 16, v0, L * 128, 0, kNonTemporal);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rW, (lds_ptr_t)(dst + 1024), 16, v0 + 8u * ldb_b, L * 128, 0,
                                             kNonTemporal);
  };
  // x fragments: slice s (k = kw + 32 s ..) lane l: row m = l & 15, 8 k at
  // kw + 32 s + 8 (l >> 4); rows past M are zero.  XLINE: x arrives a 64-k
  // window (two slices) at a time in whole 128-byte row segments: load 0 of
  // window L brings rows 0-7 (lane l: row l >> 3, chunk (l & 7) ^ (l >> 3)),
  // load 1 rows 8-15, so each load touches 8 cache lines instead of the 16
  // half lines that loads in the MFMA layout touch (M = 16: 16.15 -> 15.85
  // us, measured; at M <= 8 the MFMA-layout loads touch at most 8 lines and
  // skip the round trip through LDS: 0.06 us faster, so !XLINE there).
  // When tile L of the first row block has been read from its ring slot,
  // the window is written there in the W tiles' layout (lane l at slot l & 7
  // of line l >> 3: 16 l bytes, conflict-free) and read back as two MFMA
  // fragments with the W fragment offsets; a wave's LDS accesses run in
  // issue order, so the W reads see the tile and the reads back see the
  // window.  Tile L of the first row block brings its window right after
  // its W loads, so x (16 KB per wave at M = 16) streams beside W instead of
  // holding the load path before W starts.
  // The x loads are inline assembly: the compiler would count only them
  // (not the direct loads between them) when it places its own wait before
  // an MFMA that uses them, and so wait for more W tiles than needed.  The
  // explicit waits below count them, and xtie marks the registers as written
  // after that wait, so nothing reads them earlier.
  u32x4 xf[16];
  const int xm = lane & 15;
  const int xl = XLINE ? lane >> 3 : xm;
  const int xc = XLINE ? (lane & 7) ^ xl : lane >> 4;
  const uint16_t* xr0 = X + (int64_t)(xl < M ? xl : 0) * p.lda + kw + 8 * xc;
  const uint16_t* xr1 = XLINE ? X + (int64_t)(xl + 8 < M ? xl + 8 : 0) * p.lda + kw + 8 * xc : xr0 + 32;
  auto xload = [&](auto Lc) {
    constexpr int L = decltype(Lc)::value;
    xf[2 * L] = gload16_nowait<128 * L>(xr0);
    xf[2 * L + 1] = gload16_nowait<128 * L>(xr1);
  };
  auto xtie = [&](auto Lc) {
    constexpr int L = decltype(Lc)::value;
    tie2(xf[2 * L], xf[2 * L + 1]);
  };
  static_for<R - 1>([&](auto Lc) {
    issue(0, Lc);
    xload(Lc);
  });

  // Fragment offsets inside a tile: row l & 15, chunk 4 h + (l >> 4).
  const int f0 = (lane & 15) * 128 + (((lane >> 4) ^ (lane & 7)) << 4);
  const uint32_t ring_a = lds_addr(myring);

  f32x4 acc[MAXB];
#pragma unroll
  for (int j = 0; j < MAXB; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int T = nblk * 8;  // tiles of this wave
#pragma unroll
  for (int blk = 0; blk < MAXB; ++blk) {
    if (blk < nblk) {
      static_for<8>([&](auto Lc) {
        constexpr int L = decltype(Lc)::value;
        constexpr int LN = (L + R - 1) & 7;
        const int nb = blk + ((L + R - 1) >> 3);
        // The fences keep load issue, waits, LDS reads and MFMAs in program
        // order: the wait counts below count exactly the loads issued above.
        __builtin_amdgcn_sched_barrier(0);
        if (nb < nblk) issue(nb, std::integral_constant<int, LN>{});
        if constexpr (L + R - 1 < 8) {
          if (blk == 0) xload(std::integral_constant<int, L + R - 1>{});
        }
        __builtin_amdgcn_sched_barrier(0);
        // Loads issued after this tile's own: those of the next
        // min(R - 1, T - 1 - t) tiles, two W loads each plus two x loads
        // for tiles of the first row block.
        const int t = blk * 8 + L;
        const int after = T - 1 - t;
        static_for<R>([&](auto Ac) {
          constexpr int AF = decltype(Ac)::value;
          if (AF == R - 1 ? after >= AF : after == AF) {
            if (blk == 0) {
              // tiles t+1 .. t+AF; those below 8 carry x loads
              constexpr int XL = (L + AF < 8 ? AF : (7 - L > 0 ? 7 - L : 0));
              __builtin_amdgcn_s_waitcnt(waitcnt_imm(2 * AF + 2 * XL, 63));
            } else {
              __builtin_amdgcn_s_waitcnt(waitcnt_imm(2 * AF, 63));
            }
          }
        });
        __builtin_amdgcn_sched_barrier(0);
        if (blk == 0) xtie(Lc);
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t slot = ring_a + (L % R) * TILE;
        const uint32_t a = slot + f0;
        const u32x4 w0 = ds_read16<0>(a);       // chunk l >> 4
        const u32x4 w1 = ds_read16<0>(a ^ 64);  // chunk 4 + (l >> 4): slot bit 2 flipped
        if (XLINE && blk == 0) {
          const uint32_t wa = slot + 16 * lane;
          ds_write16<0>(wa, xf[2 * L]);
          ds_write16<1024>(wa, xf[2 * L + 1]);
          xf[2 * L] = ds_read16<0>(a);
          xf[2 * L + 1] = ds_read16<0>(a ^ 64);
        }
        __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
        __builtin_amdgcn_sched_barrier(0);
        if (blk == 0 && xm >= M) xf[2 * L] = xf[2 * L + 1] = u32x4{0u, 0u, 0u, 0u};  // rows past M
        __builtin_amdgcn_sched_barrier(0);
        acc[blk] = Mfma16<TIn>::run(w0, xf[2 * L], acc[blk]);
        acc[blk] = Mfma16<TIn>::run(w1, xf[2 * L + 1], acc[blk]);
      });
    }
  }

  // Cross-wave reduction: each wave parks its blocks in its own ring.
  f32x4* park = reinterpret_cast<f32x4*>(myring);
#pragma unroll
  for (int j = 0; j < MAXB; ++j)
    if (j < nblk) park[j * 64 + lane] = acc[j];
  __syncthreads();
  if (wave >= nblk) return;
  const int blk = wave;
  f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int w = 0; w < NW; ++w) sum += reinterpret_cast<const f32x4*>(&ring[w][0])[blk * 64 + lane];

  typedef typename Elem<TOut>::storage OutS;
  OutS* C = static_cast<OutS*>(p.C) + b * p.sC;
  const int m = lane & 15;
  const int n = r0 + blk * 16 + 4 * (lane >> 4);
  const int n_end = r0 + nrows;
  if (m >= M || n >= n_end) return;
  const bool has_bias = epi_has_bias(p.epi);
  const bool vec_ok = ((p.ldc & 3) == 0) && ((reinterpret_cast<uintptr_t>(C) & 15) == 0);
  float bv[4] = {0.f, 0.f, 0.f, 0.f};
  if (has_bias) load_bias4<TIn>(p.bias, n, n_end, bv);
  float rv[4] = {0.f, 0.f, 0.f, 0.f};
  if (p.res != nullptr) {
    const void* Rb = static_cast<const OutS*>(p.res) + b * p.sR;
    Res4<TOut>::load(Rb, (int64_t)m * p.ldr, n, n_end, res_vec_ok<TOut>(Rb, p.ldr), rv);
  }
  with_act(epi_act(p.epi), [&](auto act_c) {
    constexpr int ACT = decltype(act_c)::value;
    float v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = act_t<ACT>(sum[q] * p.alpha + bv[q]) + rv[q];
    Store4<TOut>::run(C + (int64_t)m * p.ldc, n, n_end, vec_ok, v);
  });
}

}  // namespace sf
