// attention.hpp — fused scaled-dot-product attention forward for head sizes
// up to 64, 16-bit Q/K/V/O with fp32 accumulation:
//
//   O[b] = softmax(scale * Q[b] K[b]^T) V[b],  Q [Sq, D], K, V [Sk, D].
//
// One 256-thread workgroup per 256 query rows of one batch entry; wave w
// owns 64 of them (four 16-row blocks); at most 256 registers per lane, so
// two workgroups share a CU.  The workgroup streams K and V in blocks of 64
// keys through a 3-stage LDS ring (16 KB per stage, loaded two blocks
// ahead), and per block each wave
//   1. forms S = Q K^T for its 64 x 64 scores: 32 v_mfma_f32_16x16x32 with
//      Q fragments held in registers for the whole loop and K fragments
//      read from LDS (ds_read_b128, 128-byte lines, chunk h at slot
//      h ^ (row & 7), conflict-free as in the GEMM kernels);
//   2. keeps the softmax in the exp2 domain against a per-row reference m
//      that is raised lazily: the exponents x = S scale log2 e - m come
//      straight out of the score MFMAs (PRESCALE: Q is multiplied by
//      scale log2 e once per work item, rounded once into T, and each score
//      chain starts from -m as its C operand; otherwise one FMA per score
//      forms x in place), and only when one exceeds 8 does the wave reduce
//      the row maxima across the four lanes sharing a row, raise m and
//      scale O and the row sums by 2^(m_old - m_new), so P = 2^x stays
//      <= 2^8 and the common path needs no cross-lane traffic;
//   3. packs P to 16 bits (v_cvt_pk) and adds P V into the 64 x 64 fp32 O
//      accumulator (32 MFMAs, V fragments from ds_read_b64_tr_b16, gfx950's
//      transposing LDS read) and P 1 into the row sums (8 MFMAs against a
//      fragment of ones, so the sums use the same rounded P as O).
// P's MFMA k slots follow the score accumulator layout (lane group g holds
// keys 4g..4g+3 and 16+4g..16+4g+3 of each 32-key chunk), and the V
// fragment reads use the same key order, so P never moves between lanes.
// The 2 GB score and probability tensors of the three-kernel path are never
// written.  Head size D a multiple of 8 up to 64: the tiles stay 64 wide,
// d past D reads as zeros (adding nothing to Q K^T; O's columns there are
// not stored).  Requires scale > 0 and 16-byte aligned rows; a partial last
// key block is masked.  A work item is one (batch, head) pair's 256 query
// rows, each pair with its own batch and head offsets, so Q/K/V can be read
// in place from a packed [batch, S, 3 * heads * 64] projection and O written
// straight into [batch, Sq, heads * 64] (no head split or merge copies).
//
// Split items.  Workgroups all run equally long, so when the last round of
// them is short (items mod slots small) the launch waits a whole workgroup
// time for a few of them.  The host then runs only the first full_items
// whole and splits each remaining item's key blocks into `parts` contiguous
// ranges, one workgroup each, dispatched after the whole items so they fill
// the last round; such a workgroup writes its unnormalised fp32 O with its
// row references m and row sums l (attn_part_* layout) and a second kernel,
// attn_combine_kernel, merges the parts of each item in part order:
// O = sum_p 2^(m_p - M) O_p / sum_p 2^(m_p - M) l_p, M = max_p m_p.
#pragma once

#include "gemm16nt_pp.hpp"
#include "sf_internal.hpp"

namespace sf {

struct AttnParams {
  const void* Q;
  const void* K;
  const void* V;
  void* O;
  int64_t sQ, sK, sV, sO;      // batch strides, elements
  int64_t hQ, hK, hV, hO;      // head strides, elements
  int64_t item0;               // first work item (or split part) of this launch
  int64_t full_items;          // items [0, full_items) run whole, the rest in parts
  float* ws;                   // split parts' partials, kAttnPartFloats each
  int QB;                      // query blocks of 256 rows per (batch, head) pair
  int parts;                   // key-range parts per split item (0: none)
  int H;                       // heads per batch entry
  int ldq, ldk, ldv, ldo;      // row strides, elements
  int Sq, Sk;
  int D;                       // head size: a multiple of 8, at most 64
  float scale_log2e;           // scale * log2(e), > 0
};

__device__ __forceinline__ float shfl_xor_f(float v, int mask) { return __shfl_xor(v, mask, 64); }

// One split part's partials: O as [wave 4][row block 4][d block 4][lane 64]
// f32x4 (the accumulator layout), then (m, l) as [wave 4][row block 4][lane
// 64] float pairs.
constexpr int kAttnPartOFloats = 4 * 4 * 4 * 64 * 4;
constexpr int kAttnPartFloats = kAttnPartOFloats + 4 * 4 * 64 * 2;
static_assert(kAttnPartFloats * 4 == (int)kAttnPartBytes, "partial layout and the host's size differ");

// A work item's (pair, query block) and, for a split part, its key blocks.
struct AttnItem {
  int64_t b, h;
  int qb;
  int kb0, kb1;  // key blocks [kb0, kb1)
  int64_t part;  // index of the split part among all parts, -1 for a whole item
};
__device__ __forceinline__ AttnItem attn_item(const AttnParams& p, int64_t it, int nb) {
  AttnItem w;
  int64_t item = it;
  w.part = -1;
  w.kb0 = 0;
  w.kb1 = nb;
  if (it >= p.full_items) {
    const int64_t t = it - p.full_items;
    const int64_t q = t / p.parts;
    const int r = (int)(t - q * p.parts);
    item = p.full_items + q;
    w.part = t;
    w.kb0 = (int)((int64_t)nb * r / p.parts);
    w.kb1 = (int)((int64_t)nb * (r + 1) / p.parts);
  }
  const int64_t y = item / p.QB;
  w.qb = (int)(item - y * p.QB);
  w.b = y / p.H;
  w.h = y - w.b * p.H;
  return w;
}

// Normalised output rows of one wave: row block mb's 16 rows from the
// accumulator layout (lane l: query l % 16, d = 16 db + 4 (l / 16) + 0..3),
// columns at or past D not stored.
template <typename T>
__device__ __forceinline__ void attn_store_rows(const AttnParams& p, uint16_t* Ob, int q0, int lane, int mb,
                                                const f32x4 (&o)[4], float l) {
  const float inv = 1.0f / l;
  const int r = q0 + mb * 16 + (lane & 15);
  if (r >= p.Sq) return;
  uint16_t* orow = Ob + (int64_t)r * p.ldo;
#pragma unroll
  for (int db = 0; db < 4; ++db) {
    const int d = db * 16 + 4 * (lane >> 4);
    if (d >= p.D) continue;  // columns past the head size (D % 8 == 0)
    const uint32_t lo = pack2<T>(o[db][0] * inv, o[db][1] * inv);
    const uint32_t hi = pack2<T>(o[db][2] * inv, o[db][3] * inv);
    *reinterpret_cast<u32x2*>(orow + d) = u32x2{lo, hi};
  }
}

// PRESCALE: Q is scaled by scale log2 e in registers (the host takes it
// when scale log2 e <= 1, so |Q scale log2 e| <= |Q| cannot overflow
// fp16).  It removes the 64 FMAs per key block and wave that form the
// exponents, at the cost of one extra rounding of each Q element into T:
// each exponent moves by about 2^-9 (bf16) or 2^-12 (fp16) of the size of
// the products q_d k_d, below P's own rounding for logits of a few units
// and a few times the FMA path's error for logits of tens.
template <typename T, bool PRESCALE>
__global__ __launch_bounds__(256, 2) void attn64_kernel(AttnParams p) {
  constexpr int NS = 3;
  constexpr int KB = 64;
  constexpr int BLK = KB * 128;
  constexpr float THRESH = 8.0f;
  __shared__ __attribute__((aligned(1024))) uint8_t sK[NS][BLK];
  __shared__ __attribute__((aligned(1024))) uint8_t sV[NS][BLK];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int Sq = p.Sq, Sk = p.Sk;
  // Key blocks of 64; a partial last block reads zeros past row Sk (the
  // buffer bound) and its scores there are masked to -inf.
  const int NB = (Sk + KB - 1) / KB;
  const int k_tail = Sk - (NB - 1) * KB;  // valid keys of the last block, 1..64
  const AttnItem wi = attn_item(p, p.item0 + blockIdx.x, NB);
  const int64_t b = wi.b, h = wi.h;
  const int q0 = wi.qb * 256 + wave * 64;
  const int kb0 = wi.kb0, kb1 = wi.kb1;
  const uint16_t* Qb = static_cast<const uint16_t*>(p.Q) + b * p.sQ + h * p.hQ;
  const uint16_t* Kb = static_cast<const uint16_t*>(p.K) + b * p.sK + h * p.hK;
  const uint16_t* Vb = static_cast<const uint16_t*>(p.V) + b * p.sV + h * p.hV;

  const __amdgpu_buffer_rsrc_t rK =
      __builtin_amdgcn_make_buffer_rsrc((void*)Kb, (short)0, (int)((uint32_t)Sk * (uint32_t)p.ldk * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t rV =
      __builtin_amdgcn_make_buffer_rsrc((void*)Vb, (short)0, (int)((uint32_t)Sk * (uint32_t)p.ldv * 2u), 0x00020000);
  const int drow = wave * 16 + (lane >> 3);
  const int hch = (lane & 7) ^ (lane >> 3);  // this lane's 16-byte chunk (8 d) of its rows
  const uint32_t dch = (uint32_t)(hch * 16);
  // Head sizes below 64: chunks at or past D get an offset past the buffer's
  // range (2^31 plus at most the block and row offsets, which stay below
  // 2^31) and so read as zeros.
  const bool dok = 8 * hch < p.D;
  const uint32_t vk0 = dok ? (uint32_t)drow * (uint32_t)p.ldk * 2u + dch : 0x80000000u;
  const uint32_t vv0 = dok ? (uint32_t)drow * (uint32_t)p.ldv * 2u + dch : 0x80000000u;
  const uint32_t k8 = 8u * (uint32_t)p.ldk * 2u, v8 = 8u * (uint32_t)p.ldv * 2u;
  // The block's row offset goes in the per-lane offset, not the scalar
  // offset: the buffer's range check covers only the per-lane offset (plus
  // the immediate), so rows at or past Sk then read as zeros instead of
  // whatever lies beyond the last key (the host keeps (Sk + 64) * ld * 2
  // below 2^31, so the 32-bit sum cannot wrap).
  auto issue = [&](int j) {
    const int s = j % NS;
    const uint32_t ko = (uint32_t)j * (uint32_t)(KB * p.ldk * 2), vo = (uint32_t)j * (uint32_t)(KB * p.ldv * 2);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rK, (lds_ptr_t)(&sK[s][0] + wave * 2048), 16, vk0 + ko, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rK, (lds_ptr_t)(&sK[s][0] + wave * 2048 + 1024), 16, vk0 + k8 + ko, 0, 0,
                                             0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rV, (lds_ptr_t)(&sV[s][0] + wave * 2048), 16, vv0 + vo, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rV, (lds_ptr_t)(&sV[s][0] + wave * 2048 + 1024), 16, vv0 + v8 + vo, 0, 0,
                                             0);
  };
  issue(kb0);
  if (kb0 + 1 < kb1) issue(kb0 + 1);

  u32x4 qf[4][2];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    int r = q0 + mb * 16 + (lane & 15);
    r = r < Sq ? r : Sq - 1;
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      const int d0 = kc * 32 + 8 * (lane >> 4);
      qf[mb][kc] = d0 < p.D ? *reinterpret_cast<const u32x4*>(Qb + (int64_t)r * p.ldq + d0) : u32x4{0u, 0u, 0u, 0u};
    }
  }

  const float sc = p.scale_log2e;
  if constexpr (PRESCALE) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int kc = 0; kc < 2; ++kc)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t w = qf[mb][kc][e];
          qf[mb][kc][e] = pack2<T>(Elem<T>::to_f32((uint16_t)(w & 0xffffu)) * sc,
                                   Elem<T>::to_f32((uint16_t)(w >> 16)) * sc);
        }
  }

  f32x4 o[4][4], osum[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    osum[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int db = 0; db < 4; ++db) o[mb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // -m per row block, all four values equal: the score MFMAs' C operand
  // (PRESCALE) and the FMAs' addend otherwise; set by the first key block
  f32x4 nq[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) nq[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  // 16-bit 1.0 in both halves of every dword: the X fragment of a ones block.
  const uint32_t one2 = (uint32_t)Elem<T>::from_f32(1.0f) * 0x10001u;
  const u32x4 ones = u32x4{one2, one2, one2, one2};

  const uint32_t kfo = (uint32_t)((lane & 15) * 128 + (((lane >> 4) ^ (lane & 7)) << 4));
  const int vs = lane & 15, vg = lane >> 4;
  const int vrow0 = 4 * vg + (vs >> 2);
  const uint32_t vfo_base = (uint32_t)vrow0 * 128u + (uint32_t)((vs & 1) * 8);
  const int vch = (vs & 3) >> 1;
  const int vsw = vrow0 & 7;

  for (int j = kb0; j < kb1; ++j) {
    const int st = j % NS;
    __builtin_amdgcn_sched_barrier(0);
    if (j + 1 < kb1)
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(4, 0));
    else
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if (j + 2 < kb1) issue(j + 2);
    __builtin_amdgcn_sched_barrier(0);

    // ---- S = Q K^T, K fragments per 16-key block ------------------------
    const uint32_t ka = lds_addr(&sK[st][0]) + kfo;
    f32x4 s[4][4];
    u32x4 kf0 = ds_read16<0>(ka), kf1 = ds_read16<0>(ka ^ 64);
    static_for<4>([&](auto nbc) {
      constexpr int NBK = decltype(nbc)::value;
      u32x4 nk0, nk1;
      if constexpr (NBK < 3) {
        nk0 = ds_read16<(NBK + 1) * 2048>(ka);
        nk1 = ds_read16<(NBK + 1) * 2048>(ka ^ 64);
        __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 2));  // this block's pair landed
      } else {
        __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
      }
      __builtin_amdgcn_sched_barrier(0);
      // Independent chains back to back: all kc = 0 products, then kc = 1.
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
        s[mb][NBK] = Mfma16<T>::run(kf0, qf[mb][0], PRESCALE ? nq[mb] : f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) s[mb][NBK] = Mfma16<T>::run(kf1, qf[mb][1], s[mb][NBK]);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (NBK < 3) {
        kf0 = nk0;
        kf1 = nk1;
      }
    });

    // ---- V fragments of the whole block (16 transposing reads) -----------
    // Issued now, so they land while the row maxima are formed.
    const uint32_t va = lds_addr(&sV[st][0]) + vfo_base;
    u32x4 vf[4][2];
    __builtin_amdgcn_sched_barrier(0);
    static_for<4>([&](auto dbc) {
      constexpr int DB = decltype(dbc)::value;
      const uint32_t a0 = va + (uint32_t)(((2 * DB + vch) ^ vsw) << 4);
      const u32x2 t00 = ds_read_tr16<0>(a0);
      const u32x2 t01 = ds_read_tr16<16 * 128>(a0);
      const u32x2 t10 = ds_read_tr16<32 * 128>(a0);
      const u32x2 t11 = ds_read_tr16<48 * 128>(a0);
      vf[DB][0] = u32x4{t00.x, t00.y, t01.x, t01.y};
      vf[DB][1] = u32x4{t10.x, t10.y, t11.x, t11.y};
    });
    __builtin_amdgcn_sched_barrier(0);

    // ---- keys past Sk (last block only) ----------------------------------
    // Lane l holds keys 16 nb + 4 (l >> 4) + q of the block; scale > 0, so
    // -inf stays -inf through the scaling and exp2 gives 0.
    if (k_tail < KB && j == NB - 1) {
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (nb * 16 + 4 * (lane >> 4) + q >= k_tail)
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) s[mb][nb][q] = -INFINITY;
    }

    // ---- online softmax with lazy rescale --------------------------------
    // x = s scale log2(e) - m (the exponent of P: the score MFMAs' result
    // with PRESCALE, else one FMA per score in place); each lane checks its
    // 16 values of each row against THRESH.  Only when
    // some value exceeds it, and always in the first key block (which sets m
    // from m = 0, with O and the sums still zero), does the wave reduce the
    // row maxima across the four lanes of each row, raise m by dm, lower x
    // by dm and scale O and the row sums by 2^-dm (the first key block of
    // a split part likewise sets its own m).  Otherwise P = 2^x <=
    // 2^THRESH.
    //
    // fp16 with the FMA (PCHECK): after the first key block the check runs
    // on the packed P instead, three values per v_pk_maximum3_f16 (4
    // instructions per row block instead of 8 v_max3_f32): P > 2^THRESH (as
    // 16-bit patterns, P >= 0) sends that row block through the same raise
    // and recomputes its exponentials before its P V MFMAs.
    constexpr bool PCHECK = std::is_same<T, F16>::value && !PRESCALE;
    const bool first = j == kb0;
    // Otherwise (bf16, and fp16 with PRESCALE) the maxima are checked every
    // key block, with the NaN-propagating maximum (v_maximum3_f32) on the
    // MFMA results as they are, where fmaxf would first quiet possible
    // signalling NaNs (8 fewer VALU instructions per block; a row holding a
    // NaN score is NaN either way).  For fp16 with PRESCALE this measured
    // faster than the packed check, which costs a branch per row block (C4
    // -3.7 %, packed 30-head C5 -1.7 %, A/B in one run); with the FMA the
    // packed check stays ahead (+1.8 % without it).
    auto mx2 = [](float a, float b) {
      if constexpr (PCHECK)
        return fmaxf(a, b);
      else
        return __builtin_elementwise_maximum(a, b);
    };
    auto row_max = [&](int mb) {
      float mx = mx2(mx2(s[mb][0][0], s[mb][0][1]), s[mb][0][2]);
      mx = mx2(mx2(mx, s[mb][0][3]), s[mb][1][0]);
      mx = mx2(mx2(mx, s[mb][1][1]), s[mb][1][2]);
      mx = mx2(mx2(mx, s[mb][1][3]), s[mb][2][0]);
      mx = mx2(mx2(mx, s[mb][2][1]), s[mb][2][2]);
      mx = mx2(mx2(mx, s[mb][2][3]), s[mb][3][0]);
      mx = mx2(mx2(mx, s[mb][3][1]), s[mb][3][2]);
      return mx2(mx, s[mb][3][3]);
    };
    // Raises row block mb's reference by its row maxima (all four lanes of
    // a row), lowers x, and scales O and the row sums.
    auto raise = [&](int mb, float mx) {
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      // the first block sets m to the row maximum (finite: every row has a
      // valid key there); later blocks only raise it
      const float dm = first ? mx : fmaxf(mx, 0.f);
      const float nm = nq[mb][0] - dm;
      nq[mb] = f32x4{nm, nm, nm, nm};
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int q = 0; q < 4; ++q) s[mb][nb][q] -= dm;
      if (!first) {
        const float corr = __builtin_amdgcn_exp2f(-dm);
        osum[mb] *= corr;
#pragma unroll
        for (int db = 0; db < 4; ++db) o[mb][db] *= corr;
      }
    };
    bool need = false;
    float lmx[4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      if constexpr (!PRESCALE) {
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
#pragma unroll
          for (int q = 0; q < 4; ++q) s[mb][nb][q] = __builtin_fmaf(s[mb][nb][q], sc, nq[mb][0]);
      }
      if (!PCHECK || first) {
        lmx[mb] = row_max(mb);
        need |= lmx[mb] > THRESH;
      }
    }
    if (first || (!PCHECK && __builtin_amdgcn_ballot_w64(need) != 0)) {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) raise(mb, lmx[mb]);
    }
    // ---- P = 2^(S scale - m) packed to 16 bits, O += P V, row sums -------
    // Row block mb's exponentials (VALU: 16 exp2, 8 conversions)
    // are interleaved with the MFMAs of row block mb - 1 (8 for P V, 2 for
    // the row sums): the MFMA pipe and the VALU run side by side within
    // the wave instead of one after the other.
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));  // V fragments landed
    __builtin_amdgcn_sched_barrier(0);
    u32x4 pf[4][2];
    auto expo = [&](auto mb_c) {
      constexpr int MB = decltype(mb_c)::value;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        uint32_t w[4];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int q2 = 0; q2 < 2; ++q2) {
            const float e0 = __builtin_amdgcn_exp2f(s[MB][2 * c + hh][2 * q2]);
            const float e1 = __builtin_amdgcn_exp2f(s[MB][2 * c + hh][2 * q2 + 1]);
            w[hh * 2 + q2] = pack2<T>(e0, e1);
          }
        pf[MB][c] = u32x4{w[0], w[1], w[2], w[3]};
      }
    };
    auto pv = [&](auto mb_c) {
      constexpr int MB = decltype(mb_c)::value;
      osum[MB] = Mfma16<T>::run(ones, pf[MB][0], osum[MB]);
      osum[MB] = Mfma16<T>::run(ones, pf[MB][1], osum[MB]);
#pragma unroll
      for (int db = 0; db < 4; ++db) o[MB][db] = Mfma16<T>::run(vf[db][0], pf[MB][0], o[MB][db]);
#pragma unroll
      for (int db = 0; db < 4; ++db) o[MB][db] = Mfma16<T>::run(vf[db][1], pf[MB][1], o[MB][db]);
    };
    // fp16 with the FMA, after the first key block: row block mb's packed
    // P against 2^THRESH (0x5C00 = 256 in fp16; inf and NaN patterns exceed
    // it); a row block that exceeds it is raised and its exponentials
    // recomputed.
    auto pcheck = [&](auto mb_c) {
      constexpr int R = decltype(mb_c)::value;
      if constexpr (PCHECK) {
        if (!first) {
          typedef _Float16 h2 __attribute__((ext_vector_type(2)));
          h2 d[8];
#pragma unroll
          for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              // through a scalar: a bit cast of the vector element itself
              // compiled to element 0 here
              const uint32_t w = pf[R][c][e];
              d[c * 4 + e] = __builtin_bit_cast(h2, w);
            }
          h2 m = __builtin_elementwise_maximum(__builtin_elementwise_maximum(d[0], d[1]), d[2]);
          m = __builtin_elementwise_maximum(__builtin_elementwise_maximum(m, d[3]), d[4]);
          m = __builtin_elementwise_maximum(__builtin_elementwise_maximum(m, d[5]), d[6]);
          m = __builtin_elementwise_maximum(m, d[7]);
          const uint32_t mb2 = __builtin_bit_cast(uint32_t, m);
          const bool over = (mb2 & 0xffffu) > 0x5C00u || (mb2 >> 16) > 0x5C00u;
          if (__builtin_amdgcn_ballot_w64(over) != 0) {
            raise(R, row_max(R));
            expo(mb_c);
          }
        }
      }
    };
    expo(std::integral_constant<int, 0>{});
    pcheck(std::integral_constant<int, 0>{});
    __builtin_amdgcn_sched_barrier(0);
    // Raised wave priority for the P V stretch, so a SIMD's arbiter favours
    // the wave that is issuing MFMAs over its sibling (the other workgroup
    // on the CU).  Measured A/B in one run, bit-identical output: C4 277 ->
    // 262 us; no change on the 17776-key DiT shape.
    __builtin_amdgcn_s_setprio(1);
    static_for<3>([&](auto i_c) {
      constexpr int I = decltype(i_c)::value;
      pv(std::integral_constant<int, I>{});
      expo(std::integral_constant<int, I + 1>{});
      // 10 MFMAs, each followed by four of the 40 VALU instructions.
#pragma unroll
      for (int g = 0; g < 10; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      pcheck(std::integral_constant<int, I + 1>{});
    });
    pv(std::integral_constant<int, 3>{});
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_sched_barrier(0);
  }

  if (wi.part >= 0) {
    // A split part: unnormalised O, m and l for attn_combine_kernel (rows
    // past Sq too; the combine skips them).
    float* wp = p.ws + wi.part * kAttnPartFloats;
    f32x4* po = reinterpret_cast<f32x4*>(wp) + wave * 1024 + lane;
    float2* pml = reinterpret_cast<float2*>(wp + kAttnPartOFloats) + wave * 256 + lane;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
      for (int db = 0; db < 4; ++db) po[(mb * 4 + db) * 64] = o[mb][db];
      pml[mb * 64] = float2{-nq[mb][0], osum[mb][0]};
    }
    return;
  }
  uint16_t* Ob = static_cast<uint16_t*>(p.O) + b * p.sO + h * p.hO;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) attn_store_rows<T>(p, Ob, q0, lane, mb, o[mb], osum[mb][0]);
}

// Merges the parts of split items: one 64-thread workgroup per 16 query
// rows (split item full_items + item0 + blockIdx.x / 16, wave w and row
// block mb of it from blockIdx.x % 16), lane l reading the partials lane l
// of that wave wrote, in part order.  Its time is load latency, not
// bandwidth, so the part loops are unrolled to keep several loads in flight
// and the grid has 16 workgroups per item.
template <typename T>
__global__ __launch_bounds__(64) void attn_combine_kernel(AttnParams p) {
  const int lane = threadIdx.x;
  const int wave = (blockIdx.x >> 2) & 3;
  const int mb = blockIdx.x & 3;
  const int64_t s = p.item0 + (blockIdx.x >> 4);  // split item index
  const AttnItem wi = attn_item(p, p.full_items + s * p.parts, 1);
  const int q0 = wi.qb * 256 + wave * 64;
  const float* base = p.ws + s * p.parts * (int64_t)kAttnPartFloats;
  uint16_t* Ob = static_cast<uint16_t*>(p.O) + wi.b * p.sO + wi.h * p.hO;
  const int ml_off = kAttnPartOFloats + ((wave * 4 + mb) * 64 + lane) * 2;
  const int o_off = ((wave * 4 + mb) * 256 + lane) * 4;
  float mmax = -INFINITY;
#pragma unroll 8
  for (int q = 0; q < p.parts; ++q) mmax = fmaxf(mmax, base[q * kAttnPartFloats + ml_off]);
  float l = 0.f;
  f32x4 o[4] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f},
                f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll 4
  for (int q = 0; q < p.parts; ++q) {
    const float* pq = base + q * kAttnPartFloats;
    const float2 ml = *reinterpret_cast<const float2*>(pq + ml_off);
    const float w = __builtin_amdgcn_exp2f(ml.x - mmax);
    l += w * ml.y;
    const f32x4* po = reinterpret_cast<const f32x4*>(pq + o_off);
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] += w * po[db * 64];
  }
  attn_store_rows<T>(p, Ob, q0, lane, mb, o, l);
}

}  // namespace sf
