// attention.hip — fused scaled-dot-product attention forward for head size
// 64, 16-bit Q/K/V/O with fp32 accumulation:
//
//   O[b] = softmax(scale * Q[b] K[b]^T) V[b],  Q [Sq, 64], K, V [Sk, 64].
//
// One 256-thread workgroup per 256 query rows of one batch entry; wave w
// owns 64 of them (four 16-row blocks).  The workgroup streams K and V in
// blocks of 64 keys through a 3-stage LDS ring (16 KB per stage), and per
// block each wave
//   1. forms S = Q K^T for its 64 x 64 scores: 32 v_mfma_f32_16x16x32 with
//      Q fragments held in registers for the whole loop and K fragments
//      read from LDS (ds_read_b128, 128-byte lines, chunk h at slot
//      h ^ (row & 7), conflict-free as in the GEMM kernels);
//   2. updates the online softmax in the exp2 domain: running row maximum
//      m (reduced over the four lanes sharing a row), correction
//      2^(m_old - m_new) applied to O and to the per-lane partial row sums;
//   3. packs P = 2^(S * scale * log2 e - m) to 16 bits and adds P V into
//      the 64 x 64 fp32 O accumulator: 32 more MFMAs whose V fragments come
//      from ds_read_b64_tr_b16 (gfx950's transposing LDS read).
// P's MFMA k slots follow the score accumulator layout (lane group g holds
// keys 4g..4g+3 and 16+4g..16+4g+3 of each 32-key chunk), and the V
// fragment reads use the same key order, so P never moves between lanes.
// The 2 GB score and probability tensors of the three-kernel path are never
// written.  Requires head size 64, Sk % 64 == 0, 16-byte aligned rows.
#include "sf_internal.hpp"
#include "gemm16nt_pp.hpp"

namespace sf {

struct AttnParams {
  const void* Q;
  const void* K;
  const void* V;
  void* O;
  int64_t sQ, sK, sV, sO;      // batch strides, elements
  int ldq, ldk, ldv, ldo;      // row strides, elements
  int Sq, Sk;
  float scale_log2e;           // scale * log2(e)
};

// ds_read_b64_tr_b16 as inline assembly (see ds_read16 for why): within each
// 16-lane group, lane 4a + b receives element b of the 8-byte rows addressed
// by lanes a, 4 + a, 8 + a and 12 + a (measured lane layout).
template <int OFF>
__device__ __forceinline__ u32x2 ds_read_tr16(uint32_t addr) {
  u32x2 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}

__device__ __forceinline__ float shfl_xor_f(float v, int mask) { return __shfl_xor(v, mask, 64); }

template <typename T>
__global__ __launch_bounds__(256) void attn64_kernel(AttnParams p) {
  constexpr int NS = 3;              // K/V ring stages
  constexpr int KB = 64;             // keys per block
  constexpr int BLK = KB * 128;      // 8 KB: 64 rows x 128 bytes
  __shared__ __attribute__((aligned(1024))) uint8_t sK[NS][BLK];
  __shared__ __attribute__((aligned(1024))) uint8_t sV[NS][BLK];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t b = blockIdx.y;
  const int q0 = blockIdx.x * 256 + wave * 64;
  const int Sq = p.Sq, Sk = p.Sk;
  const int NB = Sk / KB;
  const uint16_t* Qb = static_cast<const uint16_t*>(p.Q) + b * p.sQ;
  const uint16_t* Kb = static_cast<const uint16_t*>(p.K) + b * p.sK;
  const uint16_t* Vb = static_cast<const uint16_t*>(p.V) + b * p.sV;

  // K and V blocks move by buffer_load ... lds, 8 whole 128-byte rows per
  // instruction: wave w fills rows 16 w .. 16 w + 15 of each block (two
  // instructions per operand); lane l takes row + (l >> 3), slot l & 7,
  // i.e. chunk (l & 7) ^ (l >> 3) (row & 7 == l >> 3).
  const __amdgpu_buffer_rsrc_t rK =
      __builtin_amdgcn_make_buffer_rsrc((void*)Kb, (short)0, (int)((uint32_t)Sk * (uint32_t)p.ldk * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t rV =
      __builtin_amdgcn_make_buffer_rsrc((void*)Vb, (short)0, (int)((uint32_t)Sk * (uint32_t)p.ldv * 2u), 0x00020000);
  const int drow = wave * 16 + (lane >> 3);
  const uint32_t dch = (uint32_t)(((lane & 7) ^ (lane >> 3)) * 16);
  const uint32_t vk0 = (uint32_t)drow * (uint32_t)p.ldk * 2u + dch;
  const uint32_t vk1 = vk0 + 8u * (uint32_t)p.ldk * 2u;
  const uint32_t vv0 = (uint32_t)drow * (uint32_t)p.ldv * 2u + dch;
  const uint32_t vv1 = vv0 + 8u * (uint32_t)p.ldv * 2u;
  auto issue = [&](int j) {
    const int s = j % NS;
    const int ko = j * KB * p.ldk * 2, vo = j * KB * p.ldv * 2;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rK, (lds_ptr_t)(&sK[s][0] + wave * 2048), 16, vk0, ko, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rK, (lds_ptr_t)(&sK[s][0] + wave * 2048 + 1024), 16, vk1, ko, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rV, (lds_ptr_t)(&sV[s][0] + wave * 2048), 16, vv0, vo, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rV, (lds_ptr_t)(&sV[s][0] + wave * 2048 + 1024), 16, vv1, vo, 0, 0);
  };
  issue(0);
  if (NB > 1) issue(1);

  // Q fragments (Y operand): block mb, d chunk kc: row q0 + 16 mb + (l & 15),
  // d = 32 kc + 8 (l >> 4) .. + 7.  Rows past Sq read the last row.
  u32x4 qf[4][2];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    int r = q0 + mb * 16 + (lane & 15);
    r = r < Sq ? r : Sq - 1;
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
      qf[mb][kc] = *reinterpret_cast<const u32x4*>(Qb + (int64_t)r * p.ldq + kc * 32 + 8 * (lane >> 4));
  }

  f32x4 o[4][4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int db = 0; db < 4; ++db) o[mb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float mrow[4], lpart[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    mrow[mb] = -INFINITY;
    lpart[mb] = 0.f;
  }
  const float sc = p.scale_log2e;

  // K fragment (X operand) of key block nb, d chunk kc: line nb*16 + (l & 15),
  // chunk 4 kc + (l >> 4).
  const uint32_t kfo = (uint32_t)((lane & 15) * 128 + (((lane >> 4) ^ (lane & 7)) << 4));
  // V transposing reads for d block db, key chunk c, half hf: source lane
  // s = l & 15 of group g = l >> 4 addresses row 32 c + 16 hf + 4 g + (s >> 2),
  // d = 16 db + 4 (s & 3), i.e. 16-byte chunk 2 db + ((s & 3) >> 1), byte
  // 8 ((s & 3) & 1) within it, at slot chunk ^ (row & 7).
  const int vs = lane & 15, vg = lane >> 4;
  const int vrow0 = 4 * vg + (vs >> 2);  // + 32 c + 16 hf
  const uint32_t vfo_base = (uint32_t)vrow0 * 128u + (uint32_t)((vs & 1) * 8);
  const int vch = (vs & 3) >> 1;  // + 2 db
  // row & 7 == (vrow0 + 32 c + 16 hf) & 7 == vrow0 & 7
  const int vsw = vrow0 & 7;

  for (int j = 0; j < NB; ++j) {
    const int st = j % NS;
    __builtin_amdgcn_sched_barrier(0);
    if (j + 1 < NB)
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(4, 0));
    else
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
    __builtin_amdgcn_s_barrier();  // block j in LDS for all; block j-1 fully read
    __builtin_amdgcn_sched_barrier(0);
    if (j + 2 < NB) issue(j + 2);
    __builtin_amdgcn_sched_barrier(0);

    // ---- S = Q K^T -------------------------------------------------------
    const uint32_t ka = lds_addr(&sK[st][0]) + kfo;
    u32x4 kf[4][2];
    kf[0][0] = ds_read16<0 * 2048>(ka);
    kf[0][1] = ds_read16<0 * 2048>(ka ^ 64);
    kf[1][0] = ds_read16<1 * 2048>(ka);
    kf[1][1] = ds_read16<1 * 2048>(ka ^ 64);
    kf[2][0] = ds_read16<2 * 2048>(ka);
    kf[2][1] = ds_read16<2 * 2048>(ka ^ 64);
    kf[3][0] = ds_read16<3 * 2048>(ka);
    kf[3][1] = ds_read16<3 * 2048>(ka ^ 64);
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
    __builtin_amdgcn_sched_barrier(0);
    f32x4 s[4][4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        s[mb][nb] = Mfma16<T>::run(kf[nb][0], qf[mb][0], f32x4{0.f, 0.f, 0.f, 0.f});
        s[mb][nb] = Mfma16<T>::run(kf[nb][1], qf[mb][1], s[mb][nb]);
      }

    // ---- V fragments (issued early; used after the softmax) -------------
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t va = lds_addr(&sV[st][0]) + vfo_base;
    u32x4 vf[4][2];
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const uint32_t slot_b = (uint32_t)(((2 * db + vch) ^ vsw) << 4);
      const uint32_t a0 = va + slot_b;
      // c = 0: rows + 0 (hf 0) and + 16 (hf 1); c = 1: rows + 32, + 48.
      const u32x2 t00 = ds_read_tr16<0>(a0);
      const u32x2 t01 = ds_read_tr16<16 * 128>(a0);
      const u32x2 t10 = ds_read_tr16<32 * 128>(a0);
      const u32x2 t11 = ds_read_tr16<48 * 128>(a0);
      vf[db][0] = u32x4{t00.x, t00.y, t01.x, t01.y};
      vf[db][1] = u32x4{t10.x, t10.y, t11.x, t11.y};
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- online softmax ---------------------------------------------------
    u32x4 pf[4][2];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      float mx = s[mb][0][0];
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int q = 0; q < 4; ++q) mx = fmaxf(mx, s[mb][nb][q]);
      mx = fmaxf(mx, shfl_xor_f(mx, 16));
      mx = fmaxf(mx, shfl_xor_f(mx, 32));
      const float mnew = fmaxf(mrow[mb], mx * sc);
      const float corr = __builtin_amdgcn_exp2f(mrow[mb] - mnew);
      mrow[mb] = mnew;
      float ps = 0.f;
      float pv[4][4];
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          pv[nb][q] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[mb][nb][q], sc, -mnew));
          ps += pv[nb][q];
        }
      lpart[mb] = lpart[mb] * corr + ps;
#pragma unroll
      for (int db = 0; db < 4; ++db) o[mb][db] *= corr;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        uint32_t w[4];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int q2 = 0; q2 < 2; ++q2)
            w[h * 2 + q2] = (uint32_t)Elem<T>::from_f32(pv[2 * c + h][2 * q2]) |
                            ((uint32_t)Elem<T>::from_f32(pv[2 * c + h][2 * q2 + 1]) << 16);
        pf[mb][c] = u32x4{w[0], w[1], w[2], w[3]};
      }
    }

    // ---- O += P V ---------------------------------------------------------
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        o[mb][db] = Mfma16<T>::run(vf[db][0], pf[mb][0], o[mb][db]);
        o[mb][db] = Mfma16<T>::run(vf[db][1], pf[mb][1], o[mb][db]);
      }
  }

  // ---- normalise and store: lane l holds O[row 16 mb + (l & 15)][16 db + 4 (l >> 4) + q]
  uint16_t* Ob = static_cast<uint16_t*>(p.O) + b * p.sO;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    float l = lpart[mb];
    l += shfl_xor_f(l, 16);
    l += shfl_xor_f(l, 32);
    const float inv = 1.0f / l;
    const int r = q0 + mb * 16 + (lane & 15);
    if (r < Sq) {
      uint16_t* orow = Ob + (int64_t)r * p.ldo;
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int d = db * 16 + 4 * (lane >> 4);
        const uint32_t lo = Elem<T>::from_f32(o[mb][db][0] * inv) | ((uint32_t)Elem<T>::from_f32(o[mb][db][1] * inv) << 16);
        const uint32_t hi = Elem<T>::from_f32(o[mb][db][2] * inv) | ((uint32_t)Elem<T>::from_f32(o[mb][db][3] * inv) << 16);
        *reinterpret_cast<u32x2*>(orow + d) = u32x2{lo, hi};
      }
    }
  }
}

int launch_attention(const void* Q, const void* K, const void* V, void* O, int64_t batch, int64_t Sq,
                     int64_t Sk, int64_t sQ, int64_t sK, int64_t sV, int64_t sO, int64_t ldq, int64_t ldk,
                     int64_t ldv, int64_t ldo, float scale, sf_dtype dt, hipStream_t st) {
  AttnParams p;
  p.Q = Q; p.K = K; p.V = V; p.O = O;
  p.sQ = sQ; p.sK = sK; p.sV = sV; p.sO = sO;
  p.ldq = (int)ldq; p.ldk = (int)ldk; p.ldv = (int)ldv; p.ldo = (int)ldo;
  p.Sq = (int)Sq; p.Sk = (int)Sk;
  p.scale_log2e = scale * 1.4426950408889634f;
  const unsigned gx = (unsigned)((Sq + 255) / 256);
  for (int64_t b0 = 0; b0 < batch; b0 += 65535) {
    const int64_t nb = (batch - b0) < 65535 ? (batch - b0) : 65535;
    AttnParams q = p;
    q.Q = static_cast<const uint16_t*>(Q) + b0 * sQ;
    q.K = static_cast<const uint16_t*>(K) + b0 * sK;
    q.V = static_cast<const uint16_t*>(V) + b0 * sV;
    q.O = static_cast<uint16_t*>(O) + b0 * sO;
    if (dt == SF_F16)
      hipLaunchKernelGGL((attn64_kernel<F16>), dim3(gx, (unsigned)nb), dim3(256), 0, st, q);
    else
      hipLaunchKernelGGL((attn64_kernel<BF16>), dim3(gx, (unsigned)nb), dim3(256), 0, st, q);
    const int rc = check_launch("attention");
    if (rc != SF_OK) return rc;
  }
  return SF_OK;
}

}  // namespace sf
