// attention.hip — launcher of the fused attention kernel (attention.hpp).
#include "sf_internal.hpp"
#include "attention.hpp"

namespace sf {

AttnSplit attn_split_plan(const AttnShape& a, int cus) {
  AttnSplit sp;
  sp.items = a.batch * a.heads * ((a.Sq + 255) / 256);
  sp.full = sp.items;
  sp.parts = 0;
  const int64_t nb = (a.Sk + 63) / 64;
  // Two workgroups per CU, all equally long: the items past the last whole
  // round of slots (the tail) run alone.  They are split into P key ranges
  // (at least 8 key blocks a part, at most 16 parts) when that shortens
  // their phase: tail * P parts take ceil(tail * P / slots) rounds of
  // nb / P key blocks each, plus about 3 key blocks' time a part for its
  // fp32 partials and the combine, against one round of nb key blocks
  // unsplit; the smallest such cost wins if it is under 90 % of the
  // unsplit round.  A tail of at most half the slots takes P = slots /
  // tail (one round).  Measured at 17776 tokens: 30 heads (2100 items over
  // 512 slots, a tail of 52) 2.47 ms unsplit against 2.13 ms in 9 parts.
  const int64_t slots = 2 * (int64_t)cus;
  const int64_t tail = sp.items % slots;
  int64_t P = 0;
  if (tail > 0) {
    const int64_t pmax = nb / 8 < 16 ? nb / 8 : 16;
    double best = 0.9 * (double)nb;
    for (int64_t q = 2; q <= pmax; ++q) {
      const double cost = (double)((tail * q + slots - 1) / slots) * ((double)nb / (double)q + 3.0);
      if (cost < best) {
        best = cost;
        P = q;
      }
    }
  }
  // Test hook (sf_set_test_hooks): every item split into P key ranges (at
  // most one a key block, and at most 1 GiB of partials); the results must
  // agree with the unsplit kernel to rounding.
  const int tp = g_test_hooks.attn_parts.load(std::memory_order_relaxed);
  if (tp >= 2) {
    int64_t hp = tp > 16 ? 16 : tp;
    if (hp > nb) hp = nb;
    const int64_t fit = (int64_t(1) << 30) / ((int64_t)kAttnPartBytes * sp.items);
    if (hp > fit) hp = fit;
    if (hp >= 2) {
      sp.full = 0;
      sp.parts = (int)hp;
      return sp;
    }
  }
  if (P >= 2) {
    sp.full = sp.items - tail;
    sp.parts = (int)P;
  }
  return sp;
}

int launch_attention(const AttnShape& a, float scale, sf_dtype dt, const AttnSplit& sp, float* ws, hipStream_t st) {
  AttnParams p;
  p.Q = a.Q; p.K = a.K; p.V = a.V; p.O = a.O;
  p.sQ = a.sQ; p.sK = a.sK; p.sV = a.sV; p.sO = a.sO;
  p.hQ = a.hQ; p.hK = a.hK; p.hV = a.hV; p.hO = a.hO;
  p.H = (int)a.heads;
  p.ldq = (int)a.ldq; p.ldk = (int)a.ldk; p.ldv = (int)a.ldv; p.ldo = (int)a.ldo;
  p.Sq = (int)a.Sq; p.Sk = (int)a.Sk;
  p.D = (int)a.D;
  p.scale_log2e = scale * 1.4426950408889634f;
  p.QB = (int)((a.Sq + 255) / 256);
  p.full_items = sp.full;
  p.parts = sp.parts;
  p.ws = ws;
  // One workgroup per whole item, then one per split part.
  const int64_t split_items = sp.items - sp.full;
  const int64_t wgs = sp.full + (sp.parts > 0 ? split_items * sp.parts : 0);
  constexpr int64_t kChunk = int64_t(1) << 30;  // workgroups per launch (grid.x < 2^31)
  for (int64_t i0 = 0; i0 < wgs; i0 += kChunk) {
    const int64_t n = (wgs - i0) < kChunk ? (wgs - i0) : kChunk;
    p.item0 = i0;
    // Q pre-scaled by scale log2 e (attn64_kernel's PRESCALE) when
    // scale log2 e <= 1: the usual 1/sqrt(D) scales (D >= 3), where it
    // cannot overflow fp16 and Q's extra rounding moves each exponent by
    // about 2^-9 (bf16) or 2^-12 (fp16) of the logit's size; larger scales
    // keep the FMA on the fp32 scores.
    const bool pre = p.scale_log2e <= 1.0f;
    if (dt == SF_F16) {
      if (pre)
        hipLaunchKernelGGL((attn64_kernel<F16, true>), dim3((unsigned)n), dim3(256), 0, st, p);
      else
        hipLaunchKernelGGL((attn64_kernel<F16, false>), dim3((unsigned)n), dim3(256), 0, st, p);
    } else {
      if (pre)
        hipLaunchKernelGGL((attn64_kernel<BF16, true>), dim3((unsigned)n), dim3(256), 0, st, p);
      else
        hipLaunchKernelGGL((attn64_kernel<BF16, false>), dim3((unsigned)n), dim3(256), 0, st, p);
    }
    const int rc = check_launch("attention");
    if (rc != SF_OK) return rc;
  }
  if (sp.parts == 0) return SF_OK;
  for (int64_t i0 = 0; i0 < split_items; i0 += kChunk / 16) {
    const int64_t n = (split_items - i0) < kChunk / 16 ? (split_items - i0) : kChunk / 16;
    p.item0 = i0;
    if (dt == SF_F16)
      hipLaunchKernelGGL((attn_combine_kernel<F16>), dim3((unsigned)(16 * n)), dim3(64), 0, st, p);
    else
      hipLaunchKernelGGL((attn_combine_kernel<BF16>), dim3((unsigned)(16 * n)), dim3(64), 0, st, p);
    const int rc = check_launch("attention (combine)");
    if (rc != SF_OK) return rc;
  }
  return SF_OK;
}

}  // namespace sf
