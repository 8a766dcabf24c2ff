// sf_common.hpp — device-side building blocks shared by every kernel of
// libsfgemm: vector types, 16-bit conversions, the fused epilogue and the
// XCD-aware tile ordering.  gfx950 (CDNA4) only.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>
#include <stdint.h>

#include "../../include/sfgemm.h"

namespace sf {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 16-bit element tags.  Storage is always uint16_t in memory; the tag picks
// the MFMA variant and the conversions.
struct BF16 {};
struct F16 {};

// ---------------------------------------------------------------------
// Conversions.  float -> 16-bit is round-to-nearest-even with NaN kept a
// (quiet) NaN; these are the hardware conversions of gfx950
// (v_cvt_pk_bf16_f32 / v_cvt_f16_f32 honour RNE in the default mode).
// ---------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  __bf16 b = static_cast<__bf16>(f);
  return __builtin_bit_cast(uint16_t, b);
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  _Float16 h = static_cast<_Float16>(f);
  return __builtin_bit_cast(uint16_t, h);
}

template <typename T> struct Elem;
template <> struct Elem<float> {
  typedef float storage;
  __device__ __forceinline__ static float load(const float* p) { return *p; }
  __device__ __forceinline__ static float to_f32(float v) { return v; }
  __device__ __forceinline__ static float from_f32(float v) { return v; }
};
template <> struct Elem<BF16> {
  typedef uint16_t storage;
  __device__ __forceinline__ static float to_f32(uint16_t v) { return bf16_to_f32(v); }
  __device__ __forceinline__ static uint16_t from_f32(float v) { return f32_to_bf16(v); }
};
template <> struct Elem<F16> {
  typedef uint16_t storage;
  __device__ __forceinline__ static float to_f32(uint16_t v) { return f16_to_f32(v); }
  __device__ __forceinline__ static uint16_t from_f32(float v) { return f32_to_f16(v); }
};

// ---------------------------------------------------------------------
// Epilogue math (fp32).  Formulas follow the reference's CPU path:
// silu  nn/functional.py:58-59   x * 1/(1+exp(-x))
// gelu  nn/functional.py:81-82   0.5 x (1 + tanh(sqrt(2/pi)(x + 0.044715 x^3)))
// exp and the reciprocal use the hardware v_exp_f32 / v_rcp_f32 (about
// 1 ulp each).  GELU uses the identity 0.5 (1 + tanh(u)) = 1 / (1 + e^{-2u}),
// so gelu(x) = x / (1 + e^{-2u}): the same shape as SiLU, no cancellation
// for negative x (the 1 + tanh(u) form loses all digits as tanh -> -1),
// a few ulps relative error everywhere.
// ---------------------------------------------------------------------
__device__ __forceinline__ float fast_exp(float x) {
  // e^x = 2^(x * log2(e)); v_exp_f32 flushes to 0 / saturates to inf at the
  // extremes, which is the right limit for both activations.
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

__device__ __forceinline__ float silu_f32(float t) {
  // For t -> -inf, exp(-t) -> inf and rcp(inf) = 0, so silu -> -0 (the
  // true limit is 0); for t -> +inf, rcp(1) = 1.
  return t * fast_rcp(1.0f + fast_exp(-t));
}
__device__ __forceinline__ float gelu_tanh_f32(float t) {
  // e^{-2u} = 2^z with z = t (c0 + c1 t^2): the constants -2 sqrt(2/pi)
  // log2(e) and its product with 0.044715 are folded, so the polynomial is
  // one multiply and one FMA (three operations fewer than evaluating u
  // first: this runs once per output in the GEMM epilogues, where it
  // measured 34 -> 24 us of a 384 us C5 MLP-up launch).
  const float c0 = (float)(-2.0 * 0.7978845608028654 * 1.4426950408889634);
  const float c1 = (float)(-2.0 * 0.7978845608028654 * 0.044715 * 1.4426950408889634);
  const float z = t * __builtin_fmaf(c1, t * t, c0);
  // z -> +inf (t -> -inf) gives rcp(inf) = 0, i.e. gelu -> -0.
  return t * fast_rcp(1.0f + __builtin_amdgcn_exp2f(z));
}

// Activation applied after the (optional) bias add.
enum Act { ACT_NONE = 0, ACT_SILU = 1, ACT_GELU = 2 };

template <int ACT>
__device__ __forceinline__ float act_t(float v) {
  if constexpr (ACT == ACT_SILU)
    return silu_f32(v);
  else if constexpr (ACT == ACT_GELU)
    return gelu_tanh_f32(v);
  else
    return v;
}

// Two fp32 values rounded (RNE) to the 16-bit type T and packed, a in the
// low half: one v_cvt_pk_{f16,bf16}_f32.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float a, float b);
template <>
__device__ __forceinline__ uint32_t pack2<F16>(float a, float b) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, h2));
}
template <>
__device__ __forceinline__ uint32_t pack2<BF16>(float a, float b) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, b2));
}

// static_for<N>(f): f(std::integral_constant<int, 0>{}) ... f(..., N - 1>{})
// in order, each index a compile-time constant.
template <int N>
struct StaticFor {
  template <typename F>
  __device__ __forceinline__ static void run(F&& f) {
    StaticFor<N - 1>::run(f);
    f(std::integral_constant<int, N - 1>{});
  }
};
template <>
struct StaticFor<0> {
  template <typename F>
  __device__ __forceinline__ static void run(F&&) {}
};
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  StaticFor<N>::run(f);
}

// Calls f(std::integral_constant<int, ACT>{}) for the wave-uniform runtime
// activation `act`: the per-element epilogue is compiled once per activation
// instead of testing `act` for every value it writes.
template <typename F>
__device__ __forceinline__ void with_act(int act, F&& f) {
  if (act == ACT_SILU)
    f(std::integral_constant<int, ACT_SILU>{});
  else if (act == ACT_GELU)
    f(std::integral_constant<int, ACT_GELU>{});
  else
    f(std::integral_constant<int, ACT_NONE>{});
}

// Decode sf_epilogue into (has_bias, act).
__host__ __device__ inline bool epi_has_bias(int epi) {
  return epi == SF_EPI_BIAS || epi == SF_EPI_BIAS_SILU || epi == SF_EPI_BIAS_GELU_TANH;
}
__host__ __device__ inline int epi_act(int epi) {
  if (epi == SF_EPI_BIAS_SILU || epi == SF_EPI_SILU) return ACT_SILU;
  if (epi == SF_EPI_BIAS_GELU_TANH || epi == SF_EPI_GELU_TANH) return ACT_GELU;
  return ACT_NONE;
}

// ---------------------------------------------------------------------
// Tile ordering.
// The command processor hands workgroup i to XCD (i mod 8); each XCD has
// its own 4 MB L2.  xcd_remap turns the hardware order into one where the
// workgroups that land on one XCD get a contiguous range of tile ids, and
// group_tile then walks that range in GROUP_M-tall column bands so an XCD's
// resident tiles share A row-panels and B column-panels in its L2.
// ---------------------------------------------------------------------
constexpr int kNumXcd = 8;

__device__ __forceinline__ int xcd_remap(int pid, int nblocks) {
  int xcd = pid % kNumXcd;
  int local = pid / kNumXcd;
  int base = nblocks / kNumXcd;
  int extra = nblocks % kNumXcd;
  // XCDs [0, extra) own base+1 ids, the rest own base ids.
  int start = xcd * base + (xcd < extra ? xcd : extra);
  return start + local;
}

__device__ __forceinline__ void group_tile(int pid, int tiles_m, int tiles_n, int group_m,
                                           int& tm, int& tn) {
  int per_group = group_m * tiles_n;
  int gid = pid / per_group;
  int first_m = gid * group_m;
  int gsize = tiles_m - first_m;
  if (gsize > group_m) gsize = group_m;
  int r = pid - gid * per_group;
  tm = first_m + r % gsize;
  tn = r / gsize;
}

// The lane index (0..63) computed by v_mbcnt in volatile assembly, so the
// compiler neither merges it with an earlier threadIdx.x nor keeps that
// value alive across a loop: use it after register-heavy loops.
__device__ __forceinline__ int lane_id_fresh() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// Wave-wide sum / max through cross-lane permutes (64 lanes).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

}  // namespace sf
