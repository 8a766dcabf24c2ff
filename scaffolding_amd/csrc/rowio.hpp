// rowio.hpp — 8-element chunk loads and stores of the row and elementwise
// kernels, for every element type, with fp32 values in registers.
#pragma once

#include "sf_common.hpp"

namespace sf {

// Generic 8-element chunk load/store for any element type.  `vec` selects
// the 16-byte (16-bit types) / 2x16-byte (fp32) path, else per element.
template <typename T> struct Chunk8;
// NT: non-temporal (streaming) access, for tensors larger than the caches.
template <bool NT, typename V>
__device__ __forceinline__ V ld16(const V* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}
template <bool NT, typename V>
__device__ __forceinline__ void st16(V* p, V v) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

template <> struct Chunk8<float> {
  template <bool NT = false>
  __device__ __forceinline__ static void load(const void* base, int64_t i, float v[8]) {
    const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(base) + i);
    f32x4 a = ld16<NT>(p), b = ld16<NT>(p + 1);
#pragma unroll
    for (int e = 0; e < 4; ++e) { v[e] = a[e]; v[e + 4] = b[e]; }
  }
  template <bool NT = false>
  __device__ __forceinline__ static void store(void* base, int64_t i, const float v[8]) {
    f32x4* p = reinterpret_cast<f32x4*>(static_cast<float*>(base) + i);
    st16<NT>(p, f32x4{v[0], v[1], v[2], v[3]});
    st16<NT>(p + 1, f32x4{v[4], v[5], v[6], v[7]});
  }
  __device__ __forceinline__ static float get(const void* base, int64_t i) {
    return static_cast<const float*>(base)[i];
  }
  __device__ __forceinline__ static void put(void* base, int64_t i, float v) {
    static_cast<float*>(base)[i] = v;
  }
};
template <typename T> struct Chunk8 {  // BF16 / F16
  template <bool NT = false>
  __device__ __forceinline__ static void load(const void* base, int64_t i, float v[8]) {
    u32x4 w = ld16<NT>(reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + i));
#pragma unroll
    for (int e = 0; e < 8; ++e)
      v[e] = Elem<T>::to_f32(static_cast<uint16_t>(w[e >> 1] >> ((e & 1) * 16)));
  }
  template <bool NT = false>
  __device__ __forceinline__ static void store(void* base, int64_t i, const float v[8]) {
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = static_cast<uint32_t>(Elem<T>::from_f32(v[2 * e])) |
             (static_cast<uint32_t>(Elem<T>::from_f32(v[2 * e + 1])) << 16);
    st16<NT>(reinterpret_cast<u32x4*>(static_cast<uint16_t*>(base) + i), w);
  }
  __device__ __forceinline__ static float get(const void* base, int64_t i) {
    return Elem<T>::to_f32(static_cast<const uint16_t*>(base)[i]);
  }
  __device__ __forceinline__ static void put(void* base, int64_t i, float v) {
    static_cast<uint16_t*>(base)[i] = Elem<T>::from_f32(v);
  }
};

}  // namespace sf
