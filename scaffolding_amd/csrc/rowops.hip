// rowops.hip — HBM-bound row and elementwise kernels of the path:
// row softmax (with the SDPA pre-scale folded in), standalone SiLU / GELU /
// scalar-multiply / bias-add, the sum over one axis (bias gradients),
// dtype casts and a zero fill.
#include "sf_internal.hpp"
#include "rowio.hpp"

namespace sf {

// ---------------------------------------------------------------------
// Softmax, one wave per row, the row held in registers (CPL chunks of 8
// elements per lane; cols <= 512 * CPL, cols % 8 == 0, rows 16-B aligned).
// One HBM read and one write per element.
// ---------------------------------------------------------------------
template <typename TI, typename TO, int CPL, bool NT>
__global__ __launch_bounds__(256) void softmax_wave_kernel(const void* __restrict__ x,
                                                           void* __restrict__ y, int64_t rows,
                                                           int cols, float scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nch = cols >> 3;
  const int64_t base = row * cols;
  float v[CPL][8];
  float mx = -INFINITY;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = c * 64 + lane;
    if (ch < nch) {
      Chunk8<TI>::template load<NT>(x, base + ch * 8, v[c]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[c][e] *= scale;
        mx = fmaxf(mx, v[c][e]);
      }
    }
  }
  mx = wave_max(mx);
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = c * 64 + lane;
    if (ch < nch) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[c][e] = fast_exp(v[c][e] - mx);
        s += v[c][e];
      }
    }
  }
  s = wave_sum(s);
  const float inv = 1.0f / s;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = c * 64 + lane;
    if (ch < nch) {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[c][e] *= inv;
      Chunk8<TO>::template store<NT>(y, base + ch * 8, v[c]);
    }
  }
}

// Any cols / alignment: one 256-thread block per row, three passes (max,
// sum of exp, write) over the row; the re-reads hit L2 for rows that fit.
template <typename TI, typename TO>
__global__ __launch_bounds__(256) void softmax_block_kernel(const void* __restrict__ x,
                                                            void* __restrict__ y, int64_t rows,
                                                            int64_t cols, float scale) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t base = row * cols;
  float mx = -INFINITY;
  for (int64_t c = tid; c < cols; c += 256) mx = fmaxf(mx, Chunk8<TI>::get(x, base + c) * scale);
  mx = wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float s = 0.f;
  for (int64_t c = tid; c < cols; c += 256) s += fast_exp(Chunk8<TI>::get(x, base + c) * scale - mx);
  s = wave_sum(s);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  s = red[0] + red[1] + red[2] + red[3];
  const float inv = 1.0f / s;
  for (int64_t c = tid; c < cols; c += 256)
    Chunk8<TO>::put(y, base + c, fast_exp(Chunk8<TI>::get(x, base + c) * scale - mx) * inv);
}

// ---------------------------------------------------------------------
// Softmax with an additive mask (SDPA's attn_mask): y[r, :] =
// softmax(scale * x[r, :] + mask_r), the mask of row r = b * per + i at
// off(r) = (b / inner) * souter + (b % inner) * sinner + i * srow, element j
// at off(r) + j * scol (scol 0: one value for the row).  Zero strides are
// NumPy broadcasting over that axis.
// ---------------------------------------------------------------------
__device__ __forceinline__ int64_t mask_row_off(const MaskArgs& a, int64_t r) {
  const int64_t b = r / a.per, i = r - b * a.per;
  const int64_t bo = b / a.inner, bi = b - bo * a.inner;
  return bo * a.souter + bi * a.sinner + i * a.srow;
}

// One wave per row, the row in registers (as softmax_wave_kernel); the
// mask chunk loads beside the row's (scol 1: 16-byte aligned offsets).
template <typename T, typename TM, int CPL>
__global__ __launch_bounds__(256) void softmax_mask_wave_kernel(const void* __restrict__ x,
                                                                void* __restrict__ y, int64_t rows,
                                                                int cols, float scale, MaskArgs ma) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nch = cols >> 3;
  const int64_t base = row * cols;
  const int64_t mo = mask_row_off(ma, row);
  const float mrow = ma.scol == 0 ? Chunk8<TM>::get(ma.m, mo) : 0.f;
  float v[CPL][8];
  float mx = -INFINITY;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = c * 64 + lane;
    if (ch < nch) {
      float mk[8];
      Chunk8<T>::load(x, base + ch * 8, v[c]);
      if (ma.scol != 0) {
        Chunk8<TM>::load(ma.m, mo + ch * 8, mk);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) mk[e] = mrow;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[c][e] = v[c][e] * scale + mk[e];
        mx = fmaxf(mx, v[c][e]);
      }
    }
  }
  mx = wave_max(mx);
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = c * 64 + lane;
    if (ch < nch) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[c][e] = fast_exp(v[c][e] - mx);
        s += v[c][e];
      }
    }
  }
  s = wave_sum(s);
  const float inv = 1.0f / s;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = c * 64 + lane;
    if (ch < nch) {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[c][e] *= inv;
      Chunk8<T>::store(y, base + ch * 8, v[c]);
    }
  }
}

// Any cols, strides or alignment: one block per row, three passes.
template <typename T, typename TM>
__global__ __launch_bounds__(256) void softmax_mask_block_kernel(const void* __restrict__ x,
                                                                 void* __restrict__ y, int64_t rows,
                                                                 int64_t cols, float scale, MaskArgs ma) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t base = row * cols;
  const int64_t mo = mask_row_off(ma, row);
  auto val = [&](int64_t c) {
    return Chunk8<T>::get(x, base + c) * scale + Chunk8<TM>::get(ma.m, mo + c * ma.scol);
  };
  float mx = -INFINITY;
  for (int64_t c = tid; c < cols; c += 256) mx = fmaxf(mx, val(c));
  mx = wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float s = 0.f;
  for (int64_t c = tid; c < cols; c += 256) s += fast_exp(val(c) - mx);
  s = wave_sum(s);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  s = red[0] + red[1] + red[2] + red[3];
  const float inv = 1.0f / s;
  for (int64_t c = tid; c < cols; c += 256) Chunk8<T>::put(y, base + c, fast_exp(val(c) - mx) * inv);
}

// ---------------------------------------------------------------------
// Elementwise: y = f(x) over n elements, 8 per thread per iteration.
// ---------------------------------------------------------------------
enum UnaryOp { U_SILU = 0, U_GELU = 1, U_MULS = 2 };

template <typename T, int OP>
__global__ __launch_bounds__(256) void unary_kernel(const void* x, void* y, int64_t n, float s,
                                                    bool vec) {
  const int64_t stride = (int64_t)gridDim.x * 256 * 8;
  for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8; i < n; i += stride) {
    float v[8];
    const bool full = vec && i + 8 <= n;
    if (full) {
      Chunk8<T>::load(x, i, v);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (i + e < n) ? Chunk8<T>::get(x, i + e) : 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (OP == U_SILU) v[e] = silu_f32(v[e]);
      else if (OP == U_GELU) v[e] = gelu_tanh_f32(v[e]);
      else v[e] = v[e] * s;
    }
    if (full) {
      Chunk8<T>::store(y, i, v);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (i + e < n) Chunk8<T>::put(y, i + e, v[e]);
    }
  }
}

// ---------------------------------------------------------------------
// Dropout: mask[i] = scale if u_i >= p else 0, y[i] = x[i] * mask[i].
// u_i comes from a counter-based Philox4x32-10 (Salmon, Moraes, Dror, Shaw,
// SC 2011): key (k0, k1) = the seed's halves, counter (g, g >> 32, o0, o1)
// for the group g = i / 4 of four elements and the 64-bit stream offset;
// output word i % 4, top 24 bits: u_i = (r >> 8) 2^-24.  The mask depends
// only on (seed, offset, i), never on the launch geometry.
// ---------------------------------------------------------------------
__device__ __forceinline__ u32x4 philox4x32_10(u32x4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint32_t hi0 = __umulhi(0xD2511F53u, c[0]), lo0 = 0xD2511F53u * c[0];
    const uint32_t hi1 = __umulhi(0xCD9E8D57u, c[2]), lo1 = 0xCD9E8D57u * c[2];
    c = u32x4{hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0};
  }
  return c;
}

// Each thread takes 8 elements (two Philox groups) per step.
template <typename T>
__global__ __launch_bounds__(256) void dropout_kernel(const void* x, void* y, void* mask, int64_t n, float p,
                                                      float scale, uint32_t k0, uint32_t k1, uint32_t o0,
                                                      uint32_t o1, bool vec) {
  const int64_t stride = (int64_t)gridDim.x * 256 * 8;
  for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8; i < n; i += stride) {
    float v[8], m[8];
    const bool full = vec && i + 8 <= n;
    if (full) {
      Chunk8<T>::load(x, i, v);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (i + e < n) ? Chunk8<T>::get(x, i + e) : 0.f;
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint64_t g = (uint64_t)(i >> 2) + h;
      const u32x4 r = philox4x32_10(u32x4{(uint32_t)g, (uint32_t)(g >> 32), o0, o1}, k0, k1);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float u = (float)(r[q] >> 8) * (1.0f / 16777216.0f);
        m[4 * h + q] = u >= p ? scale : 0.f;
        v[4 * h + q] *= m[4 * h + q];
      }
    }
    if (full) {
      Chunk8<T>::store(y, i, v);
      if (mask != nullptr) Chunk8<T>::store(mask, i, m);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (i + e < n) {
          Chunk8<T>::put(y, i + e, v[e]);
          if (mask != nullptr) Chunk8<T>::put(mask, i + e, m[e]);
        }
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void bias_rows_kernel(void* C, const void* bias, int64_t M,
                                                        int64_t N) {
  const int64_t total = M * N;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += stride) {
    float v = Chunk8<T>::get(C, i) + Chunk8<T>::get(bias, i % N);
    Chunk8<T>::put(C, i, v);
  }
}

template <typename TI, typename TO>
__global__ __launch_bounds__(256) void cast_kernel(const void* x, void* y, int64_t n, bool vec) {
  const int64_t stride = (int64_t)gridDim.x * 256 * 8;
  for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8; i < n; i += stride) {
    float v[8];
    if (vec && i + 8 <= n) {
      Chunk8<TI>::load(x, i, v);
      Chunk8<TO>::store(y, i, v);
    } else {
      for (int e = 0; e < 8 && i + e < n; ++e) Chunk8<TO>::put(y, i + e, Chunk8<TI>::get(x, i + e));
    }
  }
}

// NT: non-temporal body stores (large fills, which would only evict the
// caches' contents).
template <bool NT>
__global__ __launch_bounds__(256) void zero_kernel(uint8_t* p, size_t nbytes) {
  // Head bytes up to 16-B alignment, 16-B body, tail bytes.
  const size_t head = (16 - (reinterpret_cast<uintptr_t>(p) & 15)) & 15;
  const size_t h = head < nbytes ? head : nbytes;
  const size_t body = (nbytes - h) / 16;
  const size_t tid = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * 256;
  if (tid < h) p[tid] = 0;
  u32x4* q = reinterpret_cast<u32x4*>(p + h);
  for (size_t i = tid; i < body; i += stride) {
    if constexpr (NT)
      __builtin_nontemporal_store(u32x4{0u, 0u, 0u, 0u}, q + i);
    else
      q[i] = u32x4{0u, 0u, 0u, 0u};
  }
  const size_t tail0 = h + body * 16;
  if (tid < nbytes - tail0) p[tail0 + tid] = 0;
}


// ---------------------------------------------------------------------
// Sum over the middle axis of x viewed as [outer, D, inner], fp32
// accumulation:  out[o, i] = sum_{d < D} x[o, d, i].
//
// Columns (inner > 1, e.g. a bias gradient: outer 1, D rows, inner
// columns): each lane owns 8 consecutive columns; the 4 waves of a
// workgroup take every 4th d of the workgroup's d-range
// [D s / S, D (s + 1) / S); the waves' sums are added in wave order through
// LDS.  With S > 1 the workgroup writes its fp32 partial to
// ws[(o S + s) inner + i] and sum_parts_kernel adds the S partials in
// order, so the result does not depend on scheduling.
// Rows (inner == 1): one wave per o, lanes stride over d, then a fixed
// xor butterfly.
// ---------------------------------------------------------------------
template <typename TI, typename TO, bool VEC>
__global__ __launch_bounds__(256) void sum_cols_kernel(const void* __restrict__ x, void* __restrict__ out,
                                                       float* __restrict__ ws, int64_t D, int64_t inner,
                                                       int S) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t o = blockIdx.z;
  const int s = blockIdx.y;
  const int64_t i0 = ((int64_t)blockIdx.x * 64 + lane) * 8;
  const int64_t d0 = D * s / S, d1 = D * (s + 1) / S;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  if (i0 < inner) {
    const int64_t base = o * D * inner + i0;
    auto ld = [&](int64_t d, float v[8]) {
      if constexpr (VEC) {
        Chunk8<TI>::load(x, base + d * inner, v);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (i0 + e < inner) ? Chunk8<TI>::get(x, base + d * inner + e) : 0.f;
      }
    };
    int64_t d = d0 + wave;
    // Four rows' loads in flight per wave, added in row order.
    for (; d + 12 < d1; d += 16) {
      float v0[8], v1[8], v2[8], v3[8];
      ld(d, v0);
      ld(d + 4, v1);
      ld(d + 8, v2);
      ld(d + 12, v3);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = (((acc[e] + v0[e]) + v1[e]) + v2[e]) + v3[e];
    }
    for (; d < d1; d += 4) {
      float v[8];
      ld(d, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += v[e];
    }
  }
  __shared__ float red[4][8][64];
#pragma unroll
  for (int e = 0; e < 8; ++e) red[wave][e][lane] = acc[e];
  __syncthreads();
  if (wave != 0 || i0 >= inner) return;
  float t[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) t[e] = ((red[0][e][lane] + red[1][e][lane]) + red[2][e][lane]) + red[3][e][lane];
  if (S == 1) {
    const int64_t ob = o * inner + i0;
    if constexpr (VEC) {
      Chunk8<TO>::store(out, ob, t);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (i0 + e < inner) Chunk8<TO>::put(out, ob + e, t[e]);
    }
  } else {
    float* w = ws + ((int64_t)o * S + s) * inner + i0;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (i0 + e < inner) w[e] = t[e];
  }
}

// Adds the S partials of each output in part order, 64 outputs per
// workgroup: the 4 waves add parts s = w, w + 4, ... (eight loads in
// flight), then wave 0 adds the four wave sums in wave order.
template <typename TO>
__global__ __launch_bounds__(256) void sum_parts_kernel(const float* __restrict__ ws, void* __restrict__ out,
                                                        int64_t outer, int64_t inner, int S) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t idx = (int64_t)blockIdx.x * 64 + lane;
  float t = 0.f;
  if (idx < outer * inner) {
    const int64_t o = idx / inner, i = idx - o * inner;
    const float* w = ws + o * S * inner + i;
    int s = wave;
    for (; s + 28 < S; s += 32) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = w[(int64_t)(s + 4 * u) * inner];
#pragma unroll
      for (int u = 0; u < 8; ++u) t += v[u];
    }
    for (; s < S; s += 4) t += w[(int64_t)s * inner];
  }
  __shared__ float red[4][64];
  red[wave][lane] = t;
  __syncthreads();
  if (wave == 0 && idx < outer * inner)
    Chunk8<TO>::put(out, idx, ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane]);
}

template <typename TI, typename TO, bool VEC>
__global__ __launch_bounds__(256) void sum_rows_kernel(const void* __restrict__ x, void* __restrict__ out,
                                                       int64_t outer, int64_t D) {
  const int lane = threadIdx.x & 63;
  const int64_t o = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (o >= outer) return;
  float acc = 0.f;
  if constexpr (VEC) {
    for (int64_t c = (int64_t)lane * 8; c < D; c += 512) {
      float v[8];
      Chunk8<TI>::load(x, o * D + c, v);
      acc += ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    }
  } else {
    for (int64_t c = lane; c < D; c += 64) acc += Chunk8<TI>::get(x, o * D + c);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane == 0) Chunk8<TO>::put(out, o, acc);
}

// ---------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------
static unsigned grid_for(int64_t work_items) {
  int64_t g = (work_items + 255) / 256;
  if (g < 1) g = 1;
  if (g > 8192) g = 8192;  // grid-stride beyond 32 blocks per CU
  return static_cast<unsigned>(g);
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <typename TI, typename TO>
static void softmax_launch_t(const void* x, void* y, int64_t rows, int64_t cols, float scale,
                             hipStream_t st) {
  const bool vec = (cols % 8 == 0) && aligned16(x) && aligned16(y) && cols <= 8192;
  if (vec) {
    const unsigned grid = static_cast<unsigned>((rows + 3) / 4);
    const int c = static_cast<int>(cols);
    // Past the 256 MB Infinity Cache nothing stays cached for the consumer:
    // stream input and output non-temporally.
    const bool nt = (double)rows * (double)cols * (double)sizeof(typename Elem<TI>::storage) > 256.0 * (1 << 20);
    auto go = [&](auto cpl_c) {
      constexpr int CPL = decltype(cpl_c)::value;
      if (nt)
        hipLaunchKernelGGL((softmax_wave_kernel<TI, TO, CPL, true>), dim3(grid), dim3(256), 0, st, x, y, rows, c, scale);
      else
        hipLaunchKernelGGL((softmax_wave_kernel<TI, TO, CPL, false>), dim3(grid), dim3(256), 0, st, x, y, rows, c, scale);
    };
    if (cols <= 512)
      go(std::integral_constant<int, 1>{});
    else if (cols <= 1024)
      go(std::integral_constant<int, 2>{});
    else if (cols <= 2048)
      go(std::integral_constant<int, 4>{});
    else if (cols <= 4096)
      go(std::integral_constant<int, 8>{});
    else
      go(std::integral_constant<int, 16>{});
  } else {
    hipLaunchKernelGGL((softmax_block_kernel<TI, TO>), dim3(static_cast<unsigned>(rows)), dim3(256), 0,
                       st, x, y, rows, cols, scale);
  }
}

template <typename TI>
static void softmax_launch_i(sf_dtype out, const void* x, void* y, int64_t rows, int64_t cols,
                             float scale, hipStream_t st) {
  if (out == SF_F32) softmax_launch_t<TI, float>(x, y, rows, cols, scale, st);
  else if (out == SF_F16) softmax_launch_t<TI, F16>(x, y, rows, cols, scale, st);
  else softmax_launch_t<TI, BF16>(x, y, rows, cols, scale, st);
}

int launch_softmax(const void* x, void* y, int64_t rows, int64_t cols, sf_dtype in, sf_dtype out,
                   float scale, hipStream_t st) {
  if (in == SF_F32) softmax_launch_i<float>(out, x, y, rows, cols, scale, st);
  else if (in == SF_F16) softmax_launch_i<F16>(out, x, y, rows, cols, scale, st);
  else softmax_launch_i<BF16>(out, x, y, rows, cols, scale, st);
  return check_launch("softmax");
}

template <typename T, typename TM>
static void softmax_mask_launch_t(const void* x, void* y, int64_t rows, int64_t cols, float scale,
                                  const MaskArgs& ma, hipStream_t st) {
  const int64_t msz = (int64_t)sizeof(typename Elem<TM>::storage);
  const bool mvec = ma.scol == 0 ||
                    (aligned16(ma.m) && (ma.srow * msz) % 16 == 0 && (ma.souter * msz) % 16 == 0 &&
                     (ma.sinner * msz) % 16 == 0);
  if ((cols % 8 == 0) && aligned16(x) && aligned16(y) && cols <= 8192 && mvec) {
    const unsigned grid = static_cast<unsigned>((rows + 3) / 4);
    const int c = static_cast<int>(cols);
    auto go = [&](auto cpl_c) {
      constexpr int CPL = decltype(cpl_c)::value;
      hipLaunchKernelGGL((softmax_mask_wave_kernel<T, TM, CPL>), dim3(grid), dim3(256), 0, st, x, y, rows, c,
                         scale, ma);
    };
    if (cols <= 512)
      go(std::integral_constant<int, 1>{});
    else if (cols <= 1024)
      go(std::integral_constant<int, 2>{});
    else if (cols <= 2048)
      go(std::integral_constant<int, 4>{});
    else if (cols <= 4096)
      go(std::integral_constant<int, 8>{});
    else
      go(std::integral_constant<int, 16>{});
  } else {
    hipLaunchKernelGGL((softmax_mask_block_kernel<T, TM>), dim3(static_cast<unsigned>(rows)), dim3(256), 0, st, x,
                       y, rows, cols, scale, ma);
  }
}

int launch_softmax_masked(const void* x, void* y, int64_t rows, int64_t cols, sf_dtype dt, float scale,
                          const MaskArgs& ma, sf_dtype mask_dt, hipStream_t st) {
  const bool mf32 = mask_dt == SF_F32;
  if (dt == SF_F32) softmax_mask_launch_t<float, float>(x, y, rows, cols, scale, ma, st);
  else if (dt == SF_F16) {
    if (mf32) softmax_mask_launch_t<F16, float>(x, y, rows, cols, scale, ma, st);
    else softmax_mask_launch_t<F16, F16>(x, y, rows, cols, scale, ma, st);
  } else {
    if (mf32) softmax_mask_launch_t<BF16, float>(x, y, rows, cols, scale, ma, st);
    else softmax_mask_launch_t<BF16, BF16>(x, y, rows, cols, scale, ma, st);
  }
  return check_launch("softmax (masked)");
}

template <typename T>
static void unary_launch_t(int op, const void* x, void* y, int64_t n, float s, hipStream_t st) {
  const bool vec = aligned16(x) && aligned16(y);
  const unsigned grid = grid_for((n + 7) / 8);
  if (op == U_SILU) hipLaunchKernelGGL((unary_kernel<T, U_SILU>), dim3(grid), dim3(256), 0, st, x, y, n, s, vec);
  else if (op == U_GELU) hipLaunchKernelGGL((unary_kernel<T, U_GELU>), dim3(grid), dim3(256), 0, st, x, y, n, s, vec);
  else hipLaunchKernelGGL((unary_kernel<T, U_MULS>), dim3(grid), dim3(256), 0, st, x, y, n, s, vec);
}

int launch_unary(int op, const void* x, void* y, int64_t n, sf_dtype dt, float s, hipStream_t st) {
  if (dt == SF_F32) unary_launch_t<float>(op, x, y, n, s, st);
  else if (dt == SF_F16) unary_launch_t<F16>(op, x, y, n, s, st);
  else unary_launch_t<BF16>(op, x, y, n, s, st);
  return check_launch("elementwise");
}

template <typename T>
static void dropout_launch_t(const void* x, void* y, void* mask, int64_t n, float p, float scale, uint64_t seed,
                             uint64_t offset, hipStream_t st) {
  const bool vec = aligned16(x) && aligned16(y) && (mask == nullptr || aligned16(mask));
  const unsigned grid = grid_for((n + 7) / 8);
  hipLaunchKernelGGL((dropout_kernel<T>), dim3(grid), dim3(256), 0, st, x, y, mask, n, p, scale, (uint32_t)seed,
                     (uint32_t)(seed >> 32), (uint32_t)offset, (uint32_t)(offset >> 32), vec);
}

int launch_dropout(const void* x, void* y, void* mask, int64_t n, sf_dtype dt, float p, uint64_t seed,
                   uint64_t offset, hipStream_t st) {
  const float scale = 1.0f / (1.0f - p);
  if (dt == SF_F32) dropout_launch_t<float>(x, y, mask, n, p, scale, seed, offset, st);
  else if (dt == SF_F16) dropout_launch_t<F16>(x, y, mask, n, p, scale, seed, offset, st);
  else dropout_launch_t<BF16>(x, y, mask, n, p, scale, seed, offset, st);
  return check_launch("dropout");
}

int launch_bias_rows(void* C, const void* bias, int64_t M, int64_t N, sf_dtype dt, hipStream_t st) {
  const unsigned grid = grid_for(M * N);
  if (dt == SF_F32) hipLaunchKernelGGL((bias_rows_kernel<float>), dim3(grid), dim3(256), 0, st, C, bias, M, N);
  else if (dt == SF_F16) hipLaunchKernelGGL((bias_rows_kernel<F16>), dim3(grid), dim3(256), 0, st, C, bias, M, N);
  else hipLaunchKernelGGL((bias_rows_kernel<BF16>), dim3(grid), dim3(256), 0, st, C, bias, M, N);
  return check_launch("bias_add_rows");
}

template <typename TI>
static void cast_launch_i(sf_dtype out, const void* x, void* y, int64_t n, hipStream_t st) {
  const bool vec = aligned16(x) && aligned16(y);
  const unsigned grid = grid_for((n + 7) / 8);
  if (out == SF_F32) hipLaunchKernelGGL((cast_kernel<TI, float>), dim3(grid), dim3(256), 0, st, x, y, n, vec);
  else if (out == SF_F16) hipLaunchKernelGGL((cast_kernel<TI, F16>), dim3(grid), dim3(256), 0, st, x, y, n, vec);
  else hipLaunchKernelGGL((cast_kernel<TI, BF16>), dim3(grid), dim3(256), 0, st, x, y, n, vec);
}

int launch_cast(const void* x, sf_dtype in, void* y, sf_dtype out, int64_t n, hipStream_t st) {
  if (in == SF_F32) cast_launch_i<float>(out, x, y, n, st);
  else if (in == SF_F16) cast_launch_i<F16>(out, x, y, n, st);
  else cast_launch_i<BF16>(out, x, y, n, st);
  return check_launch("cast");
}

// Parts S of the column sum: enough workgroups to cover the CUs once, each
// still summing at least 64 rows.
int sum_dim_parts(int64_t outer, int64_t D, int64_t inner, int cus) {
  if (inner <= 1) return 1;
  const int64_t wgs = ((inner + 511) / 512) * outer;
  int64_t S = ((int64_t)cus + wgs - 1) / wgs;
  if (S > D / 64) S = D / 64;
  if (S > 1024) S = 1024;
  return S < 1 ? 1 : (int)S;
}

template <typename TI, typename TO>
static void sum_dim_launch_t(const void* x, void* y, int64_t outer, int64_t D, int64_t inner, float* ws, int S,
                             hipStream_t st) {
  if (inner == 1) {
    const bool vec = D % 8 == 0 && aligned16(x);
    const dim3 g(static_cast<unsigned>((outer + 3) / 4));
    if (vec) hipLaunchKernelGGL((sum_rows_kernel<TI, TO, true>), g, dim3(256), 0, st, x, y, outer, D);
    else hipLaunchKernelGGL((sum_rows_kernel<TI, TO, false>), g, dim3(256), 0, st, x, y, outer, D);
    return;
  }
  const bool vec = inner % 8 == 0 && aligned16(x) && aligned16(y);
  const dim3 g(static_cast<unsigned>((inner + 511) / 512), static_cast<unsigned>(S), static_cast<unsigned>(outer));
  if (vec) hipLaunchKernelGGL((sum_cols_kernel<TI, TO, true>), g, dim3(256), 0, st, x, y, ws, D, inner, S);
  else hipLaunchKernelGGL((sum_cols_kernel<TI, TO, false>), g, dim3(256), 0, st, x, y, ws, D, inner, S);
  if (S > 1)
    hipLaunchKernelGGL((sum_parts_kernel<TO>), dim3(static_cast<unsigned>((outer * inner + 63) / 64)), dim3(256), 0, st,
                       ws, y, outer, inner, S);
}

template <typename TI>
static void sum_dim_launch_i(sf_dtype out, const void* x, void* y, int64_t outer, int64_t D, int64_t inner,
                             float* ws, int S, hipStream_t st) {
  if (out == SF_F32) sum_dim_launch_t<TI, float>(x, y, outer, D, inner, ws, S, st);
  else if (out == SF_F16) sum_dim_launch_t<TI, F16>(x, y, outer, D, inner, ws, S, st);
  else sum_dim_launch_t<TI, BF16>(x, y, outer, D, inner, ws, S, st);
}

int launch_sum_dim(const void* x, void* y, int64_t outer, int64_t D, int64_t inner, sf_dtype in, sf_dtype out,
                   float* ws, int S, hipStream_t st) {
  if (in == SF_F32) sum_dim_launch_i<float>(out, x, y, outer, D, inner, ws, S, st);
  else if (in == SF_F16) sum_dim_launch_i<F16>(out, x, y, outer, D, inner, ws, S, st);
  else sum_dim_launch_i<BF16>(out, x, y, outer, D, inner, ws, S, st);
  return check_launch("sum_dim");
}

int launch_zero(void* p, size_t nbytes, hipStream_t st) {
  if (nbytes >= (size_t(64) << 20)) {
    // Large fills (past a quarter of the 256 MB Infinity Cache): two 16-byte
    // stores per thread, as many workgroups as that takes (at most 2^20).
    // Measured over 1 GiB: 6.06 TB/s at 131072 workgroups of 256 against
    // 4.77 TB/s at the grid-stride cap of 8192.
    const size_t g = (nbytes / 16 + 511) / 512;
    const unsigned grid = static_cast<unsigned>(g > (size_t(1) << 20) ? (size_t(1) << 20) : g);
    hipLaunchKernelGGL(zero_kernel<true>, dim3(grid), dim3(256), 0, st, static_cast<uint8_t*>(p), nbytes);
  } else {
    const unsigned grid = grid_for(static_cast<int64_t>((nbytes + 15) / 16));
    hipLaunchKernelGGL(zero_kernel<false>, dim3(grid), dim3(256), 0, st, static_cast<uint8_t*>(p), nbytes);
  }
  return check_launch("zero");
}

}  // namespace sf
