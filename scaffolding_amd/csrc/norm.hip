// norm.hip — row normalisations and the elementwise add of the DiT block
// glue: layer norm with an optional adaptive (per-group scale / shift)
// modulation, RMS norm, and y = a + b.  All HBM-bound: one read of x and
// one write of y per element; gamma, beta and the modulation rows are
// small and stay in the caches.
#include "sf_internal.hpp"
#include "rowio.hpp"

namespace sf {

// Everything a normalisation kernel reads besides x (NULL pointers: none).
struct NormParams {
  const void* x;
  void* y;
  const void* gamma;
  const void* beta;
  const void* mscale;  // modulation rows, group g at g * mld
  const void* mshift;
  float* mean_out;
  float* rstd_out;
  int64_t rows;
  int64_t mld;
  int64_t group_rows;
  int cols;
  float eps;
};

// One row's affine + modulation for 8 consecutive columns starting at c.
template <typename T, bool VEC>
__device__ __forceinline__ void norm_tail8(const NormParams& p, int64_t row, int c, float v[8]) {
  float g[8], b[8], s[8], t[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) { g[e] = 1.f; b[e] = 0.f; s[e] = 0.f; t[e] = 0.f; }
  auto ld = [&](const void* base, int64_t off, float out[8]) {
    if constexpr (VEC) {
      Chunk8<T>::load(base, off + c, out);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (c + e < p.cols) out[e] = Chunk8<T>::get(base, off + c + e);
    }
  };
  if (p.gamma) ld(p.gamma, 0, g);
  if (p.beta) ld(p.beta, 0, b);
  const int64_t moff = (row / p.group_rows) * p.mld;
  if (p.mscale) ld(p.mscale, moff, s);
  if (p.mshift) ld(p.mshift, moff, t);
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (v[e] * g[e] + b[e]) * (1.0f + s[e]) + t[e];
}

// One wave per row, the row held in registers: CPL chunks of 8 elements
// per lane (cols <= 512 CPL, cols % 8 == 0, 16-byte aligned rows, gamma,
// beta and modulation rows).  Mean, then the mean squared deviation from
// the registers (two-pass: no cancellation), then the output.
// RMS = true: no centring, rstd from the mean square, gamma only.
// When the workgroup's four rows share one modulation group, its threads
// first fold gamma, beta and the group's (scale, shift) into fp32
// A = gamma (1 + scale), B = beta (1 + scale) + shift in LDS, while the
// waves' row loads are in flight: one L2 read of the four vectors per
// workgroup instead of one per row, off the rows' critical path.
template <typename T, int CPL, bool RMS>
__global__ __launch_bounds__(256) void norm_wave_kernel(NormParams p) {
  __shared__ __attribute__((aligned(16))) float sAB[2][CPL * 512];
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t row_first = (int64_t)blockIdx.x * 4;
  const int64_t row_last = (row_first + 3 < p.rows ? row_first + 3 : p.rows - 1);
  const bool folded = !RMS && row_first / p.group_rows == row_last / p.group_rows;  // workgroup-uniform
  const int nch = p.cols >> 3;
  if (folded) {
    const int64_t moff = (row_first / p.group_rows) * p.mld;
    for (int ch = threadIdx.x; ch < nch; ch += 256) {
      float gm[8], bt[8], sc[8], sh[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) { gm[e] = 1.f; bt[e] = 0.f; sc[e] = 0.f; sh[e] = 0.f; }
      if (p.gamma) Chunk8<T>::load(p.gamma, ch * 8, gm);
      if (p.beta) Chunk8<T>::load(p.beta, ch * 8, bt);
      if (p.mscale) Chunk8<T>::load(p.mscale, moff + ch * 8, sc);
      if (p.mshift) Chunk8<T>::load(p.mshift, moff + ch * 8, sh);
      f32x4 a0, a1, b0, b1;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        a0[e] = gm[e] * (1.0f + sc[e]);
        a1[e] = gm[e + 4] * (1.0f + sc[e + 4]);
        b0[e] = bt[e] * (1.0f + sc[e]) + sh[e];
        b1[e] = bt[e + 4] * (1.0f + sc[e + 4]) + sh[e + 4];
      }
      *reinterpret_cast<f32x4*>(&sAB[0][ch * 8]) = a0;
      *reinterpret_cast<f32x4*>(&sAB[0][ch * 8 + 4]) = a1;
      *reinterpret_cast<f32x4*>(&sAB[1][ch * 8]) = b0;
      *reinterpret_cast<f32x4*>(&sAB[1][ch * 8 + 4]) = b1;
    }
  }
  const bool live = row < p.rows;
  const int64_t base = row * p.cols;
  float v[CPL][8];
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = c * 64 + lane;
    if (live && ch < nch) {
      Chunk8<T>::load(p.x, base + ch * 8, v[c]);
      if constexpr (!RMS) {
#pragma unroll
        for (int e = 0; e < 8; ++e) sum += v[c][e];
      }
    }
  }
  if (folded) __syncthreads();  // the folded coefficients are in LDS
  if (!live) return;
  const float inv_n = 1.0f / (float)p.cols;
  float mu = 0.f;
  if constexpr (!RMS) mu = wave_sum(sum) * inv_n;
  float sq = 0.f;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = c * 64 + lane;
    if (ch < nch) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = v[c][e] - mu;
        sq += d * d;
      }
    }
  }
  const float rstd = 1.0f / sqrtf(wave_sum(sq) * inv_n + p.eps);
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = c * 64 + lane;
    if (ch < nch) {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[c][e] = (v[c][e] - mu) * rstd;
      if constexpr (RMS) {
        if (p.gamma) {
          float g[8];
          Chunk8<T>::load(p.gamma, ch * 8, g);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[c][e] *= g[e];
        }
      } else if (folded) {
        const f32x4 a0 = *reinterpret_cast<const f32x4*>(&sAB[0][ch * 8]);
        const f32x4 a1 = *reinterpret_cast<const f32x4*>(&sAB[0][ch * 8 + 4]);
        const f32x4 b0 = *reinterpret_cast<const f32x4*>(&sAB[1][ch * 8]);
        const f32x4 b1 = *reinterpret_cast<const f32x4*>(&sAB[1][ch * 8 + 4]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[c][e] = v[c][e] * a0[e] + b0[e];
          v[c][e + 4] = v[c][e + 4] * a1[e] + b1[e];
        }
      } else {
        norm_tail8<T, true>(p, row, ch * 8, v[c]);
      }
      Chunk8<T>::store(p.y, base + ch * 8, v[c]);
    }
  }
  if (lane == 0) {
    if (p.mean_out) p.mean_out[row] = mu;
    if (p.rstd_out) p.rstd_out[row] = rstd;
  }
}

// Any cols or alignment: one 256-thread workgroup per row, three passes
// over the row (sum, squared deviations, output); the re-reads hit the
// caches.
template <typename T, bool RMS>
__global__ __launch_bounds__(256) void norm_block_kernel(NormParams p) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t base = row * p.cols;
  auto block_sum = [&](float s) {
    s = wave_sum(s);
    __syncthreads();
    if (lane == 0) red[wave] = s;
    __syncthreads();
    return ((red[0] + red[1]) + red[2]) + red[3];
  };
  const float inv_n = 1.0f / (float)p.cols;
  float mu = 0.f;
  if constexpr (!RMS) {
    float s = 0.f;
    for (int c = tid; c < p.cols; c += 256) s += Chunk8<T>::get(p.x, base + c);
    mu = block_sum(s) * inv_n;
  }
  float sq = 0.f;
  for (int c = tid; c < p.cols; c += 256) {
    const float d = Chunk8<T>::get(p.x, base + c) - mu;
    sq += d * d;
  }
  const float rstd = 1.0f / sqrtf(block_sum(sq) * inv_n + p.eps);
  const int64_t moff = (row / p.group_rows) * p.mld;
  for (int c = tid; c < p.cols; c += 256) {
    float v = (Chunk8<T>::get(p.x, base + c) - mu) * rstd;
    if (p.gamma) v *= Chunk8<T>::get(p.gamma, c);
    if constexpr (!RMS) {
      if (p.beta) v += Chunk8<T>::get(p.beta, c);
      const float s = p.mscale ? Chunk8<T>::get(p.mscale, moff + c) : 0.f;
      const float t = p.mshift ? Chunk8<T>::get(p.mshift, moff + c) : 0.f;
      v = v * (1.0f + s) + t;
    }
    Chunk8<T>::put(p.y, base + c, v);
  }
  if (tid == 0) {
    if (p.mean_out) p.mean_out[row] = mu;
    if (p.rstd_out) p.rstd_out[row] = rstd;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void add_kernel(const void* a, const void* b, void* y, int64_t n, bool vec) {
  const int64_t stride = (int64_t)gridDim.x * 256 * 8;
  for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8; i < n; i += stride) {
    if (vec && i + 8 <= n) {
      float u[8], w[8];
      Chunk8<T>::load(a, i, u);
      Chunk8<T>::load(b, i, w);
#pragma unroll
      for (int e = 0; e < 8; ++e) u[e] += w[e];
      Chunk8<T>::store(y, i, u);
    } else {
      for (int e = 0; e < 8 && i + e < n; ++e)
        Chunk8<T>::put(y, i + e, Chunk8<T>::get(a, i + e) + Chunk8<T>::get(b, i + e));
    }
  }
}

static bool al16p(const void* q) { return q == nullptr || (reinterpret_cast<uintptr_t>(q) & 15) == 0; }

template <typename T, bool RMS>
static void launch_norm_t(const NormParams& p, bool wave_ok, hipStream_t st) {
  if (wave_ok) {
    const dim3 g((unsigned)((p.rows + 3) / 4));
    const int cpl = (p.cols + 511) / 512;
    if (cpl <= 1)
      hipLaunchKernelGGL((norm_wave_kernel<T, 1, RMS>), g, dim3(256), 0, st, p);
    else if (cpl <= 2)
      hipLaunchKernelGGL((norm_wave_kernel<T, 2, RMS>), g, dim3(256), 0, st, p);
    else if (cpl <= 4)
      hipLaunchKernelGGL((norm_wave_kernel<T, 4, RMS>), g, dim3(256), 0, st, p);
    else
      hipLaunchKernelGGL((norm_wave_kernel<T, 8, RMS>), g, dim3(256), 0, st, p);
  } else {
    hipLaunchKernelGGL((norm_block_kernel<T, RMS>), dim3((unsigned)p.rows), dim3(256), 0, st, p);
  }
}

int launch_norm(const NormArgs& a, sf_dtype dt, hipStream_t st) {
  NormParams p;
  p.x = a.x; p.y = a.y; p.gamma = a.gamma; p.beta = a.beta;
  p.mscale = a.mscale; p.mshift = a.mshift;
  p.mean_out = a.mean_out; p.rstd_out = a.rstd_out;
  p.rows = a.rows; p.cols = (int)a.cols; p.eps = a.eps;
  // Without modulation every row shares one set of coefficients (group 0).
  const bool mod = a.mscale != nullptr || a.mshift != nullptr;
  p.mld = a.mld;
  p.group_rows = mod ? (a.group_rows > 0 ? a.group_rows : 1) : (a.rows > 0 ? a.rows : 1);
  const int per16 = dt == SF_F32 ? 4 : 8;
  // The register-resident kernel loads 8-element chunks (16 or 32 bytes):
  // every row it touches must start 16-byte aligned.
  const bool wave_ok = a.cols % 8 == 0 && a.cols <= 4096 && al16p(a.x) && al16p(a.y) && al16p(a.gamma) &&
                       al16p(a.beta) && al16p(a.mscale) && al16p(a.mshift) &&
                       ((a.mscale == nullptr && a.mshift == nullptr) || a.mld % per16 == 0);
  // grid.x of the block kernel is one workgroup per row.
  if (!wave_ok && a.rows > INT32_MAX) return fail(SF_ERR_UNSUPPORTED, "norm: more than 2^31 rows");
  if (dt == SF_F32)
    a.rms ? launch_norm_t<float, true>(p, wave_ok, st) : launch_norm_t<float, false>(p, wave_ok, st);
  else if (dt == SF_F16)
    a.rms ? launch_norm_t<F16, true>(p, wave_ok, st) : launch_norm_t<F16, false>(p, wave_ok, st);
  else
    a.rms ? launch_norm_t<BF16, true>(p, wave_ok, st) : launch_norm_t<BF16, false>(p, wave_ok, st);
  return check_launch(a.rms ? "rms_norm" : "layer_norm");
}

int launch_add(const void* a, const void* b, void* y, int64_t n, sf_dtype dt, hipStream_t st) {
  const bool vec = al16p(a) && al16p(b) && al16p(y);
  int64_t blocks = (n + 256 * 8 - 1) / (256 * 8);
  if (blocks > 4096) blocks = 4096;
  const dim3 g((unsigned)blocks);
  if (dt == SF_F32)
    hipLaunchKernelGGL((add_kernel<float>), g, dim3(256), 0, st, a, b, y, n, vec);
  else if (dt == SF_F16)
    hipLaunchKernelGGL((add_kernel<F16>), g, dim3(256), 0, st, a, b, y, n, vec);
  else
    hipLaunchKernelGGL((add_kernel<BF16>), g, dim3(256), 0, st, a, b, y, n, vec);
  return check_launch("add");
}

}  // namespace sf
