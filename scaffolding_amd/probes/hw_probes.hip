// hw_probes.hip — measurement kernels for the gfx950 rules that bound this
// library's kernels.  They are not part of libsfgemm and no product path
// loads them: `bench.py --hw-probes` builds nothing, loads libsfprobe.so
// (built beside libsfgemm.so) and prints what they measure.
//
//   sfp_issue       two instruction streams on one SIMD (one wave each, or
//                   both in one wave): shader cycles per iteration from
//                   s_memtime, so the power-managed clock does not enter;
//   sfp_mfma_rate   MFMAs only (the 4096^3 GEMM's count of
//                   v_mfma_f32_16x16x32_bf16), on random or constant
//                   operands: wall time, i.e. the clock the data allows;
//   sfp_lds_read    ds_read_b128 alone, eight waves per CU: LDS read bytes
//                   per ns per CU.
//
// Every kernel touches only registers, its own LDS and one output word per
// thread (plus one cycle count per wave), sized by the host from the grid.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Streams (per iteration of one wave):
//   1 mfma16  16 independent v_mfma_f32_16x16x32_bf16 (4 accumulators)
//   2 fma     64 v_fma_f32 (16 independent chains)
//   3 exp     32 v_exp_f32 (16 independent chains)
//   4 mfma16 + fma in one wave, 1 MFMA : 4 FMA
//   5 mfma16 + exp in one wave, 1 MFMA : 2 exp
//   6 mfma32  8 v_mfma_f32_32x32x16_bf16 (2 accumulators; the same flops as 1)
//   7 cvt     64 v_cvt_pk_bf16_f32, each followed by a v_xor_b32 that feeds
//             the next conversion (so neither leaves the loop)
//   8 max3    64 v_max3_f32
enum Stream { kIdle = 0, kMfma16 = 1, kFma = 2, kExp = 3, kMfmaFma = 4, kMfmaExp = 5, kMfma32 = 6, kCvt = 7, kMax3 = 8 };

template <int R>
__device__ __forceinline__ float stream(int iters, float seed) {
  f32x4 acc[4] = {{seed, 0, 0, 0}, {0, seed, 0, 0}, {0, 0, seed, 0}, {0, 0, 0, seed}};
  f32x16 acc32[2];
  for (int i = 0; i < 16; ++i) {
    acc32[0][i] = seed * i;
    acc32[1][i] = -seed * i;
  }
  bf16x8 a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(seed * 0.001f * i);
    b[i] = (__bf16)(0.5f + 0.01f * i);
  }
  float v[16];
  uint32_t u[16];
  for (int i = 0; i < 16; ++i) {
    v[i] = seed * 0.0025f * (i + 1);
    u[i] = __builtin_bit_cast(uint32_t, v[i]);
  }
  for (int it = 0; it < iters; ++it) {
    if constexpr (R == kMfma16 || R == kMfmaFma || R == kMfmaExp) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[q], 0, 0, 0);
    }
    if constexpr (R == kMfma32) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int q = 0; q < 2; ++q) acc32[q] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc32[q], 0, 0, 0);
    }
    if constexpr (R == kFma || R == kMfmaFma) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int q = 0; q < 16; ++q) v[q] = __builtin_fmaf(v[q], 0.999f, 0.0001f);
    }
    if constexpr (R == kExp || R == kMfmaExp) {
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int q = 0; q < 16; ++q) v[q] = __builtin_amdgcn_exp2f(-v[q]);
    }
    if constexpr (R == kCvt) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          typedef float f2 __attribute__((ext_vector_type(2)));
          typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
          const float x = __builtin_bit_cast(float, u[q]);
          u[q] ^= __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{x, x}, bf2));
        }
    }
    if constexpr (R == kMax3) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int q = 0; q < 16; ++q) v[q] = __builtin_fmaxf(__builtin_fmaxf(v[q], v[(q + 5) & 15]), v[(q + 9) & 15]);
    }
    if constexpr (R == kMfmaFma) {
#pragma unroll
      for (int g = 0; g < 16; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
      }
    }
    if constexpr (R == kMfmaExp) {
#pragma unroll
      for (int g = 0; g < 16; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  float s = 0.f;
  for (int q = 0; q < 4; ++q) s += acc[q][0] + acc[q][1] + acc[q][2] + acc[q][3];
  for (int i = 0; i < 16; ++i) s += v[i] + acc32[0][i] + acc32[1][i] + (float)(u[i] & 1u);
  return s;
}

template <int R>
__device__ __forceinline__ float run_stream(int iters, float seed) {
  if constexpr (R == kIdle)
    return 0.f;
  else
    return stream<R>(iters, seed);
}

// 4 * W waves (W per SIMD), 96 KB of LDS so one workgroup per CU.  Waves
// 0-3 run stream RA, waves 4-7 stream RB; out has blockDim.x words per
// workgroup, cyc 8 per workgroup.
template <int RA, int RB>
__global__ __launch_bounds__(512) void issue_kernel(float* out, long long* cyc, int iters) {
  __shared__ float pad[24576];
  const int w = threadIdx.x >> 6;
  if (threadIdx.x == 0) pad[0] = 0.f;
  __syncthreads();
  const long long t0 = __builtin_amdgcn_s_memtime();
  const float seed = 1.0f + threadIdx.x * 1e-3f;
  const float s = w < 4 ? run_stream<RA>(iters, seed) : run_stream<RB>(iters, seed);
  const long long t1 = __builtin_amdgcn_s_memtime();
  out[blockIdx.x * blockDim.x + threadIdx.x] = s + pad[threadIdx.x & 7];
  if ((threadIdx.x & 63) == 0) cyc[blockIdx.x * 8 + w] = t1 - t0;
}

typedef void (*issue_fn)(dim3, dim3, float*, long long*, int);

template <int RA, int RB>
void launch_issue(dim3 g, dim3 b, float* out, long long* cyc, int iters) {
  hipLaunchKernelGGL((issue_kernel<RA, RB>), g, b, 0, 0, out, cyc, iters);
}

// The (A, B) pairs sfp_issue supports; B = 0 runs A alone (4 waves).
issue_fn pick_issue(int a, int b) {
  switch (a * 16 + b) {
#define SFP_CASE(A, B) \
  case A * 16 + B: return launch_issue<A, B>;
    SFP_CASE(1, 0) SFP_CASE(2, 0) SFP_CASE(3, 0) SFP_CASE(4, 0) SFP_CASE(5, 0) SFP_CASE(6, 0) SFP_CASE(7, 0)
    SFP_CASE(8, 0) SFP_CASE(1, 1) SFP_CASE(2, 2) SFP_CASE(3, 3) SFP_CASE(7, 7) SFP_CASE(8, 8) SFP_CASE(1, 2)
    SFP_CASE(1, 3) SFP_CASE(6, 2) SFP_CASE(6, 3) SFP_CASE(2, 3) SFP_CASE(1, 7)
#undef SFP_CASE
    default: return nullptr;
  }
}

// MFMA-only: 8 waves per CU, 32 independent accumulators, fragments cycled
// over 8 A and 4 B registers loaded from `ops` (random or constant data).
__global__ __launch_bounds__(512) void mfma_rate_kernel(const u32x4* __restrict__ ops, float* out, int iters) {
  const int lane = threadIdx.x & 63;
  u32x4 fa[8], fb[4];
#pragma unroll
  for (int i = 0; i < 8; ++i) fa[i] = ops[i * 64 + lane];
#pragma unroll
  for (int i = 0; i < 4; ++i) fb[i] = ops[(8 + i) * 64 + lane];
  f32x4 acc[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 32; ++i)
      acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, fa[i & 7]),
                                                       __builtin_bit_cast(bf16x8, fb[(i >> 3) & 3]), acc[i], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) s += acc[i][0] + acc[i][1] + acc[i][2] + acc[i][3];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// LDS reads only: 8 waves per CU, each lane reads 16 bytes at a
// conflict-free address per instruction, 8 reads in flight, folded by XOR.
__global__ __launch_bounds__(512) void lds_read_kernel(float* out, int iters) {
  // 96 KB so one workgroup per CU; the reads use the first 64 KB
  __shared__ __attribute__((aligned(16))) uint32_t buf[24576];
  for (int i = threadIdx.x; i < 16384; i += blockDim.x) buf[i] = i * 2654435761u;
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const uint32_t base = (uint32_t)(w * 8192 + lane * 16);  // each wave its own 8 KB
  u32x4 x = u32x4{0u, 0u, 0u, 0u};
  for (int it = 0; it < iters; ++it) {
    u32x4 r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      r[j] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint8_t*>(buf) + ((base + j * 1024 + it * 16) & 65535u));
#pragma unroll
    for (int j = 0; j < 8; ++j) x ^= r[j];
  }
  out[blockIdx.x * blockDim.x + threadIdx.x] = (float)(x[0] ^ x[1] ^ x[2] ^ x[3]);
}

int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return cus;
}

}  // namespace

extern "C" {

// Cycles per iteration (mean over waves) of stream role_a on waves 0-3 and
// role_b on waves 4-7 of one workgroup per CU; role_b < 0: no second wave
// per SIMD.  cycles[0] = group A, cycles[1] = group B (0 without one).
// Returns 1 for a pair pick_issue does not hold.
int sfp_issue(int role_a, int role_b, int iters, double* cycles) {
  if (role_a < 1 || role_a > 8 || role_b > 8 || role_b == 0 || iters < 1 || iters > 1000000) return 1;
  issue_fn f = pick_issue(role_a, role_b < 0 ? 0 : role_b);
  if (f == nullptr) return 1;
  const int cus = device_cus();
  if (cus < 1) return 2;
  const int waves = role_b < 0 ? 4 : 8;
  float* out = nullptr;
  long long* cyc = nullptr;
  if (hipMalloc(&out, (size_t)cus * 512 * sizeof(float)) != hipSuccess) return 3;
  if (hipMalloc(&cyc, (size_t)cus * 8 * sizeof(long long)) != hipSuccess) {
    (void)hipFree(out);
    return 3;
  }
  int rc = 0;
  for (int r = 0; r < 3 && rc == 0; ++r) {
    f(dim3(cus), dim3(64 * waves), out, cyc, iters);
    if (hipGetLastError() != hipSuccess) rc = 4;
  }
  std::vector<long long> h((size_t)cus * 8);
  if (rc == 0 && hipDeviceSynchronize() != hipSuccess) rc = 4;
  if (rc == 0 && hipMemcpy(h.data(), cyc, h.size() * sizeof(long long), hipMemcpyDeviceToHost) != hipSuccess) rc = 4;
  if (rc == 0) {
    double sa = 0, sb = 0;
    for (int b = 0; b < cus; ++b)
      for (int w = 0; w < waves; ++w) (w < 4 ? sa : sb) += (double)h[(size_t)b * 8 + w];
    cycles[0] = sa / (4.0 * cus) / iters;
    cycles[1] = waves == 8 ? sb / (4.0 * cus) / iters : 0.0;
  }
  (void)hipFree(out);
  (void)hipFree(cyc);
  return rc;
}

// MFMA-only launches of the 4096^3 GEMM's MFMA count (8 waves on every CU,
// 2 * 4096^3 flop per launch); random != 0: operands ~ N(0, 1)-like bf16,
// else x = 1 and w = 1/128 (every product and sum exact).  Runs `warm`
// untimed launches, then times `launches`; writes microseconds per launch.
int sfp_mfma_rate(int random, int warm, int launches, double* us_per_launch, double* flop_per_launch) {
  if (warm < 0 || launches < 1 || launches > 100000) return 1;
  const int cus = device_cus();
  if (cus < 1) return 2;
  const double total_mfma = 2.0 * 4096.0 * 4096.0 * 4096.0 / (16.0 * 16.0 * 32.0 * 2.0);
  const int waves = cus * 8;
  const int iters = (int)(total_mfma / waves / 32.0 + 0.5);
  std::vector<uint16_t> h(12 * 64 * 8);
  uint64_t st = 12345;
  for (size_t i = 0; i < h.size(); ++i) {
    if (random) {
      st = st * 6364136223846793005ULL + 1442695040888963407ULL;
      const uint32_t r = (uint32_t)(st >> 40);  // 24 random bits
      // sign, exponent in [2^-3, 2^3), 7 random mantissa bits
      h[i] = (uint16_t)(((r & 1u) << 15) | ((124u + ((r >> 1) & 7u)) << 7) | ((r >> 4) & 0x7fu));
    } else {
      h[i] = i < 8 * 64 * 8 ? 0x3F80 : 0x3C00;  // 1.0 and 1/128 in bf16
    }
  }
  u32x4* ops = nullptr;
  float* out = nullptr;
  if (hipMalloc(&ops, h.size() * 2) != hipSuccess) return 3;
  if (hipMalloc(&out, (size_t)cus * 512 * sizeof(float)) != hipSuccess) {
    (void)hipFree(ops);
    return 3;
  }
  int rc = hipMemcpy(ops, h.data(), h.size() * 2, hipMemcpyHostToDevice) == hipSuccess ? 0 : 4;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (rc == 0 && (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)) rc = 4;
  for (int i = 0; i < warm && rc == 0; ++i) {
    hipLaunchKernelGGL(mfma_rate_kernel, dim3(cus), dim3(512), 0, 0, ops, out, iters);
    if (hipGetLastError() != hipSuccess) rc = 4;
  }
  if (rc == 0 && hipEventRecord(e0, 0) != hipSuccess) rc = 4;
  for (int i = 0; i < launches && rc == 0; ++i) {
    hipLaunchKernelGGL(mfma_rate_kernel, dim3(cus), dim3(512), 0, 0, ops, out, iters);
    if (hipGetLastError() != hipSuccess) rc = 4;
  }
  float ms = 0.f;
  if (rc == 0 && (hipEventRecord(e1, 0) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
                  hipEventElapsedTime(&ms, e0, e1) != hipSuccess))
    rc = 4;
  if (rc == 0) {
    *us_per_launch = 1000.0 * ms / launches;
    *flop_per_launch = (double)waves * iters * 32.0 * 16.0 * 16.0 * 32.0 * 2.0;
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  (void)hipFree(ops);
  (void)hipFree(out);
  return rc;
}

// LDS read rate: one 8-wave workgroup per CU, `iters` rounds of 8
// ds_read_b128 per wave.  Writes bytes per ns per CU (timed over
// `launches` after 3 untimed).
int sfp_lds_read(int iters, int launches, double* bytes_per_ns_per_cu) {
  if (iters < 1 || iters > 10000000 || launches < 1 || launches > 10000) return 1;
  const int cus = device_cus();
  if (cus < 1) return 2;
  float* out = nullptr;
  if (hipMalloc(&out, (size_t)cus * 512 * sizeof(float)) != hipSuccess) return 3;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = (hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess) ? 0 : 4;
  for (int i = 0; i < 3 && rc == 0; ++i) {
    hipLaunchKernelGGL(lds_read_kernel, dim3(cus), dim3(512), 0, 0, out, iters);
    if (hipGetLastError() != hipSuccess) rc = 4;
  }
  if (rc == 0 && hipEventRecord(e0, 0) != hipSuccess) rc = 4;
  for (int i = 0; i < launches && rc == 0; ++i) {
    hipLaunchKernelGGL(lds_read_kernel, dim3(cus), dim3(512), 0, 0, out, iters);
    if (hipGetLastError() != hipSuccess) rc = 4;
  }
  float ms = 0.f;
  if (rc == 0 && (hipEventRecord(e1, 0) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
                  hipEventElapsedTime(&ms, e0, e1) != hipSuccess))
    rc = 4;
  if (rc == 0) {
    const double bytes_per_cu = 8.0 * 64.0 * 16.0 * 8.0 * iters;  // waves x lanes x 16 B x 8 reads x iters
    *bytes_per_ns_per_cu = bytes_per_cu * launches / (ms * 1e6);
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  (void)hipFree(out);
  return rc;
}

}  // extern "C"
