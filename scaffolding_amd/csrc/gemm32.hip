// gemm32.hip — fp32 GEMM instantiations and launcher.
#include "gemm32.hpp"
#include "gemm32dma.hpp"
#include "gemm32small.hpp"
#include "sf_internal.hpp"

namespace sf {

template <bool KM, bool AKM>
static int launch32_t(int cfg, const GemmParams& p, unsigned gx, unsigned gy, hipStream_t st) {
  const dim3 g(gx, gy);
  switch (cfg) {
    case TILE_128x128:
      hipLaunchKernelGGL((gemm32_kernel<128, 128, 2, 2, KM, true, AKM>), g, dim3(256), 0, st, p);
      break;
    case TILE_64x64:
      hipLaunchKernelGGL((gemm32_kernel<64, 64, 2, 2, KM, true, AKM>), g, dim3(256), 0, st, p);
      break;
    case TILE_GENERIC:
      hipLaunchKernelGGL((gemm32_kernel<64, 64, 2, 2, KM, false, AKM>), g, dim3(256), 0, st, p);
      break;
    case TILE32_SMALL1:
    case TILE32_SMALL2:
    case TILE32_DMA:
    case TILE32_DMA_SPLIT:
      if constexpr (AKM) {
        if (cfg == TILE32_SMALL1)
          hipLaunchKernelGGL((gemm32small_kernel<1, KM, 4>), g, dim3(256), 0, st, p);
        else if (cfg == TILE32_SMALL2)
          hipLaunchKernelGGL((gemm32small_kernel<2, KM, 8>), g, dim3(512), 0, st, p);
        else if (cfg == TILE32_DMA)
          hipLaunchKernelGGL((gemm32dma_kernel<64, 64, KM, 2, 2>), g, dim3(512), 0, st, p);
        else
          hipLaunchKernelGGL((gemm32dma_kernel<64, 64, KM, 3, 1>), g, dim3(256), 0, st, p);
        break;
      }
      return fail(SF_ERR_INVALID_ARG, "tile config %d needs a K-contiguous A", cfg);
    default:
      return fail(SF_ERR_INVALID_ARG, "tile config %d has no fp32 variant", cfg);
  }
  return check_launch(tile_name(cfg));
}

int launch_gemm32(bool a_kmajor, bool b_kmajor, int cfg, const GemmParams& p, int64_t batch, hipStream_t st) {
  if (p.split > kMaxSplit32 || (p.split > 0 && batch != 1) || (cfg == TILE32_DMA && p.split > 0) ||
      (cfg == TILE32_DMA && (p.K / 32) % 2 != 0))
    return fail(SF_ERR_INVALID_ARG, "fp32 plan: split %d / batch %lld / K %d do not fit tile config %d", p.split,
                (long long)batch, p.K, cfg);
  const unsigned gx = static_cast<unsigned>(p.tiles_m) * static_cast<unsigned>(p.tiles_n) *
                     static_cast<unsigned>(p.split > 0 ? p.split : 1);
  // grid.y is limited to 65535: walk the batch in chunks.
  for (int64_t b0 = 0; b0 < batch; b0 += 65535) {
    const int64_t nb = (batch - b0) < 65535 ? (batch - b0) : 65535;
    GemmParams q = p;
    q.A = static_cast<const float*>(p.A) + b0 * p.sA;
    q.B = static_cast<const float*>(p.B) + b0 * p.sB;
    q.C = static_cast<float*>(p.C) + b0 * p.sC;
    if (p.res != nullptr) q.res = static_cast<const float*>(p.res) + b0 * p.sR;
    const unsigned gy = static_cast<unsigned>(nb);
    const int rc = a_kmajor ? (b_kmajor ? launch32_t<true, true>(cfg, q, gx, gy, st)
                                        : launch32_t<false, true>(cfg, q, gx, gy, st))
                            : (b_kmajor ? launch32_t<true, false>(cfg, q, gx, gy, st)
                                        : launch32_t<false, false>(cfg, q, gx, gy, st));
    if (rc != SF_OK) return rc;
  }
  return SF_OK;
}

}  // namespace sf
