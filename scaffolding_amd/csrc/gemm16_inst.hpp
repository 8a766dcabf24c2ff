// gemm16_inst.hpp — instantiation + launch table of the 16-bit GEMM for one
// input type (included by gemm16_bf16.hip and gemm16_f16.hip).
#pragma once

#include "sf_internal.hpp"
#include "gemm16nt_4w.hpp"
#include "gemm16nt_k64.hpp"
#include "gemm16nt_pp.hpp"
#include "skinny16.hpp"

namespace sf {

// Row-segment skinny stream: NW = K / 512 waves (K in {2048, 4096, 8192}),
// an 8-tile LDS ring per wave where it fits (NW * 16 KB), else 4 tiles.
template <typename TIn, typename TOut>
static int launch_skinny_line(const GemmParams& p, const dim3& g, hipStream_t st) {
  // x in whole 128-byte lines (a round trip through LDS) only where it has
  // more than 8 rows: at M <= 8 the MFMA-layout loads touch as few lines.
  const bool xline = p.M > 8;
  switch (p.K) {
    case 2048:
      if (xline) hipLaunchKernelGGL((skinny16l_kernel<TIn, TOut, 4, 8, true>), g, dim3(256), 0, st, p);
      else hipLaunchKernelGGL((skinny16l_kernel<TIn, TOut, 4, 8, false>), g, dim3(256), 0, st, p);
      return SF_OK;
    case 4096:
      if (xline) hipLaunchKernelGGL((skinny16l_kernel<TIn, TOut, 8, 8, true>), g, dim3(512), 0, st, p);
      else hipLaunchKernelGGL((skinny16l_kernel<TIn, TOut, 8, 8, false>), g, dim3(512), 0, st, p);
      return SF_OK;
    case 8192:
      if (xline) hipLaunchKernelGGL((skinny16l_kernel<TIn, TOut, 16, 4, true>), g, dim3(1024), 0, st, p);
      else hipLaunchKernelGGL((skinny16l_kernel<TIn, TOut, 16, 4, false>), g, dim3(1024), 0, st, p);
      return SF_OK;
  }
  return fail(SF_ERR_INVALID_ARG, "skinny line kernel: K=%d is not 2048, 4096 or 8192", p.K);
}

// KM: B K-contiguous; AKM: A K-contiguous (false: A stored K x M).  The
// LDS-DMA, skinny and row-segment kernels need both K-contiguous.
template <typename TIn, typename TOut, bool KM, bool AKM>
static int launch16_t(int cfg, const GemmParams& p, unsigned gx, unsigned gy, hipStream_t st) {
  const dim3 g(gx, gy);
  switch (cfg) {
    case TILE_256x256:
      hipLaunchKernelGGL((gemm16_kernel<TIn, TOut, 256, 256, 2, 4, KM, true, AKM>), g, dim3(512), 0, st, p);
      break;
    case TILE_256x128:
      hipLaunchKernelGGL((gemm16_kernel<TIn, TOut, 256, 128, 4, 2, KM, true, AKM>), g, dim3(512), 0, st, p);
      break;
    case TILE_128x128:
      hipLaunchKernelGGL((gemm16_kernel<TIn, TOut, 128, 128, 2, 2, KM, true, AKM>), g, dim3(256), 0, st, p);
      break;
    case TILE_256x64:
      hipLaunchKernelGGL((gemm16_kernel<TIn, TOut, 256, 64, 4, 1, KM, true, AKM>), g, dim3(256), 0, st, p);
      break;
    case TILE_64x64:
      hipLaunchKernelGGL((gemm16_kernel<TIn, TOut, 64, 64, 2, 2, KM, true, AKM>), g, dim3(256), 0, st, p);
      break;
    case TILE_GENERIC:
      hipLaunchKernelGGL((gemm16_kernel<TIn, TOut, 64, 64, 2, 2, KM, false, AKM>), g, dim3(256), 0, st, p);
      break;
    case TILE_NT_BIG:
      if constexpr (KM && AKM) {
        if (p.persist > 0) {
          if (p.K % 128 != 0 || p.persist % kNumXcd != 0 || gy != 1)
            return fail(SF_ERR_INVALID_ARG, "persistent 256x256 kernel: K %% 128, grid %% 8 and batch 1 required");
          // a split tail shares its final sum among the parts (SHARED)
          if (p.split > 0)
            hipLaunchKernelGGL((gemm16nt_pp_kernel<TIn, TOut, 2, true, true, true, true>), g, dim3(512), 0, st, p);
          else
            hipLaunchKernelGGL((gemm16nt_pp_kernel<TIn, TOut, 2, true, true, true>), g, dim3(512), 0, st, p);
          break;
        }
      }
      if constexpr (AKM && !KM) {  // NN (dX = dY W): persistent tiles as for NT
        if (p.persist > 0) {
          if (p.K % 128 != 0 || p.persist % kNumXcd != 0 || gy != 1)
            return fail(SF_ERR_INVALID_ARG, "persistent 256x256 kernel: K %% 128, grid %% 8 and batch 1 required");
          if (p.split > 0)
            hipLaunchKernelGGL((gemm16nt_pp_kernel<TIn, TOut, 2, true, false, true, true>), g, dim3(512), 0, st, p);
          else
            hipLaunchKernelGGL((gemm16nt_pp_kernel<TIn, TOut, 2, true, false, true>), g, dim3(512), 0, st, p);
          break;
        }
      }
      if (p.K % 128 != 0 && (AKM || KM))
        return fail(SF_ERR_INVALID_ARG, "the 256x256 LDS-DMA kernel needs K %% 128 == 0 with a K-contiguous operand");
      if constexpr (KM && AKM) {
        if (p.wave4 > 0) {  // the planner's choice: one workgroup per tile, no split
          if (p.split > 0 || p.K < 192)
            return fail(SF_ERR_INVALID_ARG, "one-wave-per-SIMD 256x256 kernel: no split, K >= 192");
          switch (epi_act(p.epi)) {
            case ACT_SILU:
              hipLaunchKernelGGL((gemm16nt_4w_kernel<TIn, TOut, ACT_SILU>), g, dim3(256), 0, st, p);
              break;
            case ACT_GELU:
              hipLaunchKernelGGL((gemm16nt_4w_kernel<TIn, TOut, ACT_GELU>), g, dim3(256), 0, st, p);
              break;
            default:
              hipLaunchKernelGGL((gemm16nt_4w_kernel<TIn, TOut, ACT_NONE>), g, dim3(256), 0, st, p);
              break;
          }
          break;
        }
      }
      hipLaunchKernelGGL((gemm16nt_pp_kernel<TIn, TOut, 2, AKM, KM>), g, dim3(512), 0, st, p);
      break;
    case TILE_NT_K64:
      if constexpr (KM && AKM) {
        if (p.K != 64) return fail(SF_ERR_INVALID_ARG, "the K = 64 kernel got K = %d", p.K);
        switch (epi_act(p.epi)) {
          case ACT_SILU:
            hipLaunchKernelGGL((gemm16nt_k64_kernel<TIn, TOut, ACT_SILU>), g, dim3(256), 0, st, p);
            break;
          case ACT_GELU:
            hipLaunchKernelGGL((gemm16nt_k64_kernel<TIn, TOut, ACT_GELU>), g, dim3(256), 0, st, p);
            break;
          default:
            hipLaunchKernelGGL((gemm16nt_k64_kernel<TIn, TOut, ACT_NONE>), g, dim3(256), 0, st, p);
            break;
        }
        break;
      }
      return fail(SF_ERR_UNSUPPORTED, "the K = 64 kernel needs K-contiguous A and B");
    case TILE_SKINNY:
      if constexpr (KM && AKM) {
        // grid.x = ceil(N / 32): 2 row blocks per workgroup, K split over 4 waves.
        hipLaunchKernelGGL((skinny16_kernel<TIn, TOut, 4, 2, 8>), g, dim3(256), 0, st, p);
        break;
      }
      return fail(SF_ERR_UNSUPPORTED, "skinny kernels need K-contiguous A and B");
    case TILE_SKINNY_LINE:
      if constexpr (KM && AKM) {
        const int rc = launch_skinny_line<TIn, TOut>(p, g, st);
        if (rc != SF_OK) return rc;
        break;
      }
      return fail(SF_ERR_UNSUPPORTED, "skinny kernels need K-contiguous A and B");
    default:
      return fail(SF_ERR_INVALID_ARG, "unknown tile config %d", cfg);
  }
  return check_launch(tile_name(cfg));
}

// Only the tiles the dispatcher picks for an fp32 output of 16-bit inputs.
template <typename TIn, bool KM, bool AKM>
static int launch16_f32out(int cfg, const GemmParams& p, unsigned gx, unsigned gy, hipStream_t st) {
  const dim3 g(gx, gy);
  switch (cfg) {
    case TILE_128x128:
      hipLaunchKernelGGL((gemm16_kernel<TIn, float, 128, 128, 2, 2, KM, true, AKM>), g, dim3(256), 0, st, p);
      break;
    case TILE_GENERIC:
      hipLaunchKernelGGL((gemm16_kernel<TIn, float, 64, 64, 2, 2, KM, false, AKM>), g, dim3(256), 0, st, p);
      break;
    case TILE_SKINNY:
      if constexpr (KM && AKM) {
        hipLaunchKernelGGL((skinny16_kernel<TIn, float, 4, 2, 8>), g, dim3(256), 0, st, p);
        break;
      }
      return fail(SF_ERR_UNSUPPORTED, "skinny kernels need K-contiguous A and B");
    case TILE_SKINNY_LINE:
      if constexpr (KM && AKM) {
        const int rc = launch_skinny_line<TIn, float>(p, g, st);
        if (rc != SF_OK) return rc;
        break;
      }
      return fail(SF_ERR_UNSUPPORTED, "skinny kernels need K-contiguous A and B");
    default:
      return fail(SF_ERR_INVALID_ARG, "tile config %d has no fp32-output variant", cfg);
  }
  return check_launch(tile_name(cfg));
}

template <typename TIn>
static int launch16_in(sf_dtype in, sf_dtype out, bool a_kmajor, bool b_kmajor, int cfg, const GemmParams& p,
                       unsigned gx, unsigned gy, hipStream_t st) {
  (void)in;
  if (out == SF_F32) {
    if (a_kmajor)
      return b_kmajor ? launch16_f32out<TIn, true, true>(cfg, p, gx, gy, st)
                      : launch16_f32out<TIn, false, true>(cfg, p, gx, gy, st);
    return b_kmajor ? launch16_f32out<TIn, true, false>(cfg, p, gx, gy, st)
                    : launch16_f32out<TIn, false, false>(cfg, p, gx, gy, st);
  }
  if (a_kmajor)
    return b_kmajor ? launch16_t<TIn, TIn, true, true>(cfg, p, gx, gy, st)
                    : launch16_t<TIn, TIn, false, true>(cfg, p, gx, gy, st);
  return b_kmajor ? launch16_t<TIn, TIn, true, false>(cfg, p, gx, gy, st)
                  : launch16_t<TIn, TIn, false, false>(cfg, p, gx, gy, st);
}

}  // namespace sf
