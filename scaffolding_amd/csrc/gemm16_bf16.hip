// gemm16_bf16.hip — bf16-input instantiations of the 16-bit GEMM family.
#include "gemm16_inst.hpp"

namespace sf {

int launch_gemm16_bf16(sf_dtype out, bool a_kmajor, bool b_kmajor, int cfg, const GemmParams& p, unsigned gx,
                       unsigned gy, hipStream_t st) {
  return launch16_in<BF16>(SF_BF16, out, a_kmajor, b_kmajor, cfg, p, gx, gy, st);
}

}  // namespace sf
