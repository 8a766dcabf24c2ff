// attention.hip — launcher of the fused attention kernel (attention.hpp).
#include "sf_internal.hpp"
#include "attention.hpp"

namespace sf {

int launch_attention(const AttnShape& a, float scale, sf_dtype dt, hipStream_t st) {
  AttnParams p;
  p.Q = a.Q; p.K = a.K; p.V = a.V; p.O = a.O;
  p.sQ = a.sQ; p.sK = a.sK; p.sV = a.sV; p.sO = a.sO;
  p.hQ = a.hQ; p.hK = a.hK; p.hV = a.hV; p.hO = a.hO;
  p.H = (int)a.heads;
  p.ldq = (int)a.ldq; p.ldk = (int)a.ldk; p.ldv = (int)a.ldv; p.ldo = (int)a.ldo;
  p.Sq = (int)a.Sq; p.Sk = (int)a.Sk;
  p.D = (int)a.D;
  p.scale_log2e = scale * 1.4426950408889634f;
  const unsigned gx = (unsigned)((a.Sq + 255) / 256);
  const int64_t pairs = a.batch * a.heads;
  for (int64_t y0 = 0; y0 < pairs; y0 += 65535) {
    const int64_t ny = (pairs - y0) < 65535 ? (pairs - y0) : 65535;
    p.y0 = y0;
    if (dt == SF_F16)
      hipLaunchKernelGGL((attn64_kernel<F16>), dim3(gx, (unsigned)ny), dim3(256), 0, st, p);
    else
      hipLaunchKernelGGL((attn64_kernel<BF16>), dim3(gx, (unsigned)ny), dim3(256), 0, st, p);
    const int rc = check_launch("attention");
    if (rc != SF_OK) return rc;
  }
  return SF_OK;
}

}  // namespace sf
