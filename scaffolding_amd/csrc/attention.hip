// attention.hip — launcher of the fused attention kernel (attention.hpp).
#include "sf_internal.hpp"
#include "attention.hpp"

namespace sf {

int launch_attention(const void* Q, const void* K, const void* V, void* O, int64_t batch, int64_t Sq,
                     int64_t Sk, int64_t sQ, int64_t sK, int64_t sV, int64_t sO, int64_t ldq, int64_t ldk,
                     int64_t ldv, int64_t ldo, float scale, sf_dtype dt, hipStream_t st) {
  AttnParams p;
  p.Q = Q; p.K = K; p.V = V; p.O = O;
  p.sQ = sQ; p.sK = sK; p.sV = sV; p.sO = sO;
  p.ldq = (int)ldq; p.ldk = (int)ldk; p.ldv = (int)ldv; p.ldo = (int)ldo;
  p.Sq = (int)Sq; p.Sk = (int)Sk;
  p.scale_log2e = scale * 1.4426950408889634f;
  const unsigned gx = (unsigned)((Sq + 255) / 256);
  for (int64_t b0 = 0; b0 < batch; b0 += 65535) {
    const int64_t nb = (batch - b0) < 65535 ? (batch - b0) : 65535;
    AttnParams q = p;
    q.Q = static_cast<const uint16_t*>(Q) + b0 * sQ;
    q.K = static_cast<const uint16_t*>(K) + b0 * sK;
    q.V = static_cast<const uint16_t*>(V) + b0 * sV;
    q.O = static_cast<uint16_t*>(O) + b0 * sO;
    if (dt == SF_F16)
      hipLaunchKernelGGL((attn64_kernel<F16>), dim3(gx, (unsigned)nb), dim3(256), 0, st, q);
    else
      hipLaunchKernelGGL((attn64_kernel<BF16>), dim3(gx, (unsigned)nb), dim3(256), 0, st, q);
    const int rc = check_launch("attention");
    if (rc != SF_OK) return rc;
  }
  return SF_OK;
}

}  // namespace sf
