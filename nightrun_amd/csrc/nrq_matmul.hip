// Batched matmul (prefill): y[b][r] = dot(W[r,:], xs[b]).
// The reference guarantees matmul == per-token matvec bit for bit
// (kernels.rs:84-90, kquant.rs:566-569). Scalar order runs the int8-MFMA tile
// kernels (nrq_mmt.hip, nrq_mmq.hip). AVX2 order runs the int8-MFMA tiles of
// nrq_mma.hip from two tokens, and the decode kernel for one: both equal the
// 1-wide AVX2 dot per token, as the reference's 4-wide tiles do
// (kernels.rs:222-223).
#include "nrq_device.h"
#include "nrq_launch.h"

namespace nrq {

int launch_matmul(int dtype, int order, const MatmulLaunch& L) {
  if (L.rows <= 0 || L.bpr <= 0 || L.batch <= 0) return 0;
  if (order == kOrderScalar) return launch_mmq(dtype, L);
  if (L.batch >= 2) return launch_mma(dtype, L);
  const size_t xb = dtype == kQ8_0 ? (size_t)kQ8_0Bytes : (size_t)kQ8KBytes;
  for (int b = 0; b < L.batch; b++) {
    MatvecLaunch M;
    M.w = L.w;
    M.x = (const uint8_t*)L.xs + (size_t)b * L.bpr * xb;
    M.y = L.y + (size_t)b * L.rows;
    M.rows = L.rows;
    M.bpr = L.bpr;
    M.tile_rows = 0;
    M.stream = L.stream;
    int rc = launch_matvec(dtype, order, M);
    if (rc) return rc;
  }
  return 0;
}

}  // namespace nrq
