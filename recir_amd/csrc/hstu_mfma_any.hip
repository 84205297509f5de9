// General MFMA kernels (hstu_mfma_any.h): the instantiations without a bias table, and the two entry
// points the host code calls, which pick the translation unit by the presence of a bias.
#define HSTU_ANY_HAS_RAB 0
#include "hstu_mfma_any_launch.h"

namespace recir_hstu {

bool launch_mfma_any_fwd(int dtype, int dp, dim3 grid, hipStream_t stream, const Params& p) {
  BwdParams bp;
  memset(&bp, 0, sizeof(bp));
  bp.f = p;
  return p.rab ? launch_mfma_any_fwd_as<true>(dtype, dp, grid, stream, bp) : launch_mfma_any_fwd_as<false>(dtype, dp, grid, stream, bp);
}

bool launch_mfma_any_bwd(int dtype, int dp, dim3 grid_q, dim3 grid_k, hipStream_t stream, const BwdParams& bq, const BwdParams& bk) {
  return bq.f.rab ? launch_mfma_any_bwd_as<true>(dtype, dp, grid_q, grid_k, stream, bq, bk)
                  : launch_mfma_any_bwd_as<false>(dtype, dp, grid_q, grid_k, stream, bq, bk);
}

}  // namespace recir_hstu
