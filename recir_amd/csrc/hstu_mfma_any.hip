// General MFMA kernels (hstu_mfma_any.h): the instantiations without a bias table for rows that start
// at multiples of 16 bytes, and the two entry points the host code calls, which pick the translation
// unit by the presence of a bias and by the alignment of the rows.
#define HSTU_ANY_HAS_RAB 0
#define HSTU_ANY_ALIGNED 1
#include "hstu_mfma_any_launch.h"

namespace recir_hstu {

bool launch_mfma_any_fwd(int dtype, int dp, bool aligned, dim3 grid, hipStream_t stream, const Params& p) {
  BwdParams bp;
  memset(&bp, 0, sizeof(bp));
  bp.f = p;
  if (aligned)
    return p.rab ? launch_mfma_any_fwd_as<true, true>(dtype, dp, grid, stream, bp) : launch_mfma_any_fwd_as<false, true>(dtype, dp, grid, stream, bp);
  return p.rab ? launch_mfma_any_fwd_as<true, false>(dtype, dp, grid, stream, bp) : launch_mfma_any_fwd_as<false, false>(dtype, dp, grid, stream, bp);
}

bool launch_mfma_any_bwd(int dtype, int dp, bool aligned, dim3 grid_q, dim3 grid_k, hipStream_t stream, const BwdParams& bq, const BwdParams& bk) {
  if (aligned)
    return bq.f.rab ? launch_mfma_any_bwd_as<true, true>(dtype, dp, grid_q, grid_k, stream, bq, bk)
                    : launch_mfma_any_bwd_as<false, true>(dtype, dp, grid_q, grid_k, stream, bq, bk);
  return bq.f.rab ? launch_mfma_any_bwd_as<true, false>(dtype, dp, grid_q, grid_k, stream, bq, bk)
                  : launch_mfma_any_bwd_as<false, false>(dtype, dp, grid_q, grid_k, stream, bq, bk);
}

}  // namespace recir_hstu
