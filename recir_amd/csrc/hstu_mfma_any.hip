// Instantiations and launchers of the MFMA kernels for head dims other than 128, fp16 values and the
// masks the head-dim-128 kernels do not take (hstu_mfma_any.h).  A translation unit of its own so
// that it compiles beside the other one.
#include <cstring>

#include "hstu_mfma_any.h"

namespace recir_hstu {

namespace {

template <int MODE, bool F16>
bool launch_mode(int dp, dim3 grid, hipStream_t stream, const BwdParams& bp) {
  // the key-stationary mode that produces dK and dV together stops at 128; its halves take 256
  constexpr bool small = MODE != ANY_DV && MODE != ANY_DK;
  constexpr bool large = MODE != ANY_DKV;
  switch (dp) {
    case 32:
      if constexpr (small) { hipLaunchKernelGGL((hstu_mfma_any<MODE, F16, 32>), grid, dim3(256), 0, stream, bp); return true; }
      return false;
    case 64:
      if constexpr (small) { hipLaunchKernelGGL((hstu_mfma_any<MODE, F16, 64>), grid, dim3(256), 0, stream, bp); return true; }
      return false;
    case 128:
      if constexpr (small) { hipLaunchKernelGGL((hstu_mfma_any<MODE, F16, 128>), grid, dim3(256), 0, stream, bp); return true; }
      return false;
    case 256:
      if constexpr (large) { hipLaunchKernelGGL((hstu_mfma_any<MODE, F16, 256>), grid, dim3(256), 0, stream, bp); return true; }
      return false;
    default: return false;
  }
}

template <bool F16>
bool launch_bwd(int dp, dim3 grid_q, dim3 grid_k, hipStream_t stream, const BwdParams& bq, const BwdParams& bk) {
  if (dp <= 128) return launch_mode<ANY_DKV, F16>(dp, grid_k, stream, bk) && launch_mode<ANY_DQ, F16>(dp, grid_q, stream, bq);
  return launch_mode<ANY_DV, F16>(dp, grid_k, stream, bk) && launch_mode<ANY_DK, F16>(dp, grid_k, stream, bk) &&
         launch_mode<ANY_DQ, F16>(dp, grid_q, stream, bq);
}

}  // namespace

bool launch_mfma_any_fwd(int dtype, int dp, dim3 grid, hipStream_t stream, const Params& p) {
  BwdParams bp;
  memset(&bp, 0, sizeof(bp));
  bp.f = p;
  if (dtype == RECIR_HSTU_DTYPE_FP16) return launch_mode<ANY_FWD, true>(dp, grid, stream, bp);
  if (dtype == RECIR_HSTU_DTYPE_BF16) return launch_mode<ANY_FWD, false>(dp, grid, stream, bp);
  return false;
}

bool launch_mfma_any_bwd(int dtype, int dp, dim3 grid_q, dim3 grid_k, hipStream_t stream, const BwdParams& bq, const BwdParams& bk) {
  if (dtype == RECIR_HSTU_DTYPE_FP16) return launch_bwd<true>(dp, grid_q, grid_k, stream, bq, bk);
  if (dtype == RECIR_HSTU_DTYPE_BF16) return launch_bwd<false>(dp, grid_q, grid_k, stream, bq, bk);
  return false;
}

}  // namespace recir_hstu
