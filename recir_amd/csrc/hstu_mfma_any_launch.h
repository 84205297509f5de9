// Launch code of the general MFMA kernels for one value of HAS_RAB and of ALIGNED; included by the four
// translation units that hold the instantiations (HSTU_ANY_HAS_RAB and HSTU_ANY_ALIGNED defined to 0 or 1
// before the include).
#pragma once
#include <cstring>

#include "hstu_mfma_any.h"

namespace recir_hstu {

namespace {

// Which (mode, element type, padded head dim) are instantiated.  The key-stationary mode that produces
// dK and dV together holds two operand sets and two accumulators: it stops at 128 (fp32: 64), and the
// largest padded head dim (256, fp32: 128 -- its LDS tiles are twice as wide) takes its two halves.
template <int MODE, int ELT, int DP>
constexpr bool any_instantiated() {
  constexpr int top = ELT == ANY_F32 ? 128 : 256;
  if (MODE == ANY_DKV) return DP < top;
  if (MODE == ANY_DV || MODE == ANY_DK) return DP == top;
  return DP <= top;
}

template <int MODE, int ELT, int DP>
bool launch_one(dim3 grid, hipStream_t stream, const BwdParams& bp) {
  if constexpr (any_instantiated<MODE, ELT, DP>()) {
    hipLaunchKernelGGL((hstu_mfma_any<MODE, ELT, DP, HSTU_ANY_HAS_RAB != 0, HSTU_ANY_ALIGNED != 0>), grid, dim3(256), 0, stream, bp);
    return true;
  }
  return false;
}

template <int MODE, int ELT>
bool launch_mode(int dp, dim3 grid, hipStream_t stream, const BwdParams& bp) {
  switch (dp) {
    case 32: return launch_one<MODE, ELT, 32>(grid, stream, bp);
    case 64: return launch_one<MODE, ELT, 64>(grid, stream, bp);
    case 128: return launch_one<MODE, ELT, 128>(grid, stream, bp);
    case 256: return launch_one<MODE, ELT, 256>(grid, stream, bp);
    default: return false;
  }
}

template <int ELT>
bool launch_bwd(int dp, dim3 grid_q, dim3 grid_k, hipStream_t stream, const BwdParams& bq, const BwdParams& bk) {
  if (dp < (ELT == ANY_F32 ? 128 : 256))
    return launch_mode<ANY_DKV, ELT>(dp, grid_k, stream, bk) && launch_mode<ANY_DQ, ELT>(dp, grid_q, stream, bq);
  return launch_mode<ANY_DV, ELT>(dp, grid_k, stream, bk) && launch_mode<ANY_DK, ELT>(dp, grid_k, stream, bk) &&
         launch_mode<ANY_DQ, ELT>(dp, grid_q, stream, bq);
}

}  // namespace

template <>
bool launch_mfma_any_fwd_as<HSTU_ANY_HAS_RAB != 0, HSTU_ANY_ALIGNED != 0>(int dtype, int dp, dim3 grid, hipStream_t stream, const BwdParams& bp) {
  if (dtype == RECIR_HSTU_DTYPE_FP16) return launch_mode<ANY_FWD, ANY_F16>(dp, grid, stream, bp);
  if (dtype == RECIR_HSTU_DTYPE_BF16) return launch_mode<ANY_FWD, ANY_BF16>(dp, grid, stream, bp);
  if (dtype == RECIR_HSTU_DTYPE_FP32) return launch_mode<ANY_FWD, ANY_F32>(dp, grid, stream, bp);
  return false;
}

template <>
bool launch_mfma_any_bwd_as<HSTU_ANY_HAS_RAB != 0, HSTU_ANY_ALIGNED != 0>(int dtype, int dp, dim3 grid_q, dim3 grid_k, hipStream_t stream,
                                                                             const BwdParams& bq, const BwdParams& bk) {
  if (dtype == RECIR_HSTU_DTYPE_FP16) return launch_bwd<ANY_F16>(dp, grid_q, grid_k, stream, bq, bk);
  if (dtype == RECIR_HSTU_DTYPE_BF16) return launch_bwd<ANY_BF16>(dp, grid_q, grid_k, stream, bq, bk);
  if (dtype == RECIR_HSTU_DTYPE_FP32) return launch_bwd<ANY_F32>(dp, grid_q, grid_k, stream, bq, bk);
  return false;
}

}  // namespace recir_hstu
