// Dispatch of the fused bf16 / fp16 kernel to the compiled query-tile heights.
#include "avey_fused.h"

namespace avey {

template <typename T16, bool STRIDED>
static hipError_t launch_fused_t(const FwdParams& p, const Plan& plan, hipStream_t s) {
  const int nk = plan.bd / 32;
  switch (plan.bm) {
    case 16: return launch_fused_bm<T16, 16, STRIDED>(p, nk, plan.grid, s);
    case 32: return launch_fused_bm<T16, 32, STRIDED>(p, nk, plan.grid, s);
    case 64: return launch_fused_bm<T16, 64, STRIDED>(p, nk, plan.grid, s);
    default: return hipErrorInvalidConfiguration;
  }
}

hipError_t launch_fused(const FwdParams& p, int dtype, const Plan& plan, hipStream_t s) {
  // Contiguous operands (the common case) run the instantiations without strides.
  const int64_t row = p.D, item = p.C * p.D;
  const bool strided = p.zrs != row || p.zbs != item || (p.gate != nullptr && (p.grs != row || p.gbs != item));
  if (dtype == AVEY_DTYPE_BF16)
    return strided ? launch_fused_t<__bf16, true>(p, plan, s) : launch_fused_t<__bf16, false>(p, plan, s);
  if (dtype == AVEY_DTYPE_F16)
    return strided ? launch_fused_t<_Float16, true>(p, plan, s) : launch_fused_t<_Float16, false>(p, plan, s);
  return hipErrorInvalidValue;
}

}  // namespace avey
