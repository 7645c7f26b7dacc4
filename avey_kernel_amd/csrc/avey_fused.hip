// Dispatch of the fused bf16 / fp16 kernel to the compiled query-tile heights.
#include "avey_fused.h"

namespace avey {

template <typename T16>
static hipError_t launch_fused_t(const FwdParams& p, const Plan& plan, hipStream_t s) {
  const int nk = plan.bd / 32;
  switch (plan.bm) {
    case 16: return launch_fused_bm<T16, 16>(p, nk, plan.grid, s);
    case 32: return launch_fused_bm<T16, 32>(p, nk, plan.grid, s);
    case 64: return launch_fused_bm<T16, 64>(p, nk, plan.grid, s);
    default: return hipErrorInvalidConfiguration;
  }
}

hipError_t launch_fused(const FwdParams& p, int dtype, const Plan& plan, hipStream_t s) {
  if (dtype == AVEY_DTYPE_BF16) return launch_fused_t<__bf16>(p, plan, s);
  if (dtype == AVEY_DTYPE_F16) return launch_fused_t<_Float16>(p, plan, s);
  return hipErrorInvalidValue;
}

}  // namespace avey
