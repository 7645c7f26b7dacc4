// Dispatch of the fused bf16 / fp16 kernel to the compiled query-tile heights.
#include "avey_fused.h"

namespace avey {

hipError_t launch_fused(const FwdParams& p, int dtype, const Plan& plan, hipStream_t s) {
  const int nk = plan.bd / 32;
  switch (plan.bm) {
    case 16: return launch_fused_bm<16>(p, dtype, nk, plan.grid, s);
    case 32: return launch_fused_bm<32>(p, dtype, nk, plan.grid, s);
    case 64: return launch_fused_bm<64>(p, dtype, nk, plan.grid, s);
    default: return hipErrorInvalidConfiguration;
  }
}

}  // namespace avey
