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

static bool strided_operands(const FwdParams& p) {
  const int64_t row = p.D, item = p.C * p.D;
  return p.zrs != row || p.zbs != item || (p.gate != nullptr && (p.grs != row || p.gbs != item));
}

hipError_t launch_fused(const FwdParams& p, int dtype, const Plan& plan, hipStream_t s) {
  // Contiguous operands (the common case) run the instantiations without strides.
  const bool strided = strided_operands(p);
  if (dtype == AVEY_DTYPE_BF16)
    return strided ? launch_fused_t<__bf16, true>(p, plan, s) : launch_fused_t<__bf16, false>(p, plan, s);
  if (dtype == AVEY_DTYPE_F16)
    return strided ? launch_fused_t<_Float16, true>(p, plan, s) : launch_fused_t<_Float16, false>(p, plan, s);
  return hipErrorInvalidValue;
}

// Only the 16-row variants form the enricher gate (plan.bm is 16 for these calls).
hipError_t launch_fused_enriched(const FwdParams& p, int dtype, const Plan& plan, hipStream_t s) {
  if (plan.bm != 16) return hipErrorInvalidConfiguration;
  const int nk = plan.bd / 32;
  const bool strided = strided_operands(p);
  if (dtype == AVEY_DTYPE_BF16)
    return strided ? launch_fused16_enriched<__bf16, true>(p, nk, plan.grid, s)
                   : launch_fused16_enriched<__bf16, false>(p, nk, plan.grid, s);
  if (dtype == AVEY_DTYPE_F16)
    return strided ? launch_fused16_enriched<_Float16, true>(p, nk, plan.grid, s)
                   : launch_fused16_enriched<_Float16, false>(p, nk, plan.grid, s);
  return hipErrorInvalidValue;
}

}  // namespace avey
