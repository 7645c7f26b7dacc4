// Fused 16-row variants with the enricher gate formed in the epilogue, bf16, contiguous operands.
#include "avey_fused16.h"

namespace avey {

template <>
hipError_t launch_fused16_enriched<__bf16, false>(const FwdParams& p, int nk, int64_t grid, hipStream_t s) {
  return launch_fused16<__bf16, false, true>(p, nk, grid, s);
}

}  // namespace avey
