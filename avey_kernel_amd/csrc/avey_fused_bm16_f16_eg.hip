// Fused 16-row variants with the enricher gate formed in the epilogue, fp16, contiguous operands.
#include "avey_fused16.h"

namespace avey {

template <>
hipError_t launch_fused16_enriched<_Float16, false>(const FwdParams& p, int nk, int64_t grid, hipStream_t s) {
  return launch_fused16<_Float16, false, true>(p, nk, grid, s);
}

}  // namespace avey
