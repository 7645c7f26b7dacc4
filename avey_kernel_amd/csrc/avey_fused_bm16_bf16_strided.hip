// Fused kernel variants with 16 query rows per workgroup, bf16, strided z_tr / z_tl.
#include "avey_fused16.h"

namespace avey {

template <>
hipError_t launch_fused_bm<__bf16, 16, true>(const FwdParams& p, int nk, int64_t grid, hipStream_t s) {
  return launch_fused16<__bf16, true>(p, nk, grid, s);
}

}  // namespace avey
