// Fused kernel variants with 32 query rows per workgroup, bf16, strided z_tr / z_tl.
#include "avey_fused.h"

namespace avey {

template <>
hipError_t launch_fused_bm<__bf16, 32, true>(const FwdParams& p, int nk, int64_t grid, hipStream_t s) {
  return launch_fused_nk<__bf16, 32, true>(p, nk, grid, s);
}

}  // namespace avey
