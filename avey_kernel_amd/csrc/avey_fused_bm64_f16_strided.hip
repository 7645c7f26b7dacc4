// Fused kernel variants with 64 query rows per workgroup, f16, strided z_tr / z_tl.
#include "avey_fused.h"

namespace avey {

template <>
hipError_t launch_fused_bm<_Float16, 64, true>(const FwdParams& p, int nk, int64_t grid, hipStream_t s) {
  return launch_fused_nk<_Float16, 64, true>(p, nk, grid, s);
}

}  // namespace avey
