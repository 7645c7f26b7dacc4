// Fused kernel variants with 16 query rows per workgroup, f16, strided z_tr / z_tl.
#include "avey_fused16.h"

namespace avey {

template <>
hipError_t launch_fused_bm<_Float16, 16, true>(const FwdParams& p, int nk, int64_t grid, hipStream_t s) {
  return launch_fused16<_Float16, true>(p, nk, grid, s);
}

}  // namespace avey
