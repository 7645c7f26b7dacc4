// Fused kernel variants with 16 query rows per workgroup (bf16 and fp16).
#include "avey_fused.h"

namespace avey {

template <>
hipError_t launch_fused_bm<16>(const FwdParams& p, int dtype, int nk, int64_t grid, hipStream_t s) {
  if (dtype == AVEY_DTYPE_BF16) return launch_fused_nk<__bf16, 16>(p, nk, grid, s);
  if (dtype == AVEY_DTYPE_F16) return launch_fused_nk<_Float16, 16>(p, nk, grid, s);
  return hipErrorInvalidValue;
}

}  // namespace avey
