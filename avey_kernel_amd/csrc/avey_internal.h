// Internal launch interface between the C ABI (avey_capi.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "avey_hip.h"

namespace avey {

// Everything a kernel needs, by value. Pointers are device pointers.
struct FwdParams {
  const void* z;        // z_tr [B][C][D]
  const void* v;        // [C][C] or null
  const void* gate;     // z_tl [B][C][D] or null
  const void* bias;     // [D] or null
  const uint8_t* valid; // [B][C] or null
  void* out;            // [B][C][D]
  void* work;           // scratch (generic path: per-row inverse norms)
  int64_t B, C, D;
  int64_t zrs, zbs;     // z_tr row / batch strides (elements)
  int64_t grs, gbs;     // z_tl row / batch strides (elements)
  int32_t causal, normalize, act;
  double eps, norm_eps;
  // Enricher gate (avey_fwd_enriched; gate == nullptr then): z_tl = gact(xg wg^T + bg),
  // formed per row block inside the 16-row fused kernel and never stored.
  const void* xg;       // x [B][C][dm], contiguous
  const void* wg;       // [D][dm]: the enricher weight rows that produce z_tl
  const void* bg;       // [D] or null
  int64_t dm;           // model width, a multiple of 8
  int32_t gact;
};

// Arguments of the backward kernels. Every [B][C][D] operand is contiguous.
struct BwdParams {
  const void* z;        // z_tr
  const void* v;        // [C][C] or null
  const void* gate;     // z_tl or null
  const void* bias;     // [D] or null
  const uint8_t* valid; // [B][C] or null
  const void* dout;     // incoming gradient [B][C][D]
  void* dz;             // dz_tr [B][C][D]
  void* dv;             // [C][C] or null (only with v)
  void* dgate;          // dz_tl or null (only with gate)
  void* dbias;          // [D] or null (only with bias)
  void* work;           // bwd_workspace_floats(...) fp32 values
  int64_t B, C, D;
  int32_t causal, normalize, act;
  double eps, norm_eps;
};

// Largest feature width of the backward kernels (16 accumulator tiles per wave).
constexpr int64_t kBwdMaxFeatures = 1024;

// Arithmetic of the backward: fp64 for normalised (Avey-B) calls; bf16 MFMA for bf16
// with D % 8 == 0 and a 16-byte aligned z_tr; fp32 otherwise.
enum class BwdPath { Fp32, Bf16, Fp64 };
BwdPath bwd_path(int dtype, int64_t D, const void* z, bool normalize);
int64_t bwd_workspace_bytes(int64_t B, int64_t C, int64_t D, bool has_v, bool has_bias, BwdPath path);
hipError_t launch_bwd(const BwdParams& p, int dtype, hipStream_t s);

// Static tile table entry chosen on the host.
struct Plan {
  int kernel;     // 1 fused MFMA, 2 generic
  int bm, bn, bd; // query rows per WG, keys per step, features per wave slice / output tile
  int threads;
  int64_t grid;
  int64_t work_bytes;
  int64_t key_tile_steps;
};

Plan make_plan(const avey_fwd_args& a);

hipError_t launch_generic(const FwdParams& p, int dtype, const Plan& plan, hipStream_t s);
hipError_t launch_fused(const FwdParams& p, int dtype, const Plan& plan, hipStream_t s);
// The 16-row fused kernel with the enricher gate formed in its epilogue (p.wg set).
hipError_t launch_fused_enriched(const FwdParams& p, int dtype, const Plan& plan, hipStream_t s);

}  // namespace avey
