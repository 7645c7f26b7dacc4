// Device helpers shared by the contextualizer kernels (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "avey_hip.h"

namespace avey {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Element-type traits: storage type, fp conversion, accumulator type.
template <typename T> struct Elem;
template <> struct Elem<float> {
  typedef float acc;
  __device__ static float to_acc(float x) { return x; }
  __device__ static float from_acc(float x) { return x; }
};
template <> struct Elem<double> {
  typedef double acc;
  __device__ static double to_acc(double x) { return x; }
  __device__ static double from_acc(double x) { return x; }
};
template <> struct Elem<__bf16> {
  typedef float acc;
  __device__ static float to_acc(__bf16 x) { return (float)x; }
  // Round to nearest even (v_cvt_pk_bf16_f32), the same rounding as torch's .to(bfloat16).
  __device__ static __bf16 from_acc(float x) { return (__bf16)x; }
};
template <> struct Elem<_Float16> {
  typedef float acc;
  __device__ static float to_acc(_Float16 x) { return (float)x; }
  __device__ static _Float16 from_acc(float x) { return (_Float16)x; }
};

// Activations of avey_kernels/ops.py:49-58. GELU is the tanh form.
template <typename A>
__device__ __forceinline__ A activate(A x, int act) {
  switch (act) {
    case AVEY_ACT_RELU: return x > A(0) ? x : A(0);
    case AVEY_ACT_RELU2: { A r = x > A(0) ? x : A(0); return r * r; }
    case AVEY_ACT_SILU: {
      // x * sigmoid(x), with exp evaluated on -|x| so it cannot overflow.
      A e = exp(-fabs(x));
      A s = x >= A(0) ? A(1) / (A(1) + e) : e / (A(1) + e);
      return x * s;
    }
    case AVEY_ACT_GELU: {
      const A k = A(0.7978845608028654);  // sqrt(2 / pi)
      A t = k * (x + A(0.044715) * x * x * x);
      return A(0.5) * x * (A(1) + tanh(t));
    }
    default: return x;
  }
}
template <>
__device__ __forceinline__ float activate<float>(float x, int act) {
  switch (act) {
    case AVEY_ACT_RELU: return x > 0.f ? x : 0.f;
    case AVEY_ACT_RELU2: { float r = x > 0.f ? x : 0.f; return r * r; }
    case AVEY_ACT_SILU: {
      float e = expf(-fabsf(x));
      float s = x >= 0.f ? 1.f / (1.f + e) : e / (1.f + e);
      return x * s;
    }
    case AVEY_ACT_GELU: {
      float t = 0.7978845608028654f * (x + 0.044715f * x * x * x);
      return 0.5f * x * (1.f + tanhf(t));
    }
    default: return x;
  }
}

__host__ __device__ __forceinline__ int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Waves of the fused kernel's (BM query rows, NK 32-feature steps per slice)
// variants. The 16-row ones split roles over 8 waves (4 similarity waves, 4 mixing);
// 32- and 64-row ones split their query blocks over 8 waves where a wave's half of
// the state fits 256 registers (up to 192 features per slice with 32 rows, 128
// with 64), and otherwise run 4 waves of 512 registers.
__host__ __device__ constexpr bool fused_query_split(int bm, int nk) {
  return (bm == 32 && nk <= 6) || (bm == 64 && nk <= 4);
}
__host__ __device__ constexpr int fused_threads(int bm, int nk) {
  return (bm == 16 || fused_query_split(bm, nk)) ? 512 : 256;
}

// Block -> (batch item, query tile) of the fused kernels. Blocks are dispatched
// round-robin over the 8 XCDs (block i to XCD i % 8), each with its own L2.
// * Causal grids go heaviest query tile first over the whole grid, and consecutive
//   blocks walk the batch, so all query tiles of an item share an XCD when B % 8 == 0.
// * Bidirectional grids (every query tile the same work) with B % 8 == 0 place the
//   n_qt tiles of an item 8 blocks apart: they share an XCD and are dispatched
//   together, so the item's key tiles are read from that L2 by all of its query tiles
//   at about the same time, also when the grid takes more than one round.
__device__ __forceinline__ void block_item(int i, int B, int n_qt, bool causal, int& b, int& qt) {
  if (!causal && (B & 7) == 0) {
    const int r = i >> 3, g = r / n_qt, k = r - g * n_qt;
    b = 8 * g + (i & 7);
    qt = n_qt - 1 - k;
  } else {
    b = i % B;
    qt = n_qt - 1 - i / B;
  }
}

// Key tiles a query tile visits. Causal skipping keeps the tile holding the
// diagonal and drops every tile that starts after the block's last query
// (the reference rule, avey_kernels/_triton.py:38-50).
__host__ __device__ __forceinline__ int64_t key_tiles_for(int64_t query_tile, int64_t context, int64_t bm,
                                                          int64_t bn, bool causal_skip) {
  if (context <= bn) return 1;
  if (causal_skip) {
    int64_t end = (query_tile + 1) * bm;
    if (end > context) end = context;
    return cdiv(end, bn);
  }
  return cdiv(context, bn);
}

}  // namespace avey
