// Fused forward contextualizer for bf16 / fp16 on gfx950 MFMA.
//
// One workgroup (4 waves, one per SIMD) owns BM query rows of one batch item and
// streams key tiles of BN = 32 rows over them. The feature axis is split four
// ways: wave w owns the slice [w*DS, (w+1)*DS) for every product, so the 16-byte
// row chunks it loads feed only itself. Per key tile t there are three stages:
//
//   A(t) similarity S^T = Z_keys . Q^T over the wave's slice (v_mfma_f32_16x16x32):
//        an fp32 partial per wave of exact 16-bit products. The same registers
//        give the keys' partial sums of squares (v_dot2) and are staged in the
//        wave's own LDS rows for the mixing product.
//   B(t) one wave per (16-query block, 16-key half) unit sums the four partials,
//        scales by 1/||q|| and 1/||k|| (F.normalize, ops.py:68-69), multiplies by
//        V (ops.py:70-71), masks by causality / padding with selects (ops.py:72-77),
//        adds to the signed row sum in fp32 (ops.py:79-80), rounds to the 16-bit
//        type and publishes P.
//   C(t) mixing O^T += Z_keys^T . P^T (ops.py:78), the key rows read back from LDS
//        with ds_read_b64_tr_b16 so that keys run along the MFMA reduction axis.
//
// The stages are software-pipelined over two barrier intervals per tile:
//
//   interval 1:  B(t-1) [VALU]  ||  A(t) [MFMA + dot2], next tile's loads issued
//   interval 2:  C(t-1) [MFMA]  +   A(t)'s partials published, key norms of t
//
// so the reduction's VALU work overlaps the similarity MFMAs. A(t) keeps its
// partial S^T in registers until interval 2, which lets one LDS buffer hold the
// partials; the staged key rows are double-buffered (C(t-1) reads one buffer
// while A(t) fills the other).
//
// The epilogue multiplies by 1 / (den + eps), adds bias, applies the activation,
// multiplies by the gate, zeroes padded rows and rounds once (ops.py:79-91).
//
// Global memory is addressed through buffer resources rebuilt per tile in scalar
// registers: every lane's byte offset is loop-invariant, rows past the context
// (or past the resource) read as zero, and stores past it are dropped, so no
// address is clamped and no load sits under a branch.
//
// Key tiles strictly after a query tile's last row are never visited in causal
// mode (the diagonal tile is kept and masked elementwise). Blocks are numbered
// heaviest query tile first, and consecutive blocks walk the batch so that all
// query tiles of one batch item land on the same XCD (its L2 then serves the
// repeated key reads) whenever the batch is a multiple of 8.
//
// Key order along the mixing reduction axis: a 32-key tile is split in halves
// kb = 0, 1; lane group g (lanes 16g..16g+15) holds keys 4g..4g+3 of each half,
// so k-slot j of group g is key 16*(j/4) + 4g + (j%4). This is the similarity
// output layout, and two transposed LDS reads (rows 4g.., 16+4g..) produce it.
//
// Norm reciprocals use v_rsq_f32 (about 1 ulp); the bf16 / fp16 results are
// rounded far more coarsely than that.
#pragma once

#include <type_traits>

#include "avey_common.h"
#include "avey_internal.h"

namespace avey {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 256;
constexpr int kBN = 32;
// Buffer resource word 3 for gfx9 raw (unswizzled, stride 0) buffers: 32-bit data format.
constexpr int kRsrcWord3 = 0x00020000;
// A byte offset no resource covers: loads there read 0, stores there are dropped.
constexpr uint32_t kNowhere = 0x80000000u;

typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Every resource here is wave-uniform; readfirstlane keeps its fields in scalar
// registers even when the compiler evaluated them on the VALU (a resource in
// vector registers would need a waterfall loop around every access).
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  const uint32_t n = __builtin_amdgcn_readfirstlane(bytes);
  return __builtin_amdgcn_make_buffer_rsrc((void*)(((uint64_t)hi << 32) | lo), (short)0, (int)n, kRsrcWord3);
}

// Resource over rows [row0, rows) of a row-major array with `row_bytes` per row;
// empty when row0 >= rows.
__device__ __forceinline__ rsrc_t rows_rsrc(const char* base, int row0, int rows, uint32_t row_bytes) {
  const int n = rows - row0;
  return make_rsrc(base + (int64_t)row0 * row_bytes, n > 0 ? (uint32_t)n * row_bytes : 0u);
}

__device__ __forceinline__ u32x4 ld128(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ u32x2 ld64(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
__device__ __forceinline__ uint32_t ld16(rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t ld8(rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, off, 0, 0);
}
__device__ __forceinline__ void st64(u32x2 v, rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, 0);
}

__device__ __forceinline__ u32x4 zero4() { return u32x4{0u, 0u, 0u, 0u}; }

template <typename T16> struct Ops;
template <> struct Ops<__bf16> {
  // Bits of 1.0 in the type's 16-bit storage, shifted to where to_f expects them.
  static constexpr uint32_t kOne = 0x3f80u;
  __device__ static f32x4 mfma32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   c, 0, 0, 0);
  }
  __device__ static float sumsq(u32x4 x, float acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // Copy the element out first: __builtin_bit_cast of a vector element
      // would read element 0 (seen with ROCm 7.2 clang).
      const uint32_t word = x[i];
      const bf16x2 h = __builtin_bit_cast(bf16x2, word);
      acc = __builtin_amdgcn_fdot2_f32_bf16(h, h, acc, false);
    }
    return acc;
  }
  __device__ static float to_f(uint32_t u) { return __uint_as_float(u << 16); }
  // to_f(u | one): `one` is 0 or kOne, so an all-zero word can stand for 1.0.
  __device__ static float to_f_or(uint32_t u, uint32_t one) { return __uint_as_float((u | one) << 16); }
  __device__ static float hi_f(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  __device__ static uint32_t from_f(float x) { return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x); }
};
template <> struct Ops<_Float16> {
  static constexpr uint32_t kOne = 0x3c00u;
  __device__ static f32x4 mfma32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  }
  __device__ static float sumsq(u32x4 x, float acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t word = x[i];
      const f16x2 h = __builtin_bit_cast(f16x2, word);
      acc = __builtin_amdgcn_fdot2(h, h, acc, false);
    }
    return acc;
  }
  __device__ static float to_f(uint32_t u) { return (float)__builtin_bit_cast(_Float16, (uint16_t)u); }
  __device__ static float to_f_or(uint32_t u, uint32_t one) { return to_f(u | one); }
  __device__ static float hi_f(uint32_t w) { return to_f(w >> 16); }
  __device__ static uint32_t from_f(float x) { return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x); }
};

template <typename T16>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return Ops<T16>::from_f(lo) | (Ops<T16>::from_f(hi) << 16);
}

// Sum of a value over the four 16-lane groups of a wave (lanes l, l^16, l^32, l^48),
// with the gfx950 row-swap instructions (VALU only, no LDS traffic).
__device__ __forceinline__ float sum_over_groups(float x) {
  u32x2 a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  u32x2 c = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(c[0]) + __uint_as_float(c[1]);
}

__device__ __forceinline__ s16x4 lds_read_tr(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p));
}

// Workgroup barrier that orders LDS only: global loads stay in flight across it
// (__syncthreads() would also wait for every outstanding global load).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int BM, int NK>
struct Smem {
  static constexpr int QB = BM / 16;
  static constexpr int ZLD = 32 * NK + 8;  // row stride in elements; +16 B staggers LDS banks
  uint16_t zs[2][kWaves][kBN][ZLD];        // each wave's slice of a key tile, two tiles
  f32x4 sx[kWaves][2][QB][64];  // per-wave partial S^T tiles (key half, query block)
  u32x4 px[QB][64];             // P as mixing-product B operands (8 x 16-bit per lane)
  float nxp[kWaves][kBN];       // per-wave partial sums of squares of the keys; -1: padded key
  float rk[kBN];                // 1 / max(||k||, norm_eps); 0 for padded or out-of-range keys
  float nq[kWaves][BM];         // per-wave partial sums of squares of the queries
  float rq[BM];                 // 1 / max(||q||, norm_eps); 0 for padded or out-of-range rows
  float dx[QB][2][4][16];       // signed row-sum partials
  float dq[BM];                 // full signed row sums
};

}  // namespace

// FULL: D == 4 * 32 * NK, so every 16-byte chunk a wave touches lies inside the
// row. Otherwise chunks at or past D are redirected to kNowhere (D % 8 == 0 makes
// a chunk wholly in or out).
template <typename T16, int BM, int NK, bool FULL>
__global__ __launch_bounds__(kThreads, 1) void fused_fwd_kernel(FwdParams p) {
  typedef Smem<BM, NK> S;
  constexpr int QB = S::QB, DS = 32 * NK, NT = DS / 16;
  constexpr int UNITS = 2 * QB, UPW = (UNITS + kWaves - 1) / kWaves;
  __shared__ S sm;

  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int li = lane & 15, lg = lane >> 4;
  const int C = (int)p.C, D = (int)p.D, B = (int)p.B;
  const int n_qt = (C + BM - 1) / BM;
  const int b = (int)blockIdx.x % B;
  const int qt = n_qt - 1 - (int)blockIdx.x / B;
  const int q0 = qt * BM;
  const uint32_t row_bytes = (uint32_t)D * 2u;
  const char* zb = (const char*)p.z + (int64_t)b * C * row_bytes;
  const bool has_valid = p.valid != nullptr, has_v = p.v != nullptr;
  const bool has_gate = p.gate != nullptr, has_bias = p.bias != nullptr;
  // Absent operands get empty resources (their loads read 0); `or_*` turns those
  // zeros into the neutral value where 0 is not neutral.
  const char* vb = has_valid ? (const char*)p.valid + (int64_t)b * C : (const char*)p.z;
  const int valid_rows = has_valid ? C : 0;
  const uint32_t or_valid = has_valid ? 0u : 1u;
  const uint32_t or_v = has_v ? 0u : Ops<T16>::kOne;
  const int fw = w * DS;  // first feature of this wave's slice
  const bool causal = p.causal != 0;
  const float norm_eps = (float)p.norm_eps;
  const float eps2 = norm_eps * norm_eps;
  const float inv_eps = 1.f / norm_eps;

  // Byte offsets of this lane's 16-byte chunks within a 16-row block: row li,
  // features fw + 32 s + 8 lg .. +7.
  uint32_t coff[NK];
#pragma unroll
  for (int s = 0; s < NK; ++s) {
    const int col = fw + 32 * s + 8 * lg;
    coff[s] = (FULL || col < D) ? (uint32_t)li * row_bytes + (uint32_t)col * 2u : kNowhere;
  }
  auto chunk_off = [&](int s) -> uint32_t {
    if constexpr (FULL) return coff[0] + 64u * (uint32_t)s;  // folds into the instruction offset
    else return coff[s];
  };

  // Reduction units owned by this wave: unit u = w + 4j -> (query block u/2, key half u%2).
  int uq[UPW], uk[UPW], ud[UPW];
  uint32_t voff[UPW];
#pragma unroll
  for (int j = 0; j < UPW; ++j) {
    const int u = (w + kWaves * j) < UNITS ? w + kWaves * j : 0;
    uq[j] = u >> 1;
    uk[j] = u & 1;
    // key - query = ud + i - (q0 - k0) for the lane's keys i = 0..3
    ud[j] = 16 * uk[j] + 4 * lg - 16 * uq[j] - li;
    // V[q][k0 + 16 uk + 4 lg + i] relative to V + k0: row q = q0 + 16 uq + li
    voff[j] = ((uint32_t)(q0 + 16 * uq[j] + li) * (uint32_t)C + (uint32_t)(16 * uk[j] + 4 * lg)) * 2u;
  }
  const uint32_t vbytes = has_v ? (uint32_t)C * (uint32_t)C * 2u : 0u;

  // ---- loads of one key tile (similarity A operands and validity) -----------------
  u32x4 zf[2][NK];
  uint32_t zv[2];
  auto load_keys = [&](int k0) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const rsrc_t rz = rows_rsrc(zb, k0 + 16 * kb, C, row_bytes);
      const rsrc_t rv = rows_rsrc(vb, k0 + 16 * kb, valid_rows, 1u);
      zv[kb] = ld8(rv, (uint32_t)li);
#pragma unroll
      for (int s = 0; s < NK; ++s) zf[kb][s] = ld128(rz, chunk_off(s));
    }
  };
  // V entries of tile k0 for this wave's units (raw 16-bit words).
  uint32_t vv[UPW][4];
  auto load_v = [&](int k0) {
    const uint32_t skip = (uint32_t)k0 * 2u;
    const rsrc_t r = make_rsrc((const char*)(has_v ? p.v : p.z) + skip, vbytes > skip ? vbytes - skip : 0u);
#pragma unroll
    for (int j = 0; j < UPW; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) vv[j][i] = ld16(r, voff[j] + 2u * (uint32_t)i);
  };

  const int nkt = (int)key_tiles_for(qt, C, BM, kBN, causal);
  load_keys(0);

  // ---- prologue: query rows as similarity B operands, and their norms ------------
  u32x4 qf[QB][NK];
  {
    uint32_t qv[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const rsrc_t rz = rows_rsrc(zb, q0 + 16 * qb, C, row_bytes);
      const rsrc_t rv = rows_rsrc(vb, q0 + 16 * qb, valid_rows, 1u);
      qv[qb] = ld8(rv, (uint32_t)li);
#pragma unroll
      for (int s = 0; s < NK; ++s) qf[qb][s] = ld128(rz, chunk_off(s));
    }
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const bool ok = (16 * qb + li < C - q0) && ((qv[qb] | or_valid) != 0u);
      float ss = 0.f;
#pragma unroll
      for (int s = 0; s < NK; ++s) {
        qf[qb][s] = ok ? qf[qb][s] : zero4();  // select, so NaN in padded rows never enters
        ss = Ops<T16>::sumsq(qf[qb][s], ss);
      }
      ss = sum_over_groups(ss);
      if (lg == 0) sm.nq[w][16 * qb + li] = ok ? ss : -1.f;
    }
  }

  f32x4 oacc[NT][QB];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) oacc[t][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float den[UPW];
#pragma unroll
  for (int j = 0; j < UPW; ++j) den[j] = 0.f;
  f32x4 sacc[2][QB];
  float nkey[2];

  // ---- A(t): partial similarity, key partial norms, staging; next loads ---------------
  auto stage_a = [&](int t) {
    const int k0 = t * kBN;
    uint16_t(*zs)[S::ZLD] = sm.zs[t & 1][w];
    bool bad = false;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const bool ok = (16 * kb + li < C - k0) && ((zv[kb] | or_valid) != 0u);
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) sacc[kb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
      float ss = 0.f;
#pragma unroll
      for (int s = 0; s < NK; ++s) {
        // Padded keys may hold NaN: their S^T rows are masked in B and their staged
        // rows are overwritten with zeros below; the norm slot gets a sentinel.
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) sacc[kb][qb] = Ops<T16>::mfma32(zf[kb][s], qf[qb][s], sacc[kb][qb]);
        ss = Ops<T16>::sumsq(zf[kb][s], ss);
        *reinterpret_cast<u32x4*>(&zs[16 * kb + li][32 * s + 8 * lg]) = zf[kb][s];
      }
      ss = sum_over_groups(ss);
      nkey[kb] = ok ? ss : -1.f;
      bad |= !ok;
    }
    if (lg == 0) {
      sm.nxp[w][li] = nkey[0];
      sm.nxp[w][16 + li] = nkey[1];
    }
    // Zero the staged rows of padded / out-of-range keys (tiles at the context's
    // end, or with key padding) so the mixing product never sees NaN.
    if (__builtin_amdgcn_ballot_w64(bad) != 0) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bool ok = (16 * kb + li < C - k0) && ((zv[kb] | or_valid) != 0u);
        if (!ok) {
#pragma unroll
          for (int s = 0; s < NK; ++s) *reinterpret_cast<u32x4*>(&zs[16 * kb + li][32 * s + 8 * lg]) = zero4();
        }
      }
    }
    load_v(k0);
    load_keys(k0 + kBN < nkt * kBN ? k0 + kBN : C);  // past the last tile: empty resources
  };

  // ---- B(t): reduce partials, scale, weight, mask, publish P ---------------------------
  auto stage_b = [&](int t) {
    const int k0 = t * kBN;
    const int lim = causal ? q0 - k0 : (1 << 30);
#pragma unroll
    for (int j = 0; j < UPW; ++j) {
      if (UNITS % kWaves == 0 || w + kWaves * j < UNITS) {
        const int qb = uq[j], kb = uk[j];
        f32x4 sv = sm.sx[0][kb][qb][lane];
#pragma unroll
        for (int x = 1; x < kWaves; ++x) sv += sm.sx[x][kb][qb][lane];
        const f32x4 rk4 = *reinterpret_cast<const f32x4*>(&sm.rk[16 * kb + 4 * lg]);
        const float rqv = sm.rq[16 * qb + li];  // 0 for padded / out-of-range queries
        float pv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float x = sv[i] * (rk4[i] * rqv);
          x *= Ops<T16>::to_f_or(vv[j][i], or_v);
          const bool ok = rk4[i] > 0.f && ud[j] + i <= lim;
          pv[i] = ok ? x : 0.f;
          den[j] += pv[i];
        }
        reinterpret_cast<u32x2*>(&sm.px[qb][lane])[kb] = u32x2{pack2<T16>(pv[0], pv[1]), pack2<T16>(pv[2], pv[3])};
      }
    }
  };

  // ---- C(t): mixing; the key rows come back from the wave's LDS slice transposed ---------
  auto stage_c = [&](int t) {
    uint16_t(*zs)[S::ZLD] = sm.zs[t & 1][w];
    u32x4 pf[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) pf[qb] = sm.px[qb][lane];
    const int row = 4 * lg + (li >> 2);
    const int colo = 4 * (li & 3);
#pragma unroll
    for (int t2 = 0; t2 < NT; ++t2) {
      const u32x2 lo = __builtin_bit_cast(u32x2, lds_read_tr(&zs[row][16 * t2 + colo]));
      const u32x2 hi = __builtin_bit_cast(u32x2, lds_read_tr(&zs[16 + row][16 * t2 + colo]));
      const u32x4 a = u32x4{lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) oacc[t2][qb] = Ops<T16>::mfma32(a, pf[qb], oacc[t2][qb]);
    }
  };

  // ---- interval-2 publication: A(t)'s partial S^T and the tile's key norms ---------------
  auto publish = [&]() {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) sm.sx[w][kb][qb][lane] = sacc[kb][qb];
    if (w == kWaves - 1 && lane < kBN) {
      const float n = (sm.nxp[0][lane] + sm.nxp[1][lane]) + (sm.nxp[2][lane] + sm.nxp[3][lane]);
      sm.rk[lane] = n < 0.f ? 0.f : (n > eps2 ? __builtin_amdgcn_rsqf(n) : inv_eps);
    }
  };

  // t = 0: A only; then the query norms and A(0)'s publication.
  stage_a(0);
  lds_barrier();
  if (tid < BM) {
    float ss = 0.f;
#pragma unroll
    for (int x = 0; x < kWaves; ++x) ss += sm.nq[x][tid];
    // F.normalize divides by max(||q||, norm_eps); 0 marks padded / out-of-range rows.
    sm.rq[tid] = ss < 0.f ? 0.f : (ss > eps2 ? __builtin_amdgcn_rsqf(ss) : inv_eps);
  }
  publish();
  lds_barrier();
  for (int t = 1; t < nkt; ++t) {
    stage_b(t - 1);
    stage_a(t);
    lds_barrier();
    stage_c(t - 1);
    publish();
    lds_barrier();
  }
  stage_b(nkt - 1);
  lds_barrier();
  stage_c(nkt - 1);

  // ---- epilogue: lane holds query 16*qb+li, features fw+16t+4*lg .. +3 ------------------
  // Gate rows, bias and row validity; rows past the context read as zero.
  u32x2 gw[QB][NT];
  u32x2 bw[NT];
  uint32_t qv2[QB];
  const char* gb = has_gate ? (const char*)p.gate + (int64_t)b * C * row_bytes : (const char*)p.z;
  const uint32_t or_gate = has_gate ? 0u : (Ops<T16>::kOne | (Ops<T16>::kOne << 16));
  const rsrc_t rbias = make_rsrc(has_bias ? p.bias : p.z, has_bias ? row_bytes : 0u);
  uint32_t eoff[NT];
#pragma unroll
  for (int t2 = 0; t2 < NT; ++t2) {
    const int f = fw + 16 * t2 + 4 * lg;
    eoff[t2] = (FULL || f < D) ? (uint32_t)f * 2u : kNowhere;
    bw[t2] = ld64(rbias, eoff[t2]);
  }
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const rsrc_t rg = rows_rsrc(gb, q0 + 16 * qb, has_gate ? C : 0, row_bytes);
    const rsrc_t rv = rows_rsrc(vb, q0 + 16 * qb, valid_rows, 1u);
    qv2[qb] = ld8(rv, (uint32_t)li);
#pragma unroll
    for (int t2 = 0; t2 < NT; ++t2) {
      gw[qb][t2] = ld64(rg, (uint32_t)li * row_bytes + eoff[t2]);
      gw[qb][t2] = u32x2{gw[qb][t2][0] | or_gate, gw[qb][t2][1] | or_gate};
    }
  }
  float rden[QB];
  if (p.normalize) {
#pragma unroll
    for (int j = 0; j < UPW; ++j)
      if (UNITS % kWaves == 0 || w + kWaves * j < UNITS) sm.dx[uq[j]][uk[j]][lg][li] = den[j];
    lds_barrier();
    if (tid < BM) {
      float d = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int g = 0; g < 4; ++g) d += sm.dx[tid >> 4][kb][g][tid & 15];
      sm.dq[tid] = 1.f / (d + (float)p.eps);  // the signed sum, eps added, no clamp
    }
    lds_barrier();
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) rden[qb] = sm.dq[16 * qb + li];
  } else {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) rden[qb] = 1.f;
  }
  const rsrc_t rout_all = make_rsrc((char*)p.out + (int64_t)b * C * row_bytes, (uint32_t)C * row_bytes);
  auto finish = [&](auto act_tag) {
    constexpr int ACT = decltype(act_tag)::value;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int qrow = q0 + 16 * qb + li;
      const bool qok = (qv2[qb] | or_valid) != 0u;
#pragma unroll
      for (int t2 = 0; t2 < NT; ++t2) {
        float y[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t bword = bw[t2][i >> 1], gword = gw[qb][t2][i >> 1];
          float x = oacc[t2][qb][i] * rden[qb];
          x += (i & 1) ? Ops<T16>::hi_f(bword) : Ops<T16>::to_f(bword & 0xffffu);
          x = activate<float>(x, ACT);
          x *= (i & 1) ? Ops<T16>::hi_f(gword) : Ops<T16>::to_f(gword & 0xffffu);
          y[i] = qok ? x : 0.f;
        }
        // Rows past the context fall outside rout_all and are dropped.
        const uint32_t off = eoff[t2] == kNowhere ? kNowhere : (uint32_t)qrow * row_bytes + eoff[t2];
        st64(u32x2{pack2<T16>(y[0], y[1]), pack2<T16>(y[2], y[3])}, rout_all, off);
      }
    }
  };
  switch (p.act) {
    case AVEY_ACT_RELU: finish(std::integral_constant<int, AVEY_ACT_RELU>{}); break;
    case AVEY_ACT_RELU2: finish(std::integral_constant<int, AVEY_ACT_RELU2>{}); break;
    case AVEY_ACT_SILU: finish(std::integral_constant<int, AVEY_ACT_SILU>{}); break;
    case AVEY_ACT_GELU: finish(std::integral_constant<int, AVEY_ACT_GELU>{}); break;
    default: finish(std::integral_constant<int, AVEY_ACT_IDENTITY>{}); break;
  }
}

// Instantiates and launches fused_fwd_kernel<T16, BM, NK, FULL> for one BM and
// type; defined in avey_fused_bm{16,32,64}_{bf16,f16}.hip so the variants compile
// in parallel.
template <typename T16, int BM>
hipError_t launch_fused_bm(const FwdParams& p, int nk, int64_t grid, hipStream_t s);

template <typename T16, int BM, int NK>
hipError_t launch_fused_one(const FwdParams& p, int64_t grid, hipStream_t s) {
  if (p.D == 4 * 32 * NK)
    fused_fwd_kernel<T16, BM, NK, true><<<dim3((unsigned)grid), dim3(kThreads), 0, s>>>(p);
  else
    fused_fwd_kernel<T16, BM, NK, false><<<dim3((unsigned)grid), dim3(kThreads), 0, s>>>(p);
  return hipGetLastError();
}

template <typename T16, int BM>
hipError_t launch_fused_nk(const FwdParams& p, int nk, int64_t grid, hipStream_t s) {
  switch (nk) {
    case 1: return launch_fused_one<T16, BM, 1>(p, grid, s);
    case 2: return launch_fused_one<T16, BM, 2>(p, grid, s);
    case 3: return launch_fused_one<T16, BM, 3>(p, grid, s);
    case 4: return launch_fused_one<T16, BM, 4>(p, grid, s);
    case 6: return launch_fused_one<T16, BM, 6>(p, grid, s);
    case 8:
      if constexpr (BM <= 32) return launch_fused_one<T16, BM, 8>(p, grid, s);
      return hipErrorInvalidConfiguration;
    default: return hipErrorInvalidConfiguration;
  }
}

}  // namespace avey
