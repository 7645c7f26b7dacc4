// Fused forward contextualizer for bf16 / fp16 on gfx950 MFMA.
//
// One workgroup (4 waves, one per SIMD) owns BM query rows of one batch item and
// streams key tiles of BN = 32 rows over them. The feature axis is split four
// ways: wave w owns the slice [w*DS, (w+1)*DS) for every product, so the 16-byte
// row loads of a key tile it issues feed only itself. Per key tile:
//
//   A. Similarity S^T = Z_keys . Q^T over the wave's slice (v_mfma_f32_16x16x32):
//      a partial sum per wave of exact 16-bit x 16-bit products in fp32. The same
//      registers give the keys' partial sums of squares (v_dot2) and are staged
//      in the wave's own LDS rows. Partials go to LDS; the next tile is requested.
//      -- barrier --
//   B. One wave per (query block, key half) unit sums the four partials, scales by
//      1/||q|| and 1/||k|| (the reference's F.normalize, ops.py:68-69), multiplies
//      by V (ops.py:70-71), masks by causality / padding with selects
//      (ops.py:72-77), adds to the signed row sum in fp32 (ops.py:79-80), rounds
//      to the 16-bit type and publishes P. -- barrier --
//   C. Mixing O^T += Z_keys^T . P^T (ops.py:78) on v_mfma_f32_16x16x32, the key
//      rows read back from LDS with ds_read_b64_tr_b16 so that keys run along the
//      MFMA reduction axis.
//
// The epilogue multiplies by 1 / (den + eps), adds bias, applies the activation,
// multiplies by the gate, zeroes padded rows and rounds once (ops.py:79-91).
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

__device__ __forceinline__ u32x4 zero4() { return u32x4{0u, 0u, 0u, 0u}; }

// Eight consecutive 16-bit elements row[col..col+7] of a row that exists;
// elements at or beyond D read as zero. Branch-free: the address is clamped into
// the row and the value selected, so every load of a phase issues back to back.
// VEC: D % 8 == 0 and 16-byte aligned rows, so a chunk is wholly in or out.
template <bool VEC>
__device__ __forceinline__ u32x4 load8(const uint16_t* __restrict__ row, int col, int D) {
  if constexpr (VEC) {
    const bool in = col < D;
    const u32x4 v = *reinterpret_cast<const u32x4*>(row + (in ? col : 0));
    return in ? v : zero4();
  } else {
    uint32_t e[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bool in = col + i < D;
      const uint32_t x = row[in ? col + i : 0];
      e[i] = in ? x : 0u;
    }
    return u32x4{e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16)};
  }
}

template <typename T16> struct Ops;
template <> struct Ops<__bf16> {
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
  __device__ static uint32_t from_f(float x) { return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x); }
};
template <> struct Ops<_Float16> {
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

// Workgroup barrier that orders LDS only: global loads stay in flight across it
// (__syncthreads() would also wait for every outstanding global load).
__device__ __forceinline__ s16x4 lds_read_tr(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p));
}

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int BM, int NK>
struct Smem {
  static constexpr int QB = BM / 16;
  static constexpr int ZLD = 32 * NK + 8;  // row stride in elements; +16 B staggers LDS banks
  uint16_t zs[kWaves][kBN][ZLD];           // each wave's slice of the current key tile
  f32x4 sx[kWaves][2][QB][64];  // per-wave partial S^T tiles (key half, query block)
  u32x4 px[QB][64];             // P as mixing-product B operands (8 x 16-bit per lane)
  f32x4 nx[kBN];                // per-key partial sums of squares, one slot per wave;
                                // negative for padded or out-of-range keys
  float nq[kWaves][BM];         // per-wave partial sums of squares of the queries
  float rq[BM];                 // 1 / max(||q||, norm_eps); 0 for padded or out-of-range rows
  float dx[QB][2][4][16];       // signed row-sum partials
  float dq[BM];                 // full signed row sums
};

}  // namespace

template <typename T16, int BM, int NK, bool VEC>
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
  const uint16_t* __restrict__ zb = (const uint16_t*)p.z + (int64_t)b * C * D;
  // Row-validity bytes; without a mask, bytes of z_tr are read (and ignored).
  const bool has_valid = p.valid != nullptr;
  const uint8_t* __restrict__ vsrc = has_valid ? p.valid + (int64_t)b * C : (const uint8_t*)zb;
  // Absent operands are read from z_tr at index 0 (and ignored), so that no load
  // sits under a branch: a load under control flow makes the compiler wait for
  // every load in flight where the paths merge.
  const bool has_v = p.v != nullptr, has_gate = p.gate != nullptr, has_bias = p.bias != nullptr;
  const uint16_t* __restrict__ vw = has_v ? (const uint16_t*)p.v : zb;
  const uint16_t* __restrict__ gate = has_gate ? (const uint16_t*)p.gate + (int64_t)b * C * D : zb;
  const uint16_t* __restrict__ bias = has_bias ? (const uint16_t*)p.bias : zb;
  const int64_t vmask = has_v ? ~int64_t(0) : int64_t(0);
  const int fw = w * DS;  // first feature of this wave's slice
  const bool causal = p.causal != 0;
  const float norm_eps = (float)p.norm_eps;
  const float eps2 = norm_eps * norm_eps;
  const float inv_eps = 1.f / norm_eps;

  // Reduction units owned by this wave: unit u = w + 4j -> (query block u/2, key half u%2).
  int uq[UPW], uk[UPW];
  bool uon[UPW];
#pragma unroll
  for (int j = 0; j < UPW; ++j) {
    const int u = w + kWaves * j;
    uon[j] = u < UNITS;
    uq[j] = uon[j] ? (u >> 1) : 0;
    uk[j] = u & 1;
  }

  // Key rows of one tile (similarity A operands), their validity bytes and the V
  // entries the units need. Loaded values stay in their storage types until used:
  // widening them right after the load would make the compiler wait there.
  u32x4 zf[2][NK];
  uint8_t zv[2];
  uint16_t vv[UPW][4];
  auto load_tile = [&](int k0) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int k = k0 + 16 * kb + li;
      const int kc = k < C ? k : C - 1;
      zv[kb] = vsrc[kc];
#pragma unroll
      for (int s = 0; s < NK; ++s) zf[kb][s] = load8<VEC>(zb + kc * D, fw + 32 * s + 8 * lg, D);
    }
#pragma unroll
    for (int j = 0; j < UPW; ++j) {
      const int q = q0 + 16 * uq[j] + li;
      const int qc = q < C ? q : C - 1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int k = k0 + 16 * uk[j] + 4 * lg + i;
        const int kc = k < C ? k : C - 1;
        vv[j][i] = vw[((int64_t)qc * C + kc) & vmask];
      }
    }
  };

  // Epilogue operands (gate, bias, row validity); requested as soon as the key
  // loop ends, ahead of the row-sum exchange.
  u32x2 gw[QB][NT];
  uint16_t bw[NT][4];
  uint8_t qv2[QB];
  auto load_epilogue = [&]() {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int q = q0 + 16 * qb + li;
      const int qc = q < C ? q : C - 1;
      qv2[qb] = vsrc[qc];
      const uint16_t* grow = gate + (has_gate ? qc * D : 0);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int f = fw + 16 * t + 4 * lg;
        if constexpr (VEC) {
          gw[qb][t] = *reinterpret_cast<const u32x2*>(grow + (f < D ? f : 0));
        } else {
          uint16_t e[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) e[i] = grow[f + i < D ? f + i : 0];
          gw[qb][t] = u32x2{(uint32_t)e[0] | ((uint32_t)e[1] << 16), (uint32_t)e[2] | ((uint32_t)e[3] << 16)};
        }
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int f = fw + 16 * t + 4 * lg;
#pragma unroll
      for (int i = 0; i < 4; ++i) bw[t][i] = bias[f + i < D ? f + i : 0];
    }
  };

  const int nkt = (int)key_tiles_for(qt, C, BM, kBN, causal);
  load_tile(0);

  // ---- prologue: query rows as similarity B operands, and their norms ------------
  u32x4 qf[QB][NK];
  {
    uint8_t qv[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int q = q0 + 16 * qb + li;
      const int qc = q < C ? q : C - 1;
      qv[qb] = vsrc[qc];
#pragma unroll
      for (int s = 0; s < NK; ++s) qf[qb][s] = load8<VEC>(zb + qc * D, fw + 32 * s + 8 * lg, D);
    }
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int q = q0 + 16 * qb + li;
      const bool ok = q < C && (!has_valid || qv[qb] != 0);
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
  lds_barrier();
  if (tid < BM) {
    float ss = 0.f;
#pragma unroll
    for (int x = 0; x < kWaves; ++x) ss += sm.nq[x][tid];
    // F.normalize divides by max(||q||, norm_eps); 0 marks padded / out-of-range rows.
    sm.rq[tid] = ss < 0.f ? 0.f : (ss > eps2 ? __builtin_amdgcn_rsqf(ss) : inv_eps);
  }

  f32x4 oacc[NT][QB];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) oacc[t][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float den[UPW];
#pragma unroll
  for (int j = 0; j < UPW; ++j) den[j] = 0.f;

  for (int kt = 0; kt < nkt; ++kt) {
    const int k0 = kt * kBN;

    // ---- A: partial similarity over this wave's feature slice; stage the slice ---
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const bool ok = (k0 + 16 * kb + li < C) && (!has_valid || zv[kb] != 0);
      f32x4 sacc[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) sacc[qb] = f32x4{0.f, 0.f, 0.f, 0.f};
      float ss = 0.f;
#pragma unroll
      for (int s = 0; s < NK; ++s) {
        const u32x4 z = ok ? zf[kb][s] : zero4();  // select: NaN-safe
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) sacc[qb] = Ops<T16>::mfma32(z, qf[qb][s], sacc[qb]);
        ss = Ops<T16>::sumsq(z, ss);
        *reinterpret_cast<u32x4*>(&sm.zs[w][16 * kb + li][32 * s + 8 * lg]) = z;
      }
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) sm.sx[w][kb][qb][lane] = sacc[qb];
      ss = sum_over_groups(ss);
      if (lg == 0) reinterpret_cast<float*>(&sm.nx[16 * kb + li])[w] = ok ? ss : -1.f;
    }
    uint16_t vcur[UPW][4];
#pragma unroll
    for (int j = 0; j < UPW; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) vcur[j][i] = vv[j][i];
    if (kt + 1 < nkt) load_tile(k0 + kBN);
    lds_barrier();

    // ---- B: reduce partials, scale, weight, mask, publish P ------------------------
#pragma unroll
    for (int j = 0; j < UPW; ++j) {
      if (uon[j]) {
        const int qb = uq[j], kb = uk[j];
        f32x4 sv = sm.sx[0][kb][qb][lane];
#pragma unroll
        for (int x = 1; x < kWaves; ++x) sv += sm.sx[x][kb][qb][lane];
        const int q = q0 + 16 * qb + li;
        const float rqv = sm.rq[16 * qb + li];  // 0 for padded / out-of-range queries
        float pv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kl = 16 * kb + 4 * lg + i;
          const int k = k0 + kl;
          const f32x4 n4 = sm.nx[kl];
          const float nk = (n4[0] + n4[1]) + (n4[2] + n4[3]);  // negative: padded key
          const float rk = nk > eps2 ? __builtin_amdgcn_rsqf(nk) : inv_eps;
          const bool ok = nk >= 0.f && (!causal || k <= q);
          float v = sv[i] * rqv * rk;
          if (has_v) v *= Ops<T16>::to_f(vcur[j][i]);
          pv[i] = ok ? v : 0.f;
          den[j] += pv[i];
        }
        reinterpret_cast<u32x2*>(&sm.px[qb][lane])[kb] = u32x2{pack2<T16>(pv[0], pv[1]), pack2<T16>(pv[2], pv[3])};
      }
    }
    lds_barrier();

    // ---- C: mixing; the key rows come back from the wave's LDS slice transposed ------
    u32x4 pf[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) pf[qb] = sm.px[qb][lane];
    const int row = 4 * lg + (li >> 2);
    const int colo = 4 * (li & 3);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const u32x2 lo = __builtin_bit_cast(u32x2, lds_read_tr(&sm.zs[w][row][16 * t + colo]));
      const u32x2 hi = __builtin_bit_cast(u32x2, lds_read_tr(&sm.zs[w][16 + row][16 * t + colo]));
      const u32x4 a = u32x4{lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) oacc[t][qb] = Ops<T16>::mfma32(a, pf[qb], oacc[t][qb]);
    }
  }

  // ---- epilogue: lane holds query 16*qb+li, features fw+16t+4*lg .. +3 ------------------
  load_epilogue();
  float rden[QB];
  if (p.normalize) {
#pragma unroll
    for (int j = 0; j < UPW; ++j)
      if (uon[j]) sm.dx[uq[j]][uk[j]][lg][li] = den[j];
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
  uint16_t* __restrict__ out = (uint16_t*)p.out;
  auto finish = [&](auto act_tag) {
    constexpr int ACT = decltype(act_tag)::value;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int q = q0 + 16 * qb + li;
      const bool qok = !has_valid || qv2[qb] != 0;
      const int64_t rowoff = ((int64_t)b * C + (q < C ? q : 0)) * D;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int f = fw + 16 * t + 4 * lg;
        float y[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float x = oacc[t][qb][i] * rden[qb];
          if (has_bias) x += Ops<T16>::to_f(bw[t][i]);
          x = activate<float>(x, ACT);
          if (has_gate) x *= Ops<T16>::to_f((gw[qb][t][i >> 1] >> (16 * (i & 1))) & 0xffffu);
          y[i] = qok ? x : 0.f;
        }
        if (q < C && f < D) {
          if (VEC) {
            *reinterpret_cast<u32x2*>(out + rowoff + f) = u32x2{pack2<T16>(y[0], y[1]), pack2<T16>(y[2], y[3])};
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (f + i < D) out[rowoff + f + i] = (uint16_t)Ops<T16>::from_f(y[i]);
          }
        }
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

// Instantiates and launches fused_fwd_kernel<T16, BM, NK, VEC> for one BM;
// defined in avey_fused_bm{16,32,64}.hip so the variants compile in parallel.
template <int BM>
hipError_t launch_fused_bm(const FwdParams& p, int dtype, int nk, int64_t grid, hipStream_t s);

template <typename T16, int BM, int NK>
hipError_t launch_fused_one(const FwdParams& p, int64_t grid, hipStream_t s) {
  if (p.aligned)
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
