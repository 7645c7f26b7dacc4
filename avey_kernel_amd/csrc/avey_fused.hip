// Fused forward contextualizer for bf16 / fp16 on gfx950 MFMA.
//
// One workgroup (4 waves) owns BM query rows of one batch item and streams key
// tiles of BN = 32 rows over them. The feature axis is split four ways: wave w
// owns the slice [w*DS, (w+1)*DS) for both products, so its 16-byte row loads of
// a key tile feed both products without any other wave touching them.
//
//   1. Similarity, S^T = Z_keys . Q^T, on v_mfma_f32_16x16x32 over the wave's
//      slice -> a partial sum per wave, exact bf16 x bf16 products in fp32. The
//      wave also stages its slice of the key rows in its own LDS region and
//      accumulates the keys' partial sums of squares (v_dot2).
//   2. Barrier; the four partials are summed per (query block, key half) unit by
//      one wave each, scaled by 1/||q|| and 1/||k|| in fp32 (the reference's
//      F.normalize, ops.py:68-69), multiplied by V (ops.py:70-71), masked by
//      causality / padding with selects (ops.py:72-77), added to the signed row
//      sum (ops.py:79-80) before any rounding, rounded to the 16-bit type and
//      published to LDS as GEMM2 operands.
//   3. Barrier; mixing, O^T += Z_keys^T . P^T (ops.py:78), with the key rows
//      re-read from the wave's LDS slice by ds_read_b64_tr_b16 so that keys run
//      along the MFMA reduction axis.
//   4. Epilogue in registers: / (den + eps), + bias, activation, * gate, row
//      mask, one rounding to the output type (ops.py:79-91).
//
// Key tiles strictly after a query tile's last row are never visited in causal
// mode (the diagonal tile is kept and masked elementwise). Blocks are numbered
// heaviest query tile first, and consecutive blocks walk the batch so that all
// query tiles of one batch item land on the same XCD (its L2 then serves the
// repeated key reads) whenever the batch is a multiple of 8.
#include "avey_common.h"
#include "avey_internal.h"

namespace avey {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 256;
constexpr int kBN = 32;

__device__ __forceinline__ u32x4 zero4() { return u32x4{0u, 0u, 0u, 0u}; }

// Eight consecutive 16-bit elements row[col..col+7]; elements at or beyond D read as zero.
__device__ __forceinline__ u32x4 load8(const uint16_t* __restrict__ row, int64_t col, int64_t D, bool aligned) {
  if (col >= D) return zero4();
  if (aligned && col + 8 <= D) return *reinterpret_cast<const u32x4*>(row + col);
  uint16_t e[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) e[i] = (col + i < D) ? row[col + i] : (uint16_t)0;
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = (uint32_t)e[2 * i] | ((uint32_t)e[2 * i + 1] << 16);
  return r;
}

template <typename T16> struct Ops;
template <> struct Ops<__bf16> {
  __device__ static f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   c, 0, 0, 0);
  }
  __device__ static float sumsq(u32x4 x, float acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t word = x[i];  // bit_cast of a vector element would read element 0
      const bf16x2 h = __builtin_bit_cast(bf16x2, word);
      acc = __builtin_amdgcn_fdot2_f32_bf16(h, h, acc, false);
    }
    return acc;
  }
  __device__ static float to_f(uint16_t u) { return __uint_as_float((uint32_t)u << 16); }
  __device__ static uint16_t from_f(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }
};
template <> struct Ops<_Float16> {
  __device__ static f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
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
  __device__ static float to_f(uint16_t u) { return (float)__builtin_bit_cast(_Float16, u); }
  __device__ static uint16_t from_f(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }
};

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

template <int BM, int NK>
struct Smem {
  static constexpr int QB = BM / 16;
  static constexpr int DS = 32 * NK;
  static constexpr int ZLD = DS + 8;  // row stride in elements; +16 B staggers LDS banks
  uint16_t zs[kWaves][kBN][ZLD];      // each wave's slice of the current key tile
  f32x4 sx[kWaves][2][QB][64];        // per-wave partial S^T tiles
  u32x4 px[QB][64];                   // P as GEMM2 B operands (8 x 16-bit per lane)
  float nx[kWaves][kBN];              // per-wave partial sums of squares of the keys
  float nq[kWaves][BM];               // per-wave partial sums of squares of the queries
  float rq[BM];                       // 1 / max(||q||, norm_eps)
  float dx[QB][2][4][16];             // signed row-sum partials
  float dq[BM];                       // full signed row sums
};

}  // namespace

template <typename T16, int BM, int NK>
__global__ __launch_bounds__(kThreads, 1) void fused_fwd_kernel(FwdParams p) {
  typedef Smem<BM, NK> S;
  constexpr int QB = S::QB, DS = S::DS, NT = DS / 16;
  constexpr int UNITS = 2 * QB, UPW = (UNITS + kWaves - 1) / kWaves;
  __shared__ S sm;

  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int li = lane & 15, lg = lane >> 4;
  const int64_t C = p.C, D = p.D;
  const int64_t n_qt = cdiv(C, BM);
  const int64_t b = blockIdx.x % p.B;
  const int64_t qt = n_qt - 1 - (int64_t)blockIdx.x / p.B;
  const int64_t q0 = qt * BM;
  const uint16_t* zb = (const uint16_t*)p.z + b * C * D;
  const uint8_t* vb = p.valid ? p.valid + b * C : nullptr;
  const uint16_t* vw = (const uint16_t*)p.v;
  const int64_t fw = (int64_t)w * DS;  // first feature of this wave's slice
  const bool aligned = p.aligned != 0;
  const float norm_eps = (float)p.norm_eps;

  // ---- prologue: query rows as GEMM1 B operands, and their norms -------------
  u32x4 qf[QB][NK];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int64_t q = q0 + 16 * qb + li;
    const bool ok = q < C && (!vb || vb[q]);
    float ss = 0.f;
#pragma unroll
    for (int s = 0; s < NK; ++s) {
      qf[qb][s] = ok ? load8(zb + q * D, fw + 32 * s + 8 * lg, D, aligned) : zero4();
      ss = Ops<T16>::sumsq(qf[qb][s], ss);
    }
    ss = sum_over_groups(ss);
    if (lg == 0) sm.nq[w][16 * qb + li] = ss;
  }
  __syncthreads();
  if (tid < BM) {
    float ss = 0.f;
#pragma unroll
    for (int x = 0; x < kWaves; ++x) ss += sm.nq[x][tid];
    sm.rq[tid] = 1.f / fmaxf(sqrtf(ss), norm_eps);
  }

  f32x4 oacc[NT][QB];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) oacc[t][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float den[UPW];
#pragma unroll
  for (int j = 0; j < UPW; ++j) den[j] = 0.f;

  const int64_t nkt = key_tiles_for(qt, C, BM, kBN, p.causal != 0);
  for (int64_t kt = 0; kt < nkt; ++kt) {
    const int64_t k0 = kt * kBN;

    // ---- phase 1: partial similarity over this wave's feature slice ----------
    u32x4 zf[2][NK];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int64_t k = k0 + 16 * kb + li;
      const bool ok = k < C && (!vb || vb[k]);
#pragma unroll
      for (int s = 0; s < NK; ++s) zf[kb][s] = ok ? load8(zb + k * D, fw + 32 * s + 8 * lg, D, aligned) : zero4();
    }
    f32x4 sacc[2][QB];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      float ss = 0.f;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) sacc[kb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < NK; ++s) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) sacc[kb][qb] = Ops<T16>::mfma(zf[kb][s], qf[qb][s], sacc[kb][qb]);
        ss = Ops<T16>::sumsq(zf[kb][s], ss);
        *reinterpret_cast<u32x4*>(&sm.zs[w][16 * kb + li][32 * s + 8 * lg]) = zf[kb][s];
      }
      ss = sum_over_groups(ss);
      if (lg == 0) sm.nx[w][16 * kb + li] = ss;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) sm.sx[w][kb][qb][lane] = sacc[kb][qb];
    }
    __syncthreads();

    // ---- phase 2: reduce partials, scale, weight, mask, publish P -------------
#pragma unroll
    for (int j = 0; j < UPW; ++j) {
      const int u = w + kWaves * j;
      if (u < UNITS) {
        const int qb = u >> 1, kb = u & 1;
        f32x4 sv = sm.sx[0][kb][qb][lane];
#pragma unroll
        for (int x = 1; x < kWaves; ++x) sv += sm.sx[x][kb][qb][lane];
        const int64_t q = q0 + 16 * qb + li;
        const bool qok = q < C && (!vb || vb[q]);
        const float rqv = sm.rq[16 * qb + li];
        uint16_t pb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kl = 16 * kb + 4 * lg + i;
          const int64_t k = k0 + kl;
          float nk = sm.nx[0][kl];
#pragma unroll
          for (int x = 1; x < kWaves; ++x) nk += sm.nx[x][kl];
          const float rk = 1.f / fmaxf(sqrtf(nk), norm_eps);
          const bool ok = qok && k < C && (!vb || vb[k]) && (!p.causal || k <= q);
          float pv = 0.f;
          if (ok) {
            pv = sv[i] * rqv * rk;
            if (vw) pv *= Ops<T16>::to_f(vw[q * C + k]);
          }
          den[j] += pv;
          pb[i] = Ops<T16>::from_f(pv);
        }
        u32x2 packed;
        packed[0] = (uint32_t)pb[0] | ((uint32_t)pb[1] << 16);
        packed[1] = (uint32_t)pb[2] | ((uint32_t)pb[3] << 16);
        reinterpret_cast<u32x2*>(&sm.px[qb][lane])[kb] = packed;
      }
    }
    __syncthreads();

    // ---- phase 3: mixing, keys along the MFMA reduction axis -----------------
    u32x4 pf[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) pf[qb] = sm.px[qb][lane];
    const int row = 4 * lg + (li >> 2);
    const int colo = 4 * (li & 3);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      s16x4 lo = lds_read_tr(&sm.zs[w][row][16 * t + colo]);
      s16x4 hi = lds_read_tr(&sm.zs[w][16 + row][16 * t + colo]);
      const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
      const u32x4 a = u32x4{l2[0], l2[1], h2[0], h2[1]};
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) oacc[t][qb] = Ops<T16>::mfma(a, pf[qb], oacc[t][qb]);
    }
  }

  // ---- signed row sums -----------------------------------------------------------
  if (p.normalize) {
#pragma unroll
    for (int j = 0; j < UPW; ++j) {
      const int u = w + kWaves * j;
      if (u < UNITS) sm.dx[u >> 1][u & 1][lg][li] = den[j];
    }
    __syncthreads();
    if (tid < BM) {
      float d = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int g = 0; g < 4; ++g) d += sm.dx[tid >> 4][kb][g][tid & 15];
      sm.dq[tid] = d;
    }
    __syncthreads();
  }

  // ---- epilogue: lane holds query 16*qb+li, features fw+16*t+4*lg .. +3 -------------
  const uint16_t* bias = (const uint16_t*)p.bias;
  const uint16_t* gate = (const uint16_t*)p.gate;
  uint16_t* out = (uint16_t*)p.out;
  const float eps = (float)p.eps;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int64_t q = q0 + 16 * qb + li;
    if (q >= C) continue;
    const bool qok = !vb || vb[q];
    const float dd = p.normalize ? sm.dq[16 * qb + li] + eps : 1.f;
    const int64_t rowoff = (b * C + q) * D;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int64_t f = fw + 16 * t + 4 * lg;
      if (f >= D) continue;
      const bool vec = aligned && f + 4 <= D;
      float gv[4] = {1.f, 1.f, 1.f, 1.f};
      if (gate) {
        if (vec) {
          u32x2 g2 = *reinterpret_cast<const u32x2*>(gate + rowoff + f);
          gv[0] = Ops<T16>::to_f((uint16_t)(g2[0] & 0xffff));
          gv[1] = Ops<T16>::to_f((uint16_t)(g2[0] >> 16));
          gv[2] = Ops<T16>::to_f((uint16_t)(g2[1] & 0xffff));
          gv[3] = Ops<T16>::to_f((uint16_t)(g2[1] >> 16));
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) gv[i] = (f + i < D) ? Ops<T16>::to_f(gate[rowoff + f + i]) : 0.f;
        }
      }
      uint16_t ov[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float y = oacc[t][qb][i];
        if (p.normalize) y = y / dd;
        if (bias && f + i < D) y += Ops<T16>::to_f(bias[f + i]);
        y = activate<float>(y, p.act);
        if (gate) y *= gv[i];
        ov[i] = Ops<T16>::from_f(qok ? y : 0.f);
      }
      if (vec) {
        u32x2 o2;
        o2[0] = (uint32_t)ov[0] | ((uint32_t)ov[1] << 16);
        o2[1] = (uint32_t)ov[2] | ((uint32_t)ov[3] << 16);
        *reinterpret_cast<u32x2*>(out + rowoff + f) = o2;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (f + i < D) out[rowoff + f + i] = ov[i];
      }
    }
  }
}

namespace {

template <typename T16, int BM, int NK>
hipError_t launch_one(const FwdParams& p, int64_t grid, hipStream_t s) {
  fused_fwd_kernel<T16, BM, NK><<<dim3((unsigned)grid), dim3(kThreads), 0, s>>>(p);
  return hipGetLastError();
}

template <typename T16, int BM>
hipError_t launch_bm(const FwdParams& p, int nk, int64_t grid, hipStream_t s) {
  switch (nk) {
    case 1: return launch_one<T16, BM, 1>(p, grid, s);
    case 2: return launch_one<T16, BM, 2>(p, grid, s);
    case 3: return launch_one<T16, BM, 3>(p, grid, s);
    case 4: return launch_one<T16, BM, 4>(p, grid, s);
    case 6: return launch_one<T16, BM, 6>(p, grid, s);
    case 8:
      if constexpr (BM <= 32) return launch_one<T16, BM, 8>(p, grid, s);
      return hipErrorInvalidConfiguration;
    default: return hipErrorInvalidConfiguration;
  }
}

template <typename T16>
hipError_t launch_t(const FwdParams& p, const Plan& plan, hipStream_t s) {
  const int nk = plan.bd / 32;
  switch (plan.bm) {
    case 16: return launch_bm<T16, 16>(p, nk, plan.grid, s);
    case 32: return launch_bm<T16, 32>(p, nk, plan.grid, s);
    case 64: return launch_bm<T16, 64>(p, nk, plan.grid, s);
    default: return hipErrorInvalidConfiguration;
  }
}

}  // namespace

hipError_t launch_fused(const FwdParams& p, int dtype, const Plan& plan, hipStream_t s) {
  if (dtype == AVEY_DTYPE_BF16) return launch_t<__bf16>(p, plan, s);
  if (dtype == AVEY_DTYPE_F16) return launch_t<_Float16>(p, plan, s);
  return hipErrorInvalidValue;
}

}  // namespace avey
