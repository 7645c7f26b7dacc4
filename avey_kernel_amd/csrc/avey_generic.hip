// Generic contextualizer kernels (VALU, any element type).
//
// Used for fp32 and fp64 inputs and for feature widths beyond the fused MFMA
// kernel's register budget. Arithmetic follows the reference's eager path
// (avey_kernels/ops.py:61-91) in the accumulation type of Elem<T> (fp32, or fp64
// for fp64 inputs): inverse row norms first, then per output tile the
// similarity of every allowed (query, key) pair, the learned weight, masks, the
// signed row sum and the mixing sum, then the fused epilogue.
#include "avey_common.h"
#include "avey_internal.h"

namespace avey {

// inv[b*C + j] = 1 / max(||z_j||_2, norm_eps); padded rows count as zero rows
// (ops.py:64-68). One wave per row; rows `zrs` and batch items `zbs` elements apart.
template <typename T>
__global__ __launch_bounds__(256) void row_inv_norm_kernel(const T* __restrict__ z, const uint8_t* __restrict__ valid,
                                                           typename Elem<T>::acc* __restrict__ inv, int64_t rows,
                                                           int64_t C, int64_t D, int64_t zrs, int64_t zbs,
                                                           double norm_eps) {
  typedef typename Elem<T>::acc A;
  const int64_t row = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  if (row >= rows) return;
  A ss = 0;
  if (!valid || valid[row]) {
    const T* zr = z + (row / C) * zbs + (row % C) * zrs;
    for (int64_t f = lane; f < D; f += 64) {
      A x = Elem<T>::to_acc(zr[f]);
      ss += x * x;
    }
  }
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  if (lane == 0) {
    A n = sqrt(ss);
    A e = (A)norm_eps;
    inv[row] = A(1) / (n > e ? n : e);
  }
}

// One workgroup per (batch, 16-query tile, 64-feature output tile), numbered on a
// 1-D grid. Key tiles of 16 rows; the similarity tile is recomputed for every
// output tile.
template <typename T>
__global__ __launch_bounds__(256) void generic_fwd_kernel(FwdParams p) {
  typedef typename Elem<T>::acc A;
  constexpr int BQ = 16, BK = 16, BF = 64, DC = 64;
  __shared__ A qs[BQ][DC + 1];
  __shared__ A ks[BK][DC + 1];
  __shared__ A ss[BQ][BK + 1];
  __shared__ A kf[BK][BF + 1];
  __shared__ A den_s[BQ];
  __shared__ A rq[BQ];

  const int t = threadIdx.x;
  const int64_t C = p.C, D = p.D;
  const int64_t nft = cdiv(D, BF), nqt = cdiv(C, BQ);
  const int64_t ft = (int64_t)blockIdx.x % nft;
  const int64_t qt = ((int64_t)blockIdx.x / nft) % nqt;
  const int64_t b = (int64_t)blockIdx.x / nft / nqt;
  const int64_t q0 = qt * BQ, f0 = ft * BF;
  const T* zb = (const T*)p.z + b * p.zbs;  // row r at zb + r * p.zrs
  const uint8_t* vb = p.valid ? p.valid + b * C : nullptr;
  const A* inv = (const A*)p.work + b * C;
  const T* vw = (const T*)p.v;

  const int si = t / BK, sj = t % BK;       // similarity element owned
  const int oi = t / 16, of = (t % 16) * 4;  // output row / first feature owned
  A acc[4] = {A(0), A(0), A(0), A(0)};
  if (t < BQ) {
    den_s[t] = A(0);
    const int64_t q = q0 + t;
    rq[t] = q < C ? inv[q] : A(0);
  }
  // Guarded loads are written without branches: the load always goes out (to element 0
  // when the guard is false) and the value is selected, so a group of loads shares one
  // wait instead of each sitting in a branch that waits for it.
  auto row_ok = [&](int64_t r) {
    const bool in = r < C;
    return vb ? (in & (vb[in ? r : 0] != 0)) : in;
  };
  auto ldz = [&](bool ok, int64_t idx) -> A {
    const A x = Elem<T>::to_acc(zb[ok ? idx : 0]);
    return ok ? x : A(0);
  };
  const bool hv = vw != nullptr;
  const T* vwp = hv ? vw : zb;  // stand-in when V is absent
  const bool small = D <= DC;  // one feature chunk (C1's shape)

  const int64_t nkt = key_tiles_for(qt, C, BQ, BK, p.causal != 0);
  if (small) {
    // The query rows are loaded once, a key tile's rows serve both the similarities
    // and the mixing (BF == DC), and the next tile's rows, this thread's V entry and
    // key inverse norm are loaded while the current tile is used, so a tile waits on
    // no global-load round trip. Same arithmetic in the same order as below.
    static_assert(BF == DC && BK * DC % 256 == 0, "key rows serve the mixing");
#pragma unroll
    for (int i = 0; i < BQ * DC / 256; ++i) {
      const int e = t + 256 * i, r = e / DC, c = e % DC;
      const int64_t q = q0 + r;
      qs[r][c] = ldz(c < D && row_ok(q), q * p.zrs + c);
    }
    constexpr int KE = BK * DC / 256;  // key-row elements per thread
    A kr[KE];
    auto load_keys = [&](int64_t k0) {
#pragma unroll
      for (int i = 0; i < KE; ++i) {
        const int e = t + 256 * i, r = e / DC, c = e % DC;
        const int64_t k = k0 + r;
        kr[i] = ldz(c < D && row_ok(k), k * p.zrs + c);
      }
    };
    load_keys(0);
    for (int64_t kt = 0; kt < nkt; ++kt) {
      const int64_t k0 = kt * BK;
      const int64_t q = q0 + si, k = k0 + sj;
      const bool allowed = row_ok(q) && row_ok(k) && (!p.causal || k <= q);
      const A ikl = inv[allowed ? k : 0], ik = allowed ? ikl : A(0);
      const A vl = Elem<T>::to_acc(vwp[allowed && hv ? q * C + k : 0]), vv = hv ? vl : A(1);
      __syncthreads();  // the previous tile's reads of ks and ss are done
#pragma unroll
      for (int i = 0; i < KE; ++i) ks[(t + 256 * i) / DC][(t + 256 * i) % DC] = kr[i];
      if (kt + 1 < nkt) load_keys(k0 + BK);
      __syncthreads();
      A s = A(0);
#pragma unroll 8
      for (int c = 0; c < DC; ++c) s += qs[si][c] * ks[sj][c];
      s = allowed ? (hv ? s * rq[si] * ik * vv : s * rq[si] * ik) : A(0);
      ss[si][sj] = s;
      __syncthreads();
      if (p.normalize && t < BQ) {
        A d = A(0);
        for (int j = 0; j < BK; ++j) d += ss[t][j];
        den_s[t] += d;
      }
#pragma unroll 4
      for (int j = 0; j < BK; ++j) {
        const A sv = ss[oi][j];
        for (int u = 0; u < 4; ++u) acc[u] += sv * ks[j][of + u];
      }
    }
  }
  for (int64_t kt = 0; kt < (small ? 0 : nkt); ++kt) {
    const int64_t k0 = kt * BK;
    A s = A(0);
    for (int64_t d0 = 0; d0 < D; d0 += DC) {
      __syncthreads();
#pragma unroll
      for (int i = 0; i < BQ * DC / 256; ++i) {
        const int e = t + 256 * i, r = e / DC, c = e % DC;
        const int64_t f = d0 + c;
        const int64_t q = q0 + r, k = k0 + r;
        qs[r][c] = ldz(f < D && row_ok(q), q * p.zrs + f);
        ks[r][c] = ldz(f < D && row_ok(k), k * p.zrs + f);
      }
      __syncthreads();
#pragma unroll 8
      for (int c = 0; c < DC; ++c) s += qs[si][c] * ks[sj][c];
    }
    {
      const int64_t q = q0 + si, k = k0 + sj;
      const bool allowed = row_ok(q) && row_ok(k) && (!p.causal || k <= q);
      const A ik = inv[allowed ? k : 0];
      const A vv = Elem<T>::to_acc(vwp[allowed && hv ? q * C + k : 0]);
      s = allowed ? (hv ? s * rq[si] * ik * vv : s * rq[si] * ik) : A(0);
      ss[si][sj] = s;
    }
#pragma unroll
    for (int i = 0; i < BK * BF / 256; ++i) {
      const int e = t + 256 * i, r = e / BF, c = e % BF;
      const int64_t k = k0 + r, f = f0 + c;
      kf[r][c] = ldz(f < D && row_ok(k), k * p.zrs + f);
    }
    __syncthreads();
    if (p.normalize && t < BQ) {
      A d = A(0);
      for (int j = 0; j < BK; ++j) d += ss[t][j];
      den_s[t] += d;
    }
#pragma unroll 4
    for (int j = 0; j < BK; ++j) {
      const A sv = ss[oi][j];
      for (int u = 0; u < 4; ++u) acc[u] += sv * kf[j][of + u];
    }
  }
  __syncthreads();

  const int64_t q = q0 + oi;
  if (q >= C) return;
  const bool qv = row_ok(q);
  const T* bias = (const T*)p.bias;
  const T* gate = (const T*)p.gate;
  T* out = (T*)p.out + (b * C + q) * D;
  const A dd = p.normalize ? den_s[oi] + (A)p.eps : A(1);
  // Bias and gate words first: the output stores may alias them as far as the compiler
  // can tell, so loads after a store would wait for it.
  const T* biasp = bias ? bias : zb;
  const T* gatep = gate ? gate + b * p.gbs + q * p.grs : zb;
  A bv[4], gv[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t f = f0 + of + u;
    const bool fin = f < D;
    const A bl = Elem<T>::to_acc(biasp[fin && bias ? f : 0]);
    const A gl = Elem<T>::to_acc(gatep[fin && gate ? f : 0]);
    bv[u] = bias ? bl : A(0);
    gv[u] = gate ? (qv ? gl : A(0)) : A(1);
  }
  for (int u = 0; u < 4; ++u) {
    const int64_t f = f0 + of + u;
    if (f >= D) break;
    A y = acc[u];
    if (p.normalize) y = y / dd;
    if (bias) y += bv[u];
    y = activate<A>(y, p.act);
    if (gate) y *= gv[u];
    out[f] = Elem<T>::from_acc(qv ? y : A(0));
  }
}

template <typename T>
static hipError_t launch_generic_t(const FwdParams& p, hipStream_t s) {
  const int64_t rows = p.B * p.C;
  row_inv_norm_kernel<T><<<dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, s>>>(
      (const T*)p.z, p.valid, (typename Elem<T>::acc*)p.work, rows, p.C, p.D, p.zrs, p.zbs, p.norm_eps);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t grid = cdiv(p.C, 16) * cdiv(p.D, 64) * p.B;
  generic_fwd_kernel<T><<<dim3((unsigned)grid), dim3(256), 0, s>>>(p);
  return hipGetLastError();
}

hipError_t launch_generic(const FwdParams& p, int dtype, const Plan&, hipStream_t s) {
  switch (dtype) {
    case AVEY_DTYPE_F32: return launch_generic_t<float>(p, s);
    case AVEY_DTYPE_F64: return launch_generic_t<double>(p, s);
    case AVEY_DTYPE_BF16: return launch_generic_t<__bf16>(p, s);
    case AVEY_DTYPE_F16: return launch_generic_t<_Float16>(p, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace avey
