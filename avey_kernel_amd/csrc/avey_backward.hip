// Backward of the contextualizer on gfx950: gradients w.r.t. z_tr, v, z_tl and
// bias, computed without storing any C x C tile in HBM.
//
// The reference has no written backward: gradients are autograd over its eager
// path (avey_kernels/ops.py:96-106, :61-91), which materialises [B, C, C]. Here,
// per batch item, with P = S * V * M (S the cosine similarity, M the causal /
// key-padding mask), y = num / den (normalize) or num, u = y + bias, r the
// valid-row mask and g the incoming gradient:
//   dz_tl = g * act(u) * r,  du = g * gate * act'(u) * r,  dbias = sum du,
//   dnum = du / den, dden_i = -sum_d du_id y_id / den_i   (normalize; else du, 0),
//   dP_ij = dnum_i . z_j + dden_i,  dS = dP * V * M,  dv = sum_b dP * S * M,
//   dz = r * (P^T dnum + J(dS zhat + dS^T zhat)),
//   J(x) = (x - zhat (zhat . x)) / ||z||  (||z|| >= norm_eps), else x / norm_eps.
//
// Kernels (arithmetic type A: fp32 with v_mfma_f32_16x16x4f32, or fp64 with
// v_mfma_f64_16x16x4f64 for the normalised (Avey-B) calls, whose gradients divide by
// signed row sums that may cancel; a bf16 MFMA variant follows further down):
//   bwd_prep   row norms ||z|| of the masked rows; clears the dv / dbias accumulators.
//   bwd_rows   one workgroup per (batch item, 16 query rows). Pass 1 over key
//              tiles recomputes S, P, num and den (the forward); the epilogue
//              writes dz_tl, dnum, dden and adds dbias. Pass 2 recomputes S, forms
//              dP = dnum z^T + dden and dS, adds dP * S into dv and accumulates the
//              query-side dS zhat, written to the workspace.
//   bwd_cols   one workgroup per (batch item, 16 key rows), over query tiles:
//              P^T dnum and the key-side dS^T zhat, then J and the row mask; writes
//              dz_tr.
//   bwd_final  dv and dbias cast from their fp32 accumulators.
// A workgroup is 4 waves. Products that contract over features ("row dots":
// S, dP) give each wave 16 of the 64 keys (or queries) of a tile; products that
// contract over rows (P z, dS z, P^T dnum, dS^T z) give each wave every fourth
// 16-column tile of the [16, D] accumulator, with the [16, 64] P / dS tile passed
// through LDS. Operand rows are read from global memory (they stay in L1 / L2);
// rows of padded tokens are never loaded, so NaN padding reaches nothing.
#include <math.h>

#include "avey_common.h"
#include "avey_internal.h"

namespace avey {

namespace {

constexpr int kRows = 16;      // query (bwd_rows) or key (bwd_cols) rows per workgroup
constexpr int kTile = 64;      // rows of the other side per pipeline step
constexpr int kPitch = kTile + 4;  // LDS row pitch of a [16][64] tile (floats)

typedef double f64x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
// Same operand layout as the fp32 form (lane (lg, lr) supplies A[lr][lg] and
// B[lg][lr]), but lane (lg, lr) holds C[lg + 4 i][lr] in result register i.
__device__ __forceinline__ f64x4 mfma4(double a, double b, f64x4 c) {
  return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

// Row of the 16 x 16 result that lane group lg holds in accumulator element i.
template <typename A>
__device__ __forceinline__ int acc_row(int lg, int i) {
  return sizeof(A) == 8 ? lg + 4 * i : 4 * lg + i;
}

template <typename A> struct Vec4;
template <> struct Vec4<float> { using type = f32x4; };
template <> struct Vec4<double> { using type = f64x4; };
template <typename A> using v4 = typename Vec4<A>::type;

// Element loads converted to fp32.
template <typename T> struct Io;
template <> struct Io<float> {
  __device__ static float one(const float* p) { return *p; }
  __device__ static f32x4 four(const float* p) { return *(const f32x4*)p; }
  __device__ static void put(float* p, float x) { *p = x; }
};
template <> struct Io<__bf16> {
  __device__ static float one(const __bf16* p) { return (float)*p; }
  __device__ static f32x4 four(const __bf16* p) {
    u32x2 u = *(const u32x2*)p;
    return f32x4{__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                 __uint_as_float(u.y & 0xffff0000u)};
  }
  __device__ static void put(__bf16* p, float x) { *p = (__bf16)x; }
};
template <> struct Io<_Float16> {
  __device__ static float one(const _Float16* p) { return (float)*p; }
  __device__ static f32x4 four(const _Float16* p) {
    f16x4 h = *(const f16x4*)p;
    return f32x4{(float)h.x, (float)h.y, (float)h.z, (float)h.w};
  }
  __device__ static void put(_Float16* p, float x) { *p = (_Float16)x; }
};
// fp64 workspace rows of the fp64 path (dnum); 4-element loads are 32-byte aligned.
template <> struct Io<double> {
  __device__ static double one(const double* p) { return *p; }
  __device__ static f64x4 four(const double* p) { return *(const f64x4*)p; }
};

// Guarded loads without a branch. Written as `ok ? p[i] : other`, a load the compiler
// cannot prove in bounds goes into a branch that waits for it before the branches
// join: one memory round trip per element. Here the load always goes out (to element
// 0 when !ok, which every caller's array holds) and the result is selected, so a
// group of loads shares one wait.
template <typename T>
__device__ __forceinline__ T ld_sel(const T* p, int64_t i, bool ok, T other) {
  const T v = p[ok ? i : 0];
  return ok ? v : other;
}

__device__ __forceinline__ bool row_valid(const uint8_t* valid, int64_t b, int64_t C, int64_t row) {
  const bool in = row < C;
  if (!valid) return in;
  return in & (valid[in ? b * C + row : 0] != 0);
}

__device__ __forceinline__ float inv_norm(const float* nrm, int64_t idx, float norm_eps) {
  return 1.f / fmaxf(nrm[idx], norm_eps);
}
__device__ __forceinline__ double inv_norm(const double* nrm, int64_t idx, double norm_eps) {
  return 1.0 / fmax(nrm[idx], norm_eps);
}
// 1 / max(||row||, norm_eps) when ok, else 0 (branch-free, as ld_sel).
template <typename A>
__device__ __forceinline__ A inv_norm_sel(const A* nrm, int64_t idx, bool ok, A norm_eps) {
  const A x = inv_norm(nrm, ok ? idx : 0, norm_eps);
  return ok ? x : A(0);
}

// Four consecutive features d..d+3 of one row (zero past D), converted to A. `vec`:
// rows are 4-element aligned (D % 4 == 0), so a vector load is in bounds when d + 4 <= D.
template <typename A, typename T>
__device__ __forceinline__ v4<A> row4(const T* row, int d, int D, bool vec) {
  if (vec && d + 4 <= D) return __builtin_convertvector(Io<T>::four(row + d), v4<A>);
  v4<A> x = {A(0), A(0), A(0), A(0)};
  if (d < D) x[0] = (A)Io<T>::one(row + d);
  if (d + 1 < D) x[1] = (A)Io<T>::one(row + d + 1);
  if (d + 2 < D) x[2] = (A)Io<T>::one(row + d + 2);
  if (d + 3 < D) x[3] = (A)Io<T>::one(row + d + 3);
  return x;
}

// 16 x 16 block of A B^T contracted over D features. A row lr of the block is
// `a` (scaled by sa), B row lr is `b` (scaled by sb); both are always readable rows,
// taken as zeros where !aok / !bok. Lane (lg, lr) feeds features 16s + 4lg + t at
// sub-step t of step s to both operands (any bijection of the contracted index gives
// the same sum), so every load is four consecutive features. With 4-element aligned
// rows, the loads of U steps go out before their MFMAs and no load sits in a branch
// (see ld_sel). Result: lane holds C[acc_row<A>(lg, i)][lr], i = 0..3.
template <typename A, typename TA, typename TB>
__device__ __forceinline__ v4<A> row_dot(const TA* a, bool aok, A sa, const TB* b, bool bok, A sb, int D, bool vec,
                                         int lg) {
  v4<A> c = {A(0), A(0), A(0), A(0)};
  const int steps = (D + 15) >> 4;
  if (vec) {
    constexpr int U = sizeof(A) == 8 ? 2 : 4;
    for (int s0 = 0; s0 < steps; s0 += U) {
      decltype(Io<TA>::four(a)) x[U];
      decltype(Io<TB>::four(b)) y[U];
      bool xo[U], yo[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int d = 16 * (s0 + u) + 4 * lg;
        const bool in = s0 + u < steps && d < D;  // D % 4 == 0: then d + 4 <= D
        x[u] = Io<TA>::four(a + (in ? d : 0));
        y[u] = Io<TB>::four(b + (in ? d : 0));
        xo[u] = in && aok;
        yo[u] = in && bok;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (s0 + u >= steps) break;
#pragma unroll
        for (int t = 0; t < 4; ++t)
          c = mfma4((xo[u] ? (A)x[u][t] : A(0)) * sa, (yo[u] ? (A)y[u][t] : A(0)) * sb, c);
      }
    }
    return c;
  }
  for (int s = 0; s < steps; ++s) {
    const int d = 16 * s + 4 * lg;
    v4<A> x = aok ? row4<A, TA>(a, d, D, false) : v4<A>{A(0), A(0), A(0), A(0)};
    v4<A> y = bok ? row4<A, TB>(b, d, D, false) : v4<A>{A(0), A(0), A(0), A(0)};
#pragma unroll
    for (int t = 0; t < 4; ++t) c = mfma4(x[t] * sa, y[t] * sb, c);
  }
  return c;
}

// acc[t] (16 x 16, columns 16 (w + 4t) ..) += At (16 x 64, LDS, pitch kPitch)
// times rows r0 .. r0+63 of Y (row stride D). Row r0 + 4s + lg is read only when
// bit s of `rows_ok` is set.
template <typename A, typename T, int MAXT>
__device__ __forceinline__ void rows_acc(v4<A> (&acc)[MAXT], const A* At, const T* Y, int64_t r0, uint32_t rows_ok,
                                         int D, int w, int lr, int lg) {
  A af[16];
#pragma unroll
  for (int s = 0; s < 16; ++s) af[s] = At[lr * kPitch + 4 * s + lg];
  const int ntiles = (D + 15) >> 4;
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    const int tile = w + 4 * t;
    if (tile >= ntiles) break;
    const int col = 16 * tile + lr;
    A yv[16];
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const bool ok = ((rows_ok >> s) & 1u) && col < D;
      yv[s] = (A)ld_sel(Y, (r0 + lg + 4 * s) * (int64_t)D + col, ok, T(0));
    }
#pragma unroll
    for (int s = 0; s < 16; ++s) acc[t] = mfma4(af[s], yv[s], acc[t]);
  }
}

// Sum over the 16 lanes of a lane group (lanes sharing lg).
template <typename A>
__device__ __forceinline__ A sum16(A x) {
  x += __shfl_xor(x, 1);
  x += __shfl_xor(x, 2);
  x += __shfl_xor(x, 4);
  x += __shfl_xor(x, 8);
  return x;
}

// d act(u) / du; the derivatives autograd takes of ops.py:49-58.
template <typename A>
__device__ __forceinline__ A act_grad(A x, int act) {
  switch (act) {
    case AVEY_ACT_RELU: return x > A(0) ? A(1) : A(0);
    case AVEY_ACT_RELU2: return x > A(0) ? A(2) * x : A(0);
    case AVEY_ACT_SILU: {
      A e = exp(-fabs(x));
      A s = x >= A(0) ? A(1) / (A(1) + e) : e / (A(1) + e);
      return s * (A(1) + x * (A(1) - s));
    }
    case AVEY_ACT_GELU: {
      const A k = A(0.7978845608028654);
      A t = tanh(k * (x + A(0.044715) * x * x * x));
      return A(0.5) * (A(1) + t) + A(0.5) * x * (A(1) - t * t) * k * (A(1) + A(3) * A(0.044715) * x * x);
    }
    default: return A(1);
  }
}

// (batch item, row tile) of this workgroup in a 1-D grid of B * nt workgroups.
// Workgroups are dealt to the 8 XCDs round-robin by linear id, so ids are mapped
// such that the tiles of one batch item run on one XCD (B a multiple of 8) or on
// 8 / B of them (B divides 8), and that batch item's rows stay in those XCDs' L2.
// `heavy_last`: tiles are visited last-first (causal query tiles grow heavier).
__device__ __forceinline__ void tile_of_block(int64_t B, int64_t nt, bool heavy_last, int64_t& b, int64_t& t) {
  const int64_t L = blockIdx.x;
  if (B % 8 == 0) {
    const int64_t slot = L >> 3;
    b = (L & 7) + 8 * (slot / nt);
    t = slot % nt;
  } else {
    b = L % B;
    t = L / B;
  }
  if (heavy_last) t = nt - 1 - t;
}

// Workspace of a path computing in A (the bf16 path: A = float).
template <typename A>
struct WsT {
  A *nrm, *dnum, *dden, *dzr, *dv, *db;
  // bf16 path only: z transposed per batch item [D][cp] (padded rows zero),
  // dnum in bf16 row-major [C][D] and transposed [D][cp].
  __bf16 *zt, *dn16, *dnt;
  int64_t cp;
};
using Ws = WsT<float>;

// Workspace layout in elements of A (each part 64 elements, so at least 256 bytes,
// aligned): nrm [B*C], dden [B*C], dzr [B*C*D]; then the A paths' dnum [B*C*D], or
// the bf16 path's zt [B*D*cp], dn16 [B*C*D] and dnt [B*D*cp] bf16 (cp = C rounded up
// to 128); then dv [C*C] and dbias [D] when present.
__host__ __device__ inline int64_t up64(int64_t n) { return (n + 63) & ~int64_t(63); }

template <typename A>
__host__ inline int64_t ws_parts(int64_t B, int64_t C, int64_t D, bool has_v, bool has_bias, bool fast,
                                 WsT<A>* w, void* base) {
  const int64_t cp = (C + 127) & ~int64_t(127);  // a multiple of the bf16 kernels' 128-row tiles
  int64_t off = 0;
  auto take = [&](int64_t n) { const int64_t o = off; off += up64(n); return o; };
  const int64_t o_nrm = take(B * C), o_dden = take(B * C), o_dzr = take(B * C * D);
  const int64_t o_dnum = fast ? -1 : take(B * C * D);
  const int64_t o_zt = fast ? take((B * D * cp + 1) / 2) : -1;
  const int64_t o_dn16 = fast ? take((B * C * D + 1) / 2) : -1;
  const int64_t o_dnt = fast ? take((B * D * cp + 1) / 2) : -1;
  const int64_t o_dv = has_v ? take(C * C) : -1;
  const int64_t o_db = has_bias ? take(D) : -1;
  if (w) {
    A* f = (A*)base;
    w->nrm = f + o_nrm;
    w->dden = f + o_dden;
    w->dzr = f + o_dzr;
    w->dnum = o_dnum >= 0 ? f + o_dnum : nullptr;
    w->zt = o_zt >= 0 ? (__bf16*)(f + o_zt) : nullptr;
    w->dn16 = o_dn16 >= 0 ? (__bf16*)(f + o_dn16) : nullptr;
    w->dnt = o_dnt >= 0 ? (__bf16*)(f + o_dnt) : nullptr;
    w->dv = o_dv >= 0 ? f + o_dv : nullptr;
    w->db = o_db >= 0 ? f + o_db : nullptr;
    w->cp = cp;
  }
  return off;
}

template <typename A>
__host__ inline WsT<A> carve(void* base, int64_t B, int64_t C, int64_t D, bool has_v, bool has_bias, bool fast) {
  WsT<A> w;
  ws_parts<A>(B, C, D, has_v, has_bias, fast, &w, base);
  return w;
}

// One wave per row: ||z|| of the masked row. Every thread also clears a share of
// the dv / dbias accumulators.
template <typename T, typename A>
__global__ __launch_bounds__(256) void bwd_prep_kernel(BwdParams p, WsT<A> ws) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t rows = p.B * p.C;
  if (row < rows) {
    const int64_t b = row / p.C, c = row % p.C;
    A ss = A(0);
    if (row_valid(p.valid, b, p.C, c)) {
      const T* z = (const T*)p.z + row * p.D;
      for (int64_t d = lane; d < p.D; d += 64) {
        A x = (A)Io<T>::one(z + d);
        ss += x * x;
      }
    }
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    if (lane == 0) ws.nrm[row] = sqrt(ss);
  }
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x, nt = (int64_t)gridDim.x * blockDim.x;
  if (ws.dv)
    for (int64_t i = tid; i < p.C * p.C; i += nt) ws.dv[i] = A(0);
  if (ws.db)
    for (int64_t i = tid; i < p.D; i += nt) ws.db[i] = A(0);
}

template <typename T, typename A, int MAXT>
__global__ __launch_bounds__(256) void bwd_rows_kernel(BwdParams p, WsT<A> ws) {
  constexpr int dp = 64 * MAXT + 4;          // pitch of dnl; D <= 64 * MAXT
  __shared__ A tile[kRows * kPitch];         // [16][kPitch]: P, then dS * inv(key)
  __shared__ A red[4 * kRows];               // [4 waves][16]
  __shared__ A stat[2 * kRows];              // den, dden of the block's rows
  __shared__ __attribute__((aligned(32))) A dnl[kRows * dp];  // dnum of the block's rows
  const int D = (int)p.D;
  // Heaviest query tiles first (in causal mode the last ones visit the most key tiles).
  const int64_t C = p.C;
  int64_t b, qtile;
  tile_of_block(p.B, cdiv(C, kRows), true, b, qtile);
  const int64_t q0 = qtile * kRows;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, lr = l & 15, lg = l >> 4;
  const bool vec = (D & 3) == 0;
  const A neps = (A)p.norm_eps;
  const T* zb = (const T*)p.z + b * C * D;
  const int64_t qend = q0 + kRows < C ? q0 + kRows : C;
  const int64_t nkt = p.causal ? cdiv(qend, kTile) : cdiv(C, kTile);
  const bool hv = p.v != nullptr;
  const T* vt = hv ? (const T*)p.v : zb;  // stand-in when absent (see ld_sel)

  // A-operand rows of the row dots: query q0 + lr.
  const int64_t qa = q0 + lr;
  const bool qa_ok = row_valid(p.valid, b, C, qa);
  const T* qa_row = zb + (qa_ok ? qa : 0) * D;
  const A qa_inv = inv_norm_sel(ws.nrm, b * C + qa, qa_ok, neps);

  // ---- pass 1: num, den ----
  v4<A> acc[MAXT];
#pragma unroll
  for (int t = 0; t < MAXT; ++t) acc[t] = v4<A>{A(0), A(0), A(0), A(0)};
  A den4[4] = {A(0), A(0), A(0), A(0)};
  for (int64_t kt = 0; kt < nkt; ++kt) {
    const int64_t k = kt * kTile + 16 * w + lr;  // this lane's key (B row, output column)
    const bool k_ok = row_valid(p.valid, b, C, k);
    const A k_inv = inv_norm_sel(ws.nrm, b * C + k, k_ok, neps);
    v4<A> s4 = row_dot<A, T, T>(qa_row, qa_ok, qa_inv, zb + (k_ok ? k : 0) * D, k_ok, k_inv, D, vec, lg);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t q = q0 + acc_row<A>(lg, i);
      const bool m = k_ok && q < C && (!p.causal || k <= q);
      const A vl = (A)ld_sel(vt, q * C + k, m && hv, T(0)), vv = hv ? vl : A(1);
      const A pv = m ? s4[i] * vv : A(0);  // a select: a use inside `if (m)` sinks the load there
      den4[i] += pv;
      tile[acc_row<A>(lg, i) * kPitch + 16 * w + lr] = pv;
    }
    uint32_t rows_ok = 0;
#pragma unroll
    for (int s = 0; s < 16; ++s) rows_ok |= (uint32_t)row_valid(p.valid, b, C, kt * kTile + 4 * s + lg) << s;
    __syncthreads();
    rows_acc<A, T, MAXT>(acc, tile, zb, kt * kTile, rows_ok, D, w, lr, lg);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    A x = sum16(den4[i]);
    if (lr == 0) red[w * kRows + acc_row<A>(lg, i)] = x;
  }
  __syncthreads();
  if (threadIdx.x < kRows) {
    const int i = threadIdx.x;
    stat[i] = red[i] + red[kRows + i] + red[2 * kRows + i] + red[3 * kRows + i] + (A)p.eps;
  }
  __syncthreads();

  // ---- epilogue 1: dz_tl, dnum, dden, dbias ----
  const int ntiles = (D + 15) >> 4;
  A ddp[4] = {A(0), A(0), A(0), A(0)};
  const bool hg = p.gate != nullptr, hb = p.bias != nullptr;
  const T* ob = (const T*)p.dout + b * C * D;
  const T* gb = hg ? (const T*)p.gate + b * C * D : ob;  // stand-ins when absent (see ld_sel)
  const T* bsp = hb ? (const T*)p.bias : ob;
  T* dgb = p.dgate ? (T*)p.dgate + b * C * D : nullptr;
  bool rqv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) rqv[i] = row_valid(p.valid, b, C, q0 + acc_row<A>(lg, i));
  // Four column tiles at a time, inputs loaded before the first store: the stores may
  // alias the inputs as far as the compiler can tell, so otherwise every element's
  // loads wait until the previous element's stores have gone out.
  constexpr int EB = MAXT < 4 ? MAXT : 4;
#pragma unroll
  for (int t0 = 0; t0 < MAXT; t0 += EB) {
    if (w + 4 * t0 >= ntiles) break;
    float gov[EB][4], gtv[EB][4], bsv[EB];
#pragma unroll
    for (int e = 0; e < EB; ++e) {
      const int col = 16 * (w + 4 * (t0 + e)) + lr;
      const bool cin = w + 4 * (t0 + e) < ntiles && col < D;
      bsv[e] = (float)ld_sel(bsp, col, cin && hb, T(0));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t q = q0 + acc_row<A>(lg, i);
        const bool ok = cin && rqv[i];
        gov[e][i] = (float)ld_sel(ob, q * D + col, ok, T(0));
        const float gl = (float)ld_sel(gb, q * D + col, ok && hg, T(0));
        gtv[e][i] = hg ? gl : 1.f;
      }
    }
#pragma unroll
    for (int e = 0; e < EB; ++e) {
      const int t = t0 + e;
      const int tile_i = w + 4 * t;
      if (tile_i >= ntiles) break;
      const int col = 16 * tile_i + lr;
      A dbs = A(0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = acc_row<A>(lg, i);
        const int64_t q = q0 + row;
        A dn = A(0);
        if (col < D && q < C) {
          const A den = stat[row];
          const A y = p.normalize ? acc[t][i] / den : acc[t][i];
          const A u = y + (A)bsv[e];
          const A go = (A)gov[e][i];
          const A gt = (A)gtv[e][i];
          if (dgb) Io<T>::put(dgb + q * D + col, (float)(go * activate<A>(u, p.act)));
          const A du = go * gt * act_grad(u, p.act);
          dbs += du;
          dn = p.normalize ? du / den : du;
          ddp[i] += du * y;
          ws.dnum[(b * C + q) * D + col] = dn;
        }
        dnl[row * dp + col] = dn;
      }
      if (ws.db) {
        dbs += __shfl_xor(dbs, 16);
        dbs += __shfl_xor(dbs, 32);
        if (lg == 0 && col < D) unsafeAtomicAdd(ws.db + col, dbs);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    A x = sum16(ddp[i]);
    if (lr == 0) red[w * kRows + acc_row<A>(lg, i)] = x;
  }
  __syncthreads();
  if (threadIdx.x < kRows) {
    const int i = threadIdx.x;
    const int64_t q = q0 + i;
    A dd = A(0);
    if (p.normalize) dd = -(red[i] + red[kRows + i] + red[2 * kRows + i] + red[3 * kRows + i]) / stat[i];
    stat[kRows + i] = dd;
    if (q < C) ws.dden[b * C + q] = dd;
  }
  __syncthreads();

  // ---- pass 2: dP, dS, dv, dS zhat ----
#pragma unroll
  for (int t = 0; t < MAXT; ++t) acc[t] = v4<A>{A(0), A(0), A(0), A(0)};
  const A* dn_row = dnl + lr * dp;  // A rows of dP = dnum z^T (zeros for rows past C)
  for (int64_t kt = 0; kt < nkt; ++kt) {
    const int64_t k = kt * kTile + 16 * w + lr;
    const bool k_ok = row_valid(p.valid, b, C, k);
    const A k_inv = inv_norm_sel(ws.nrm, b * C + k, k_ok, neps);
    const T* k_row = zb + (k_ok ? k : 0) * D;
    v4<A> s4 = row_dot<A, T, T>(qa_row, qa_ok, qa_inv, k_row, k_ok, k_inv, D, vec, lg);
    v4<A> d4 = row_dot<A, A, T>(dn_row, true, A(1), k_row, k_ok, A(1), D, vec, lg);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t q = q0 + acc_row<A>(lg, i);
      const bool m = k_ok && q < C && (!p.causal || k <= q);
      const A vl = (A)ld_sel(vt, q * C + k, m && hv, T(0)), vv = hv ? vl : A(1);
      const A dpv = d4[i] + stat[kRows + acc_row<A>(lg, i)];
      const A dsv = m ? dpv * vv * k_inv : A(0);
      if (m && ws.dv) unsafeAtomicAdd(ws.dv + q * C + k, dpv * s4[i]);
      tile[acc_row<A>(lg, i) * kPitch + 16 * w + lr] = dsv;
    }
    uint32_t rows_ok = 0;
#pragma unroll
    for (int s = 0; s < 16; ++s) rows_ok |= (uint32_t)row_valid(p.valid, b, C, kt * kTile + 4 * s + lg) << s;
    __syncthreads();
    rows_acc<A, T, MAXT>(acc, tile, zb, kt * kTile, rows_ok, D, w, lr, lg);
    __syncthreads();
  }
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    const int tile_i = w + 4 * t;
    if (tile_i >= ntiles) break;
    const int col = 16 * tile_i + lr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t q = q0 + acc_row<A>(lg, i);
      if (col < D && q < C) ws.dzr[(b * C + q) * D + col] = acc[t][i];
    }
  }
}

template <typename T, typename A, int MAXT>
__global__ __launch_bounds__(256) void bwd_cols_kernel(BwdParams p, WsT<A> ws) {
  __shared__ A pt[kRows * kPitch];  // P^T tile [16 keys][64 queries]
  __shared__ A dt[kRows * kPitch];  // (dS * inv(query))^T tile
  __shared__ A red[4 * kRows];
  __shared__ A rad[kRows];
  const int D = (int)p.D;
  const int64_t C = p.C;
  int64_t b, ktile;
  tile_of_block(p.B, cdiv(C, kRows), false, b, ktile);  // causal: the first key tiles are the heaviest
  const int64_t k0 = ktile * kRows;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, lr = l & 15, lg = l >> 4;
  const bool vec = (D & 3) == 0;
  const A neps = (A)p.norm_eps;
  const T* zb = (const T*)p.z + b * C * D;
  const A* dnb = ws.dnum + b * C * D;
  const bool hv = p.v != nullptr;
  const T* vt = hv ? (const T*)p.v : zb;  // stand-in when absent (see ld_sel)

  const int64_t ka = k0 + lr;  // A row of the row dots: key k0 + lr
  const bool ka_ok = row_valid(p.valid, b, C, ka);
  const T* ka_row = zb + (ka_ok ? ka : 0) * D;
  const A ka_inv = inv_norm_sel(ws.nrm, b * C + ka, ka_ok, neps);

  v4<A> acc1[MAXT], acc2[MAXT];
#pragma unroll
  for (int t = 0; t < MAXT; ++t) acc1[t] = acc2[t] = v4<A>{A(0), A(0), A(0), A(0)};
  const int64_t qstart = p.causal ? k0 : 0;
  for (int64_t qt = qstart; qt < C; qt += kTile) {
    const int64_t q = qt + 16 * w + lr;  // this lane's query (B row, output column)
    const bool q_in = q < C;
    const bool q_ok = row_valid(p.valid, b, C, q);
    const A q_inv = inv_norm_sel(ws.nrm, b * C + q, q_ok, neps);
    v4<A> s4 = row_dot<A, T, T>(ka_row, ka_ok, ka_inv, zb + (q_ok ? q : 0) * D, q_ok, q_inv, D, vec, lg);
    v4<A> d4 = row_dot<A, T, A>(ka_row, ka_ok, A(1), dnb + (q_in ? q : 0) * D, q_in, A(1), D, vec, lg);
    const A dd = ld_sel(ws.dden, b * C + q, q_in, A(0));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t k = k0 + acc_row<A>(lg, i);
      const bool m = q_in && row_valid(p.valid, b, C, k) && (!p.causal || k <= q);
      const A vl = (A)ld_sel(vt, q * C + k, m && hv, T(0)), vv = hv ? vl : A(1);
      const A pv = m ? s4[i] * vv : A(0);
      const A dsv = m ? (d4[i] + dd) * vv * q_inv : A(0);
      pt[acc_row<A>(lg, i) * kPitch + 16 * w + lr] = pv;
      dt[acc_row<A>(lg, i) * kPitch + 16 * w + lr] = dsv;
    }
    uint32_t in_ok = 0, rows_ok = 0;
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int64_t r = qt + 4 * s + lg;
      in_ok |= (uint32_t)(r < C) << s;
      rows_ok |= (uint32_t)row_valid(p.valid, b, C, r) << s;
    }
    __syncthreads();
    rows_acc<A, A, MAXT>(acc1, pt, dnb, qt, in_ok, D, w, lr, lg);
    rows_acc<A, T, MAXT>(acc2, dt, zb, qt, rows_ok, D, w, lr, lg);
    __syncthreads();
  }

  // Epilogue: dzhat = key-side + query-side parts; J; row mask. Loads are branch-free
  // (see ld_sel), and the stores go out four column tiles at a time after that group's
  // loads (the compiler cannot tell dz_tr from z apart).
  const int ntiles = (D + 15) >> 4;
  bool kv[4];
  A kinv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t k = k0 + acc_row<A>(lg, i);
    kv[i] = row_valid(p.valid, b, C, k);
    kinv[i] = inv_norm_sel(ws.nrm, b * C + k, kv[i], neps);
  }
  A rp[4] = {A(0), A(0), A(0), A(0)};
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    const int tile_i = w + 4 * t;
    if (tile_i >= ntiles) break;
    const int col = 16 * tile_i + lr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t k = k0 + acc_row<A>(lg, i);
      const bool ok = col < D && kv[i];
      const A dq = ld_sel(ws.dzr, (b * C + k) * D + col, ok, A(0));
      const A zv = (A)ld_sel(zb, k * D + col, ok, T(0));
      if (ok) {
        const A g = acc2[t][i] + dq;
        acc2[t][i] = g;
        rp[i] += zv * g;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    A x = sum16(rp[i]);
    if (lr == 0) red[w * kRows + acc_row<A>(lg, i)] = x;
  }
  __syncthreads();
  if (threadIdx.x < kRows) {
    const int i = threadIdx.x;
    const int64_t k = k0 + i;
    A r = A(0);
    if (row_valid(p.valid, b, C, k)) {
      const A n = ws.nrm[b * C + k];
      // zhat . dzhat / ||z|| when the norm is not clamped; no radial term otherwise.
      if (n >= neps) r = (red[i] + red[kRows + i] + red[2 * kRows + i] + red[3 * kRows + i]) / n;
    }
    rad[i] = r;
  }
  __syncthreads();
  T* dzb = (T*)p.dz + b * C * D;
  constexpr int EB = MAXT < 4 ? MAXT : 4;
#pragma unroll
  for (int t0 = 0; t0 < MAXT; t0 += EB) {
    if (w + 4 * t0 >= ntiles) break;
    float zv[EB][4];
#pragma unroll
    for (int e = 0; e < EB; ++e) {
      const int col = 16 * (w + 4 * (t0 + e)) + lr;
      const bool cin = w + 4 * (t0 + e) < ntiles && col < D;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        zv[e][i] = (float)ld_sel(zb, (k0 + acc_row<A>(lg, i)) * D + col, cin && kv[i], T(0));
    }
#pragma unroll
    for (int e = 0; e < EB; ++e) {
      const int t = t0 + e;
      const int tile_i = w + 4 * t;
      if (tile_i >= ntiles) break;
      const int col = 16 * tile_i + lr;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t k = k0 + acc_row<A>(lg, i);
        if (col >= D || k >= C) continue;
        A g = A(0);
        if (kv[i]) {
          const A zh = (A)zv[e][i] * kinv[i];
          g = acc1[t][i] + (acc2[t][i] - zh * rad[acc_row<A>(lg, i)]) * kinv[i];
        }
        Io<T>::put(dzb + k * D + col, (float)g);
      }
    }
  }
}

template <typename T, typename A>
__global__ __launch_bounds__(256) void bwd_final_kernel(BwdParams p, WsT<A> ws) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x, nt = (int64_t)gridDim.x * blockDim.x;
  if (p.dv)
    for (int64_t i = tid; i < p.C * p.C; i += nt) Io<T>::put((T*)p.dv + i, (float)ws.dv[i]);
  if (p.dbias)
    for (int64_t i = tid; i < p.D; i += nt) Io<T>::put((T*)p.dbias + i, (float)ws.db[i]);
}

// ---------------------------------------------------------------------------
// bf16 path: 16x16x32 bf16 MFMA (fp32 accumulation) on bf16 operands, every
// operand a 16-byte load. Products over features take z rows as stored (the
// similarity is scaled by both inverse norms afterwards, so no operand is
// re-rounded); products over rows take their right operand from transposed
// copies (z^T, dnum^T) so that 8 consecutive rows of one column are adjacent.
// P and dS are rounded to bf16 as MFMA operands, and so is dnum in the products
// over rows (P^T dnum); the row dots of dP take dnum as two bf16 parts (hi and the
// rounding remainder). den, dden, dv, the accumulators and the epilogues stay fp32.
// Needs D % 8 == 0 and a 16-byte aligned z_tr.

// The bf16 kernels run NW waves per workgroup: row tiles of KT = 16 NW rows on the
// other side, a [16][KT] P / dS tile in LDS (pitch KT + 8 bf16), and wave w owning
// the 16-column tiles w, w + NW, w + 2 NW, ... of the [16, D] accumulators.
template <int NW>
__device__ __forceinline__ float sum_waves(const float* red, int i) {
  float x = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) x += red[w * kRows + i];
  return x;
}

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 ld8(const __bf16* p) { return *(const bf16x8*)p; }
__device__ __forceinline__ bf16x8 zero8() { return __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u}); }

// 16 x 16 block of A B^T over D features (A row lr = a, in LDS; B row lr = b, a row
// of global memory that is always readable, taken as zeros where !bok). Lane group lg
// feeds features 32s + 8lg .. +7 at step s. Loads of 8 steps are issued before their
// MFMAs, without branches (see ld_sel). Result: lane holds C[4 lg + i][lr].
__device__ __forceinline__ f32x4 row_dot16(const __bf16* a, const __bf16* b, bool bok, int D, int lg) {
  f32x4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
  const int steps = (D + 31) >> 5;
  for (int s0 = 0; s0 < steps; s0 += 8) {
    bf16x8 x[8], y[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int d = 32 * (s0 + u) + 8 * lg;
      const bool in = s0 + u < steps && d < D;
      x[u] = in ? ld8(a + d) : zero8();
      const bf16x8 yl = ld8(b + (in ? d : 0));
      y[u] = (bok && in) ? yl : zero8();
    }
#pragma unroll
    for (int u = 0; u < 8; u += 2) {
      c0 = mfma16(x[u], y[u], c0);
      c1 = mfma16(x[u + 1], y[u + 1], c1);
    }
  }
  return c0 + c1;
}

// Two row dots sharing the LDS operand: c1 = a b1^T and c2 = a b2^T (a loaded once;
// b1, b2 readable global rows, zeros where !ok1 / !ok2). Same lane layout as row_dot16.
__device__ __forceinline__ void row_dot16x2(const __bf16* a, const __bf16* b1, bool ok1, const __bf16* b2, bool ok2,
                                            int D, int lg, f32x4& c1, f32x4& c2) {
  c1 = f32x4{0.f, 0.f, 0.f, 0.f};
  c2 = f32x4{0.f, 0.f, 0.f, 0.f};
  const int steps = (D + 31) >> 5;
  for (int s0 = 0; s0 < steps; s0 += 4) {
    bf16x8 x1[4], y1[4], y2[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int d = 32 * (s0 + u) + 8 * lg;
      const bool in = s0 + u < steps && d < D;
      const int dl = in ? d : 0;
      x1[u] = in ? ld8(a + d) : zero8();
      const bf16x8 l1 = ld8(b1 + dl), l2 = ld8(b2 + dl);
      y1[u] = (ok1 && in) ? l1 : zero8();
      y2[u] = (ok2 && in) ? l2 : zero8();
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      c1 = mfma16(x1[u], y1[u], c1);
      c2 = mfma16(x1[u], y2[u], c2);
    }
  }
}

// Three row dots sharing the global operand: c1 = a1 b^T, c2 = a2 b^T, c3 = a3 b^T
// (a1..a3 in LDS; b a readable global row, zeros where !bok, loaded once). Same lane
// layout as row_dot16.
__device__ __forceinline__ void row_dot16x3(const __bf16* a1, const __bf16* a2, const __bf16* a3, const __bf16* b,
                                            bool bok, int D, int lg, f32x4& c1, f32x4& c2, f32x4& c3) {
  c1 = f32x4{0.f, 0.f, 0.f, 0.f};
  c2 = f32x4{0.f, 0.f, 0.f, 0.f};
  c3 = f32x4{0.f, 0.f, 0.f, 0.f};
  const int steps = (D + 31) >> 5;
  for (int s0 = 0; s0 < steps; s0 += 4) {
    bf16x8 x1[4], x2[4], x3[4], y[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int d = 32 * (s0 + u) + 8 * lg;
      const bool in = s0 + u < steps && d < D;
      x1[u] = in ? ld8(a1 + d) : zero8();
      x2[u] = in ? ld8(a2 + d) : zero8();
      x3[u] = in ? ld8(a3 + d) : zero8();
      const bf16x8 yl = ld8(b + (in ? d : 0));
      y[u] = (bok && in) ? yl : zero8();
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      c1 = mfma16(x1[u], y[u], c1);
      c2 = mfma16(x2[u], y[u], c2);
      c3 = mfma16(x3[u], y[u], c3);
    }
  }
}

// Copies rows r0 .. r0+15 of z (features contiguous) into LDS rows of pitch `pitch`
// bf16, zero for padded or out-of-range rows. D % 8 == 0.
__device__ __forceinline__ void stage_rows16(__bf16* dst, int pitch, const __bf16* zb, const uint8_t* valid, int64_t b,
                                             int64_t C, int64_t r0, int D) {
  const int chunks = D >> 3;
  for (int i = threadIdx.x; i < kRows * chunks; i += blockDim.x) {
    const int r = i / chunks, c = (i - r * chunks) * 8;
    const int64_t row = r0 + r;
    const bool ok = row_valid(valid, b, C, row);
    const bf16x8 x = ld8(zb + (ok ? row : 0) * D + c);
    *(bf16x8*)(dst + r * pitch + c) = ok ? x : zero8();
  }
}

// acc[t] (columns 16 (w + NW t) ..) += A (16 x KT bf16 in LDS, pitch KT + 8) times
// rows r0 .. r0+KT-1 of Y, read from its transpose Yt [D][cp] (zero past the rows).
// Operands of up to 4 column tiles are in flight at a time.
template <int NW, int MAXT>
__device__ __forceinline__ void rows_acc16(f32x4 (&acc)[MAXT], const __bf16* A, const __bf16* Yt, int64_t r0, int D,
                                           int64_t cp, int w, int lr, int lg) {
  constexpr int KS = NW / 2;  // 32-row MFMA steps per tile
  constexpr int TP = 16 * NW + 8;
  constexpr int G = MAXT < 4 ? MAXT : 4;
  bf16x8 a[KS];
#pragma unroll
  for (int k = 0; k < KS; ++k) a[k] = ld8(A + lr * TP + 32 * k + 8 * lg);
  const int ntiles = (D + 15) >> 4;
#pragma unroll
  for (int t0 = 0; t0 < MAXT; t0 += G) {
    if (w + NW * t0 >= ntiles) break;
    bf16x8 y[G][KS];
#pragma unroll
    for (int t = 0; t < G; ++t) {
      const int col = 16 * (w + NW * (t0 + t)) + lr;
      const bool in = w + NW * (t0 + t) < ntiles && col < D;
      const __bf16* yp = Yt + (int64_t)(in ? col : 0) * cp + r0 + 8 * lg;  // always readable (see ld_sel)
#pragma unroll
      for (int k = 0; k < KS; ++k) {
        const bf16x8 l = ld8(yp + 32 * k);
        y[t][k] = in ? l : zero8();
      }
    }
#pragma unroll
    for (int t = 0; t < G; ++t) {
      if (w + NW * (t0 + t) >= ntiles) break;
#pragma unroll
      for (int k = 0; k < KS; ++k) acc[t0 + t] = mfma16(a[k], y[t][k], acc[t0 + t]);
    }
  }
}

// z^T per batch item into zt [D][cp] (padded and invalid rows zero), and zeros in
// dnum^T's columns from C rounded up to 16 to cp (the rows kernel writes the rest).
// One workgroup per (64 rows, 64 features) block through an LDS tile.
__global__ __launch_bounds__(256) void bwd16_transpose_kernel(BwdParams p, Ws ws) {
  __shared__ __bf16 tl[64][66];
  const int64_t C = p.C, D = p.D, cp = ws.cp, b = blockIdx.z;
  const int64_t c0 = (int64_t)blockIdx.x * 64, d0 = (int64_t)blockIdx.y * 64;
  const __bf16* zb = (const __bf16*)p.z + b * C * D;
  for (int i = threadIdx.x; i < 512; i += 256) {
    const int r = i >> 3, ch = (i & 7) * 8;
    const int64_t c = c0 + r, d = d0 + ch;
    bf16x8 x = zero8();
    if (d < D && row_valid(p.valid, b, C, c)) x = ld8(zb + c * D + d);
#pragma unroll
    for (int e = 0; e < 8; ++e) tl[r][ch + e] = x[e];
  }
  __syncthreads();
  const int64_t c16 = (C + 15) & ~int64_t(15);
  for (int i = threadIdx.x; i < 512; i += 256) {
    const int dd = i >> 3, ch = (i & 7) * 8;
    const int64_t d = d0 + dd, c = c0 + ch;
    if (d >= D) continue;
    bf16x8 x;
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = tl[ch + e][dd];
    *(bf16x8*)(ws.zt + (b * D + d) * cp + c) = x;
    if (c >= c16) *(bf16x8*)(ws.dnt + (b * D + d) * cp + c) = zero8();
  }
}

template <int NW, int MAXT>
__global__ __launch_bounds__(64 * NW) void bwd16_rows_kernel(BwdParams p, Ws ws) {
  constexpr int KT = 16 * NW, TP = KT + 8;
  constexpr int dp = 16 * NW * MAXT + 8;  // bf16 pitch of dnl; D <= 16 NW MAXT
  __shared__ __attribute__((aligned(16))) __bf16 tile[kRows * TP];
  __shared__ float red[NW * kRows];
  __shared__ float stat[2 * kRows];
  __shared__ __attribute__((aligned(16))) __bf16 dnl[kRows * dp];
  // dnum - bf16(dnum): with dnl, the row dots of dP = dnum . z see dnum to about 2^-17
  // of itself, so dP keeps the cancellation between its terms that rounding dnum to
  // bf16 alone would break (measured at C2: dv at 4x the flat bf16 bound with dnum in
  // one part, 0.18 of it with two), and dv and dS are as accurate as fp32 products.
  __shared__ __attribute__((aligned(16))) __bf16 dnlo[kRows * dp];
  __shared__ __attribute__((aligned(16))) __bf16 qzl[kRows * dp];  // the block's query rows
  const int D = (int)p.D;
  // Heaviest query tiles first (in causal mode the last ones visit the most key tiles).
  const int64_t C = p.C, cp = ws.cp;
  int64_t b, qtile;
  tile_of_block(p.B, cdiv(C, kRows), true, b, qtile);
  const int64_t q0 = qtile * kRows;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, lr = l & 15, lg = l >> 4;
  const float neps = (float)p.norm_eps;
  const __bf16* zb = (const __bf16*)p.z + b * C * D;
  const __bf16* ztb = ws.zt + b * D * cp;
  // Optional operands read through a stand-in pointer when absent (selected away), so
  // that no load sits in a branch (see ld_sel).
  const bool hv = p.v != nullptr;
  const __bf16* vt = hv ? (const __bf16*)p.v : zb;
  const int64_t qend = q0 + kRows < C ? q0 + kRows : C;
  const int64_t nkt = p.causal ? cdiv(qend, KT) : cdiv(C, KT);

  stage_rows16(qzl, dp, zb, p.valid, b, C, q0, D);
  const __bf16* qa_row = qzl + lr * dp;  // A rows of the row dots (zero when padded)
  float qinv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t q = q0 + 4 * lg + i;
    qinv[i] = inv_norm_sel(ws.nrm, b * C + q, row_valid(p.valid, b, C, q), neps);
  }

  __syncthreads();

  // ---- pass 1: num, den ----
  f32x4 acc[MAXT];
#pragma unroll
  for (int t = 0; t < MAXT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float den4[4] = {0.f, 0.f, 0.f, 0.f};
  for (int64_t kt = 0; kt < nkt; ++kt) {
    const int64_t k = kt * KT + 16 * w + lr;
    const bool k_ok = row_valid(p.valid, b, C, k);
    const float k_inv = inv_norm_sel(ws.nrm, b * C + k, k_ok, neps);
    // V's words go out ahead of the row dot, and P is formed with selects: a use inside
    // `if (m)` lets the compiler sink each load into its branch and wait there.
    float vv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t q = q0 + 4 * lg + i;
      const bool m = k_ok && q < C && (!p.causal || k <= q);
      const float vl = (float)ld_sel(vt, q * C + k, m && hv, (__bf16)0.f);
      vv[i] = hv ? vl : 1.f;
    }
    const f32x4 s4 = row_dot16(qa_row, zb + (k_ok ? k : 0) * D, k_ok, D, lg);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t q = q0 + 4 * lg + i;
      const bool m = k_ok && q < C && (!p.causal || k <= q);
      const float pv = m ? s4[i] * qinv[i] * k_inv * vv[i] : 0.f;
      den4[i] += pv;
      tile[(4 * lg + i) * TP + 16 * w + lr] = (__bf16)pv;
    }
    __syncthreads();
    rows_acc16<NW, MAXT>(acc, tile, ztb, kt * KT, D, cp, w, lr, lg);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float x = sum16(den4[i]);
    if (lr == 0) red[w * kRows + 4 * lg + i] = x;
  }
  __syncthreads();
  if (threadIdx.x < kRows) {
    const int i = threadIdx.x;
    stat[i] = sum_waves<NW>(red, i) + (float)p.eps;
  }
  __syncthreads();

  // ---- epilogue 1: dz_tl, dnum (LDS, row-major and transposed bf16), dden, dbias ----
  const int ntiles = (D + 15) >> 4;
  float ddp[4] = {0.f, 0.f, 0.f, 0.f};
  const bool hg = p.gate != nullptr, hb = p.bias != nullptr;
  const __bf16* ob = (const __bf16*)p.dout + b * C * D;
  const __bf16* gb = hg ? (const __bf16*)p.gate + b * C * D : ob;
  const __bf16* bsp = hb ? (const __bf16*)p.bias : ob;
  __bf16* dgb = p.dgate ? (__bf16*)p.dgate + b * C * D : nullptr;
  // Every input of the epilogue is loaded before its first store: the stores (dz_tl,
  // dnum) may alias the inputs as far as the compiler can tell, so otherwise each
  // element's loads wait until the previous element's stores have been issued, one
  // memory round trip per element (38% of the heaviest workgroup's time at C2).
  bool rqv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) rqv[i] = row_valid(p.valid, b, C, q0 + 4 * lg + i);
  float gov[MAXT][4], gtv[MAXT][4], bsv[MAXT];
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    const int col = 16 * (w + NW * t) + lr;
    const bool cin = w + NW * t < ntiles && col < D;
    bsv[t] = (float)ld_sel(bsp, col, cin && hb, (__bf16)0.f);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t q = q0 + 4 * lg + i;
      const bool ok = cin && rqv[i];
      gov[t][i] = (float)ld_sel(ob, q * D + col, ok, (__bf16)0.f);
      const float gl = (float)ld_sel(gb, q * D + col, ok && hg, (__bf16)0.f);
      gtv[t][i] = hg ? gl : 1.f;
    }
  }
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    const int tile_i = w + NW * t;
    if (tile_i >= ntiles) break;
    const int col = 16 * tile_i + lr;
    float dbs = 0.f;
    bf16x4 dn4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * lg + i;
      const int64_t q = q0 + row;
      float dn = 0.f;
      if (col < D && q < C) {
        const float den = stat[row];
        const float y = p.normalize ? acc[t][i] / den : acc[t][i];
        const float u = y + bsv[t];
        const float go = gov[t][i], gt = gtv[t][i];
        if (dgb) dgb[q * D + col] = (__bf16)(go * activate<float>(u, p.act));
        const float du = go * gt * act_grad(u, p.act);
        dbs += du;
        dn = p.normalize ? du / den : du;
        ddp[i] += du * y;
        ws.dn16[(b * C + q) * D + col] = (__bf16)dn;
      }
      dn4[i] = (__bf16)dn;
      dnl[row * dp + col] = dn4[i];
      dnlo[row * dp + col] = (__bf16)(dn - (float)dn4[i]);
    }
    if (col < D) *(bf16x4*)(ws.dnt + (b * D + col) * cp + q0 + 4 * lg) = dn4;
    if (ws.db) {
      dbs += __shfl_xor(dbs, 16);
      dbs += __shfl_xor(dbs, 32);
      if (lg == 0 && col < D) unsafeAtomicAdd(ws.db + col, dbs);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float x = sum16(ddp[i]);
    if (lr == 0) red[w * kRows + 4 * lg + i] = x;
  }
  __syncthreads();
  if (threadIdx.x < kRows) {
    const int i = threadIdx.x;
    const int64_t q = q0 + i;
    float dd = 0.f;
    if (p.normalize) dd = -(sum_waves<NW>(red, i)) / stat[i];
    stat[kRows + i] = dd;
    if (q < C) ws.dden[b * C + q] = dd;
  }
  __syncthreads();

  // ---- pass 2: dP, dS, dv, dS zhat ----
#pragma unroll
  for (int t = 0; t < MAXT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const __bf16* dn_row = dnl + lr * dp;
  const __bf16* dnlo_row = dnlo + lr * dp;
  for (int64_t kt = 0; kt < nkt; ++kt) {
    const int64_t k = kt * KT + 16 * w + lr;
    const bool k_ok = row_valid(p.valid, b, C, k);
    const float k_inv = inv_norm_sel(ws.nrm, b * C + k, k_ok, neps);
    float vv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t q = q0 + 4 * lg + i;
      const bool m = k_ok && q < C && (!p.causal || k <= q);
      const float vl = (float)ld_sel(vt, q * C + k, m && hv, (__bf16)0.f);
      vv[i] = hv ? vl : 1.f;
    }
    f32x4 s4, d4, d4lo;
    row_dot16x3(qa_row, dn_row, dnlo_row, zb + (k_ok ? k : 0) * D, k_ok, D, lg, s4, d4, d4lo);
    d4 += d4lo;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t q = q0 + 4 * lg + i;
      const bool m = k_ok && q < C && (!p.causal || k <= q);
      const float dpv = d4[i] + stat[kRows + 4 * lg + i];
      const float dsv = m ? dpv * vv[i] * k_inv : 0.f;
      if (m && ws.dv) unsafeAtomicAdd(ws.dv + q * C + k, dpv * s4[i] * qinv[i] * k_inv);
      tile[(4 * lg + i) * TP + 16 * w + lr] = (__bf16)dsv;
    }
    __syncthreads();
    rows_acc16<NW, MAXT>(acc, tile, ztb, kt * KT, D, cp, w, lr, lg);
    __syncthreads();
  }
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    const int tile_i = w + NW * t;
    if (tile_i >= ntiles) break;
    const int col = 16 * tile_i + lr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t q = q0 + 4 * lg + i;
      if (col < D && q < C) ws.dzr[(b * C + q) * D + col] = acc[t][i];
    }
  }
}

template <int NW, int MAXT>
__global__ __launch_bounds__(64 * NW) void bwd16_cols_kernel(BwdParams p, Ws ws) {
  constexpr int KT = 16 * NW, TP = KT + 8;
  __shared__ __attribute__((aligned(16))) __bf16 pt[kRows * TP];  // P^T [16 keys][KT queries]
  __shared__ __attribute__((aligned(16))) __bf16 dt[kRows * TP];  // (dS * inv(query))^T
  __shared__ float red[NW * kRows];
  __shared__ float rad[kRows];
  constexpr int dp = 16 * NW * MAXT + 8;
  __shared__ __attribute__((aligned(16))) __bf16 kzl[kRows * dp];  // the block's key rows
  const int D = (int)p.D;
  const int64_t C = p.C, cp = ws.cp;
  int64_t b, ktile;
  tile_of_block(p.B, cdiv(C, kRows), false, b, ktile);  // causal: the first key tiles are the heaviest
  const int64_t k0 = ktile * kRows;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, lr = l & 15, lg = l >> 4;
  const float neps = (float)p.norm_eps;
  const __bf16* zb = (const __bf16*)p.z + b * C * D;
  const __bf16* ztb = ws.zt + b * D * cp;
  const __bf16* dnb = ws.dn16 + b * C * D;
  const __bf16* dntb = ws.dnt + b * D * cp;
  const bool hv = p.v != nullptr;
  const __bf16* vt = hv ? (const __bf16*)p.v : zb;  // stand-in when absent (see ld_sel)

  stage_rows16(kzl, dp, zb, p.valid, b, C, k0, D);
  const __bf16* ka_row = kzl + lr * dp;  // A rows of the row dots (zero when padded)
  float kinv[4];
  bool kok[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t k = k0 + 4 * lg + i;
    kok[i] = row_valid(p.valid, b, C, k);
    kinv[i] = inv_norm_sel(ws.nrm, b * C + k, kok[i], neps);
  }

  __syncthreads();
  f32x4 acc1[MAXT], acc2[MAXT];
#pragma unroll
  for (int t = 0; t < MAXT; ++t) acc1[t] = acc2[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Query tiles start at multiples of KT so that the KT rows each one reads from
  // the transposed copies stay inside their cp (a multiple of KT) columns.
  const int64_t qstart = p.causal ? (k0 / KT) * KT : 0;
  for (int64_t qt = qstart; qt < C; qt += KT) {
    const int64_t q = qt + 16 * w + lr;
    const bool q_in = q < C;
    const bool q_ok = row_valid(p.valid, b, C, q);
    const float q_inv = inv_norm_sel(ws.nrm, b * C + q, q_ok, neps);
    float vv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t k = k0 + 4 * lg + i;
      const bool m = q_in && kok[i] && (!p.causal || k <= q);
      const float vl = (float)ld_sel(vt, q * C + k, m && hv, (__bf16)0.f);
      vv[i] = hv ? vl : 1.f;
    }
    const float dd = ld_sel(ws.dden, b * C + q, q_in, 0.f);
    f32x4 s4, d4;
    row_dot16x2(ka_row, zb + (q_ok ? q : 0) * D, q_ok, dnb + (q_in ? q : 0) * D, q_in, D, lg, s4, d4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t k = k0 + 4 * lg + i;
      const bool m = q_in && kok[i] && (!p.causal || k <= q);
      const float pv = m ? s4[i] * kinv[i] * q_inv * vv[i] : 0.f;
      const float dsv = m ? (d4[i] + dd) * vv[i] * q_inv : 0.f;
      pt[(4 * lg + i) * TP + 16 * w + lr] = (__bf16)pv;
      dt[(4 * lg + i) * TP + 16 * w + lr] = (__bf16)dsv;
    }
    __syncthreads();
    rows_acc16<NW, MAXT>(acc1, pt, dntb, qt, D, cp, w, lr, lg);
    rows_acc16<NW, MAXT>(acc2, dt, ztb, qt, D, cp, w, lr, lg);
    __syncthreads();
  }

  // The block's z values are loaded here once and kept for the dz_tr stores below, so
  // that no load follows a store there (the compiler cannot tell dz_tr from z apart and
  // would finish each store's round trip before the next load).
  const int ntiles = (D + 15) >> 4;
  float rp[4] = {0.f, 0.f, 0.f, 0.f};
  float zv[MAXT][4];
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    const int col = 16 * (w + NW * t) + lr;
    const bool cin = w + NW * t < ntiles && col < D;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t k = k0 + 4 * lg + i;
      const bool ok = cin && kok[i];
      const float dq = ld_sel(ws.dzr, (b * C + k) * D + col, ok, 0.f);
      zv[t][i] = (float)ld_sel(zb, k * D + col, ok, (__bf16)0.f);
      const float g = acc2[t][i] + dq;
      acc2[t][i] = g;
      rp[i] += zv[t][i] * g;
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float x = sum16(rp[i]);
    if (lr == 0) red[w * kRows + 4 * lg + i] = x;
  }
  __syncthreads();
  if (threadIdx.x < kRows) {
    const int i = threadIdx.x;
    const int64_t k = k0 + i;
    float r = 0.f;
    if (row_valid(p.valid, b, C, k)) {
      const float n = ws.nrm[b * C + k];
      if (n >= neps) r = (sum_waves<NW>(red, i)) / n;
    }
    rad[i] = r;
  }
  __syncthreads();
  __bf16* dzb = (__bf16*)p.dz + b * C * D;
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    const int tile_i = w + NW * t;
    if (tile_i >= ntiles) break;
    const int col = 16 * tile_i + lr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t k = k0 + 4 * lg + i;
      if (col >= D || k >= C) continue;
      float g = 0.f;
      if (kok[i]) {
        const float zh = zv[t][i] * kinv[i];
        g = acc1[t][i] + (acc2[t][i] - zh * rad[4 * lg + i]) * kinv[i];
      }
      dzb[k * D + col] = (__bf16)g;
    }
  }
}

template <int NW, int MAXT>
hipError_t launch_bwd16_t(const BwdParams& p, hipStream_t s) {
  Ws ws = carve<float>(p.work, p.B, p.C, p.D, p.dv != nullptr, p.dbias != nullptr, true);
  const int64_t rows = p.B * p.C;
  hipLaunchKernelGGL((bwd_prep_kernel<__bf16, float>), dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, s, p, ws);
  hipLaunchKernelGGL(bwd16_transpose_kernel, dim3((unsigned)(ws.cp / 64), (unsigned)cdiv(p.D, 64), (unsigned)p.B),
                     dim3(256), 0, s, p, ws);
  const dim3 grid((unsigned)(cdiv(p.C, kRows) * p.B));  // 1-D, mapped by tile_of_block
  hipLaunchKernelGGL((bwd16_rows_kernel<NW, MAXT>), grid, dim3(64 * NW), 0, s, p, ws);
  hipLaunchKernelGGL((bwd16_cols_kernel<NW, MAXT>), grid, dim3(64 * NW), 0, s, p, ws);
  if (p.dv || p.dbias) {
    const int64_t n = p.dv ? p.C * p.C : p.D;
    const int64_t blocks = cdiv(n, 256) < 1024 ? cdiv(n, 256) : 1024;
    hipLaunchKernelGGL((bwd_final_kernel<__bf16, float>), dim3((unsigned)blocks), dim3(256), 0, s, p, ws);
  }
  return hipGetLastError();
}

template <typename T, typename A, int MAXT>
hipError_t launch_bwd_t(const BwdParams& p, hipStream_t s) {
  WsT<A> ws = carve<A>(p.work, p.B, p.C, p.D, p.dv != nullptr, p.dbias != nullptr, false);
  const int64_t rows = p.B * p.C;
  hipLaunchKernelGGL((bwd_prep_kernel<T, A>), dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, s, p, ws);
  const dim3 grid((unsigned)(cdiv(p.C, kRows) * p.B));  // 1-D, mapped by tile_of_block
  hipLaunchKernelGGL((bwd_rows_kernel<T, A, MAXT>), grid, dim3(256), 0, s, p, ws);
  hipLaunchKernelGGL((bwd_cols_kernel<T, A, MAXT>), grid, dim3(256), 0, s, p, ws);
  if (p.dv || p.dbias) {
    const int64_t n = p.dv ? p.C * p.C : p.D;
    const int64_t blocks = cdiv(n, 256) < 1024 ? cdiv(n, 256) : 1024;
    hipLaunchKernelGGL((bwd_final_kernel<T, A>), dim3((unsigned)blocks), dim3(256), 0, s, p, ws);
  }
  return hipGetLastError();
}

// Accumulator tiles per wave: 4 waves share the (D + 15) / 16 column tiles. The fp64
// path adds a 12-tile step so that D = 768 keeps 2 x 12 (not 2 x 16) fp64
// accumulators of 8 registers each in the cols kernel.
template <typename T, typename A>
hipError_t launch_bwd_d(const BwdParams& p, hipStream_t s) {
  const int64_t tiles = cdiv(p.D, 16);
  if (tiles <= 8) return launch_bwd_t<T, A, 2>(p, s);
  if (tiles <= 16) return launch_bwd_t<T, A, 4>(p, s);
  if (tiles <= 32) return launch_bwd_t<T, A, 8>(p, s);
  if constexpr (sizeof(A) == 8) {
    if (tiles <= 48) return launch_bwd_t<T, A, 12>(p, s);
  }
  return launch_bwd_t<T, A, 16>(p, s);
}

// 8 waves per workgroup: each holds 16-column tiles of up to 8 x 16 features per
// accumulator, so two waves share a SIMD and cover each other's operand loads.
hipError_t launch_bwd16(const BwdParams& p, hipStream_t s) {
  const int64_t tiles = cdiv(p.D, 16);
  if (tiles <= 16) return launch_bwd16_t<8, 2>(p, s);
  if (tiles <= 32) return launch_bwd16_t<8, 4>(p, s);
  return launch_bwd16_t<8, 8>(p, s);
}

}  // namespace

// Normalised (Avey-B) calls compute in fp64 whatever the stored type: their
// gradients divide by the signed row sums den_i, so an evaluation error e in den_i,
// S or num moves every gradient that depends on row i by about e * sum|P_i.| / |den_i|.
// On N(0, 1) inputs that factor reaches 1e4-3e5 (C3, C5): fp32 arithmetic, the
// reference's own autograd included, then misses the flat tol * (1 + |w|) bound by up
// to ~900x, and the bf16 operands of the fast path by more; fp64 leaves ~1e-11.
// The other calls: bf16 with D % 8 == 0 and a 16-byte aligned z_tr take the bf16
// MFMA path, the rest fp32.
BwdPath bwd_path(int dtype, int64_t D, const void* z, bool normalize) {
  if (normalize) return BwdPath::Fp64;
  if (dtype == AVEY_DTYPE_BF16 && D % 8 == 0 && ((uintptr_t)z & 15) == 0) return BwdPath::Bf16;
  return BwdPath::Fp32;
}

int64_t bwd_workspace_bytes(int64_t B, int64_t C, int64_t D, bool has_v, bool has_bias, BwdPath path) {
  if (path == BwdPath::Fp64) return 8 * ws_parts<double>(B, C, D, has_v, has_bias, false, nullptr, nullptr);
  return 4 * ws_parts<float>(B, C, D, has_v, has_bias, path == BwdPath::Bf16, nullptr, nullptr);
}

template <typename A>
hipError_t launch_bwd_a(const BwdParams& p, int dtype, hipStream_t s) {
  switch (dtype) {
    case AVEY_DTYPE_BF16: return launch_bwd_d<__bf16, A>(p, s);
    case AVEY_DTYPE_F16: return launch_bwd_d<_Float16, A>(p, s);
    case AVEY_DTYPE_F32: return launch_bwd_d<float, A>(p, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_bwd(const BwdParams& p, int dtype, hipStream_t s) {
  switch (bwd_path(dtype, p.D, p.z, p.normalize != 0)) {
    case BwdPath::Bf16: return launch_bwd16(p, s);
    case BwdPath::Fp64: return launch_bwd_a<double>(p, dtype, s);
    default: return launch_bwd_a<float>(p, dtype, s);
  }
}

}  // namespace avey
