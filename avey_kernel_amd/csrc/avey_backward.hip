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
// Kernels (all fp32 arithmetic, fp32 MFMA v_mfma_f32_16x16x4f32):
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

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

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

// Four consecutive features d..d+3 of one row (zero past D). `vec`: rows are
// 4-element aligned (D % 4 == 0), so a vector load is in bounds when d + 4 <= D.
template <typename T>
__device__ __forceinline__ f32x4 row4(const T* row, int d, int D, bool vec) {
  if (vec && d + 4 <= D) return Io<T>::four(row + d);
  f32x4 x = {0.f, 0.f, 0.f, 0.f};
  if (d < D) x[0] = Io<T>::one(row + d);
  if (d + 1 < D) x[1] = Io<T>::one(row + d + 1);
  if (d + 2 < D) x[2] = Io<T>::one(row + d + 2);
  if (d + 3 < D) x[3] = Io<T>::one(row + d + 3);
  return x;
}

// 16 x 16 block of A B^T contracted over D features. A row lr of the block is
// `a` (scaled by sa), B row lr is `b` (scaled by sb); a null row contributes
// zeros and is not read. Lane (lg, lr) feeds features 16s + 4lg + t at sub-step
// t of step s to both operands (any bijection of the contracted index gives the
// same sum), so every load is four consecutive features. Result: lane holds
// C[4 lg + i][lr], i = 0..3.
template <typename TA, typename TB>
__device__ __forceinline__ f32x4 row_dot(const TA* a, float sa, const TB* b, float sb, int D, bool vec, int lg) {
  f32x4 c = {0.f, 0.f, 0.f, 0.f};
  const int steps = (D + 15) >> 4;
  for (int s = 0; s < steps; ++s) {
    const int d = 16 * s + 4 * lg;
    f32x4 x = a ? row4<TA>(a, d, D, vec) : f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 y = b ? row4<TB>(b, d, D, vec) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t) c = mfma4(x[t] * sa, y[t] * sb, c);
  }
  return c;
}

// acc[t] (16 x 16, columns 16 (w + 4t) ..) += A (16 x 64, LDS, pitch kPitch)
// times rows r0 .. r0+63 of Y (row stride D). Row r0 + 4s + lg is read only when
// bit s of `rows_ok` is set.
template <typename T, int MAXT>
__device__ __forceinline__ void rows_acc(f32x4 (&acc)[MAXT], const float* A, const T* Y, int64_t r0, uint32_t rows_ok,
                                         int D, int w, int lr, int lg) {
  float af[16];
#pragma unroll
  for (int s = 0; s < 16; ++s) af[s] = A[lr * kPitch + 4 * s + lg];
  const int ntiles = (D + 15) >> 4;
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    const int tile = w + 4 * t;
    if (tile >= ntiles) break;
    const int col = 16 * tile + lr;
    const T* y = Y + (r0 + lg) * (int64_t)D + col;
    float yv[16];
#pragma unroll
    for (int s = 0; s < 16; ++s)
      yv[s] = (((rows_ok >> s) & 1u) && col < D) ? Io<T>::one(y + (int64_t)(4 * s) * D) : 0.f;
#pragma unroll
    for (int s = 0; s < 16; ++s) acc[t] = mfma4(af[s], yv[s], acc[t]);
  }
}

__device__ __forceinline__ bool row_valid(const uint8_t* valid, int64_t b, int64_t C, int64_t row) {
  return row < C && (!valid || valid[b * C + row] != 0);
}

__device__ __forceinline__ float inv_norm(const float* nrm, int64_t idx, float norm_eps) {
  return 1.f / fmaxf(nrm[idx], norm_eps);
}

// Sum over the 16 lanes of a lane group (lanes sharing lg).
__device__ __forceinline__ float sum16(float x) {
  x += __shfl_xor(x, 1);
  x += __shfl_xor(x, 2);
  x += __shfl_xor(x, 4);
  x += __shfl_xor(x, 8);
  return x;
}

// d act(u) / du; the derivatives autograd takes of ops.py:49-58.
__device__ __forceinline__ float act_grad(float x, int act) {
  switch (act) {
    case AVEY_ACT_RELU: return x > 0.f ? 1.f : 0.f;
    case AVEY_ACT_RELU2: return x > 0.f ? 2.f * x : 0.f;
    case AVEY_ACT_SILU: {
      float e = expf(-fabsf(x));
      float s = x >= 0.f ? 1.f / (1.f + e) : e / (1.f + e);
      return s * (1.f + x * (1.f - s));
    }
    case AVEY_ACT_GELU: {
      const float k = 0.7978845608028654f;
      float t = tanhf(k * (x + 0.044715f * x * x * x));
      return 0.5f * (1.f + t) + 0.5f * x * (1.f - t * t) * k * (1.f + 3.f * 0.044715f * x * x);
    }
    default: return 1.f;
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

struct Ws {
  float *nrm, *dnum, *dden, *dzr, *dv, *db;
  // bf16 path only: z transposed per batch item [D][cp] (padded rows zero),
  // dnum in bf16 row-major [C][D] and transposed [D][cp].
  __bf16 *zt, *dn16, *dnt;
  int64_t cp;
};

// Workspace layout (each part 256-byte aligned): nrm [B*C], dden [B*C], dzr
// [B*C*D] fp32; then the fp32 path's dnum [B*C*D] fp32, or the bf16 path's zt
// [B*D*cp], dn16 [B*C*D] and dnt [B*D*cp] bf16 (cp = C rounded up to 128); then
// dv [C*C] and dbias [D] fp32 when present.
__host__ __device__ inline int64_t up64(int64_t n) { return (n + 63) & ~int64_t(63); }

__host__ inline int64_t ws_floats_parts(int64_t B, int64_t C, int64_t D, bool has_v, bool has_bias, bool fast,
                                        Ws* w, void* base) {
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
    float* f = (float*)base;
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

__host__ inline Ws carve(void* base, int64_t B, int64_t C, int64_t D, bool has_v, bool has_bias, bool fast) {
  Ws w;
  ws_floats_parts(B, C, D, has_v, has_bias, fast, &w, base);
  return w;
}

__host__ inline int64_t ws_floats(int64_t B, int64_t C, int64_t D, bool has_v, bool has_bias, bool fast) {
  return ws_floats_parts(B, C, D, has_v, has_bias, fast, nullptr, nullptr);
}

// One wave per row: ||z|| of the masked row. Every thread also clears a share of
// the dv / dbias accumulators.
template <typename T>
__global__ __launch_bounds__(256) void bwd_prep_kernel(BwdParams p, Ws ws) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t rows = p.B * p.C;
  if (row < rows) {
    const int64_t b = row / p.C, c = row % p.C;
    float ss = 0.f;
    if (row_valid(p.valid, b, p.C, c)) {
      const T* z = (const T*)p.z + row * p.D;
      for (int64_t d = lane; d < p.D; d += 64) {
        float x = Io<T>::one(z + d);
        ss += x * x;
      }
    }
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    if (lane == 0) ws.nrm[row] = sqrtf(ss);
  }
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x, nt = (int64_t)gridDim.x * blockDim.x;
  if (ws.dv)
    for (int64_t i = tid; i < p.C * p.C; i += nt) ws.dv[i] = 0.f;
  if (ws.db)
    for (int64_t i = tid; i < p.D; i += nt) ws.db[i] = 0.f;
}

template <typename T, int MAXT>
__global__ __launch_bounds__(256) void bwd_rows_kernel(BwdParams p, Ws ws) {
  constexpr int dp = 64 * MAXT + 4;          // pitch of dnl; D <= 64 * MAXT
  __shared__ float tile[kRows * kPitch];     // [16][kPitch]: P, then dS * inv(key)
  __shared__ float red[4 * kRows];           // [4 waves][16]
  __shared__ float stat[2 * kRows];          // den, dden of the block's rows
  __shared__ __attribute__((aligned(16))) float dnl[kRows * dp];  // dnum of the block's rows
  const int D = (int)p.D;
  // Heaviest query tiles first (in causal mode the last ones visit the most key tiles).
  const int64_t C = p.C;
  int64_t b, qtile;
  tile_of_block(p.B, cdiv(C, kRows), true, b, qtile);
  const int64_t q0 = qtile * kRows;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, lr = l & 15, lg = l >> 4;
  const bool vec = (D & 3) == 0;
  const float neps = (float)p.norm_eps;
  const T* zb = (const T*)p.z + b * C * D;
  const int64_t qend = q0 + kRows < C ? q0 + kRows : C;
  const int64_t nkt = p.causal ? cdiv(qend, kTile) : cdiv(C, kTile);
  const T* vt = (const T*)p.v;

  // A-operand rows of the row dots: query q0 + lr.
  const int64_t qa = q0 + lr;
  const bool qa_ok = row_valid(p.valid, b, C, qa);
  const T* qa_row = qa_ok ? zb + qa * D : nullptr;
  const float qa_inv = qa_ok ? inv_norm(ws.nrm, b * C + qa, neps) : 0.f;

  // ---- pass 1: num, den ----
  f32x4 acc[MAXT];
#pragma unroll
  for (int t = 0; t < MAXT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float den4[4] = {0.f, 0.f, 0.f, 0.f};
  for (int64_t kt = 0; kt < nkt; ++kt) {
    const int64_t k = kt * kTile + 16 * w + lr;  // this lane's key (B row, output column)
    const bool k_ok = row_valid(p.valid, b, C, k);
    const float k_inv = k_ok ? inv_norm(ws.nrm, b * C + k, neps) : 0.f;
    f32x4 s4 = row_dot<T, T>(qa_row, qa_inv, k_ok ? zb + k * D : nullptr, k_inv, D, vec, lg);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t q = q0 + 4 * lg + i;
      const bool m = k_ok && q < C && (!p.causal || k <= q);
      float pv = 0.f;
      if (m) pv = s4[i] * (vt ? Io<T>::one(vt + q * C + k) : 1.f);
      den4[i] += pv;
      tile[(4 * lg + i) * kPitch + 16 * w + lr] = pv;
    }
    uint32_t rows_ok = 0;
#pragma unroll
    for (int s = 0; s < 16; ++s) rows_ok |= (uint32_t)row_valid(p.valid, b, C, kt * kTile + 4 * s + lg) << s;
    __syncthreads();
    rows_acc<T, MAXT>(acc, tile, zb, kt * kTile, rows_ok, D, w, lr, lg);
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
    stat[i] = red[i] + red[kRows + i] + red[2 * kRows + i] + red[3 * kRows + i] + (float)p.eps;
  }
  __syncthreads();

  // ---- epilogue 1: dz_tl, dnum, dden, dbias ----
  const int ntiles = (D + 15) >> 4;
  float ddp[4] = {0.f, 0.f, 0.f, 0.f};
  const T* gb = p.gate ? (const T*)p.gate + b * C * D : nullptr;
  const T* ob = (const T*)p.dout + b * C * D;
  T* dgb = p.dgate ? (T*)p.dgate + b * C * D : nullptr;
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    const int tile_i = w + 4 * t;
    if (tile_i >= ntiles) break;
    const int col = 16 * tile_i + lr;
    float dbs = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * lg + i;
      const int64_t q = q0 + row;
      float dn = 0.f;
      if (col < D && q < C) {
        const bool rq = row_valid(p.valid, b, C, q);
        const float den = stat[row];
        const float y = p.normalize ? acc[t][i] / den : acc[t][i];
        const float u = y + (p.bias ? Io<T>::one((const T*)p.bias + col) : 0.f);
        const float go = rq ? Io<T>::one(ob + q * D + col) : 0.f;
        const float gt = gb ? (rq ? Io<T>::one(gb + q * D + col) : 0.f) : 1.f;
        if (dgb) Io<T>::put(dgb + q * D + col, go * activate<float>(u, p.act));
        const float du = go * gt * act_grad(u, p.act);
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
    if (p.normalize) dd = -(red[i] + red[kRows + i] + red[2 * kRows + i] + red[3 * kRows + i]) / stat[i];
    stat[kRows + i] = dd;
    if (q < C) ws.dden[b * C + q] = dd;
  }
  __syncthreads();

  // ---- pass 2: dP, dS, dv, dS zhat ----
#pragma unroll
  for (int t = 0; t < MAXT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const float* dn_row = dnl + lr * dp;  // A rows of dP = dnum z^T (zeros for rows past C)
  for (int64_t kt = 0; kt < nkt; ++kt) {
    const int64_t k = kt * kTile + 16 * w + lr;
    const bool k_ok = row_valid(p.valid, b, C, k);
    const float k_inv = k_ok ? inv_norm(ws.nrm, b * C + k, neps) : 0.f;
    const T* k_row = k_ok ? zb + k * D : nullptr;
    f32x4 s4 = row_dot<T, T>(qa_row, qa_inv, k_row, k_inv, D, vec, lg);
    f32x4 d4 = row_dot<float, T>(dn_row, 1.f, k_row, 1.f, D, vec, lg);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t q = q0 + 4 * lg + i;
      const bool m = k_ok && q < C && (!p.causal || k <= q);
      float dsv = 0.f;
      if (m) {
        const float dpv = d4[i] + stat[kRows + 4 * lg + i];
        const float vv = vt ? Io<T>::one(vt + q * C + k) : 1.f;
        dsv = dpv * vv * k_inv;
        if (ws.dv) unsafeAtomicAdd(ws.dv + q * C + k, dpv * s4[i]);
      }
      tile[(4 * lg + i) * kPitch + 16 * w + lr] = dsv;
    }
    uint32_t rows_ok = 0;
#pragma unroll
    for (int s = 0; s < 16; ++s) rows_ok |= (uint32_t)row_valid(p.valid, b, C, kt * kTile + 4 * s + lg) << s;
    __syncthreads();
    rows_acc<T, MAXT>(acc, tile, zb, kt * kTile, rows_ok, D, w, lr, lg);
    __syncthreads();
  }
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    const int tile_i = w + 4 * t;
    if (tile_i >= ntiles) break;
    const int col = 16 * tile_i + lr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t q = q0 + 4 * lg + i;
      if (col < D && q < C) ws.dzr[(b * C + q) * D + col] = acc[t][i];
    }
  }
}

template <typename T, int MAXT>
__global__ __launch_bounds__(256) void bwd_cols_kernel(BwdParams p, Ws ws) {
  __shared__ float pt[kRows * kPitch];  // P^T tile [16 keys][64 queries]
  __shared__ float dt[kRows * kPitch];  // (dS * inv(query))^T tile
  __shared__ float red[4 * kRows];
  __shared__ float rad[kRows];
  const int D = (int)p.D;
  const int64_t C = p.C;
  int64_t b, ktile;
  tile_of_block(p.B, cdiv(C, kRows), false, b, ktile);  // causal: the first key tiles are the heaviest
  const int64_t k0 = ktile * kRows;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, lr = l & 15, lg = l >> 4;
  const bool vec = (D & 3) == 0;
  const float neps = (float)p.norm_eps;
  const T* zb = (const T*)p.z + b * C * D;
  const float* dnb = ws.dnum + b * C * D;
  const T* vt = (const T*)p.v;

  const int64_t ka = k0 + lr;  // A row of the row dots: key k0 + lr
  const bool ka_ok = row_valid(p.valid, b, C, ka);
  const T* ka_row = ka_ok ? zb + ka * D : nullptr;
  const float ka_inv = ka_ok ? inv_norm(ws.nrm, b * C + ka, neps) : 0.f;

  f32x4 acc1[MAXT], acc2[MAXT];
#pragma unroll
  for (int t = 0; t < MAXT; ++t) acc1[t] = acc2[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int64_t qstart = p.causal ? k0 : 0;
  for (int64_t qt = qstart; qt < C; qt += kTile) {
    const int64_t q = qt + 16 * w + lr;  // this lane's query (B row, output column)
    const bool q_in = q < C;
    const bool q_ok = row_valid(p.valid, b, C, q);
    const float q_inv = q_ok ? inv_norm(ws.nrm, b * C + q, neps) : 0.f;
    f32x4 s4 = row_dot<T, T>(ka_row, ka_inv, q_ok ? zb + q * D : nullptr, q_inv, D, vec, lg);
    f32x4 d4 = row_dot<T, float>(ka_row, 1.f, q_in ? dnb + q * D : nullptr, 1.f, D, vec, lg);
    const float dd = q_in ? ws.dden[b * C + q] : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t k = k0 + 4 * lg + i;
      const bool m = q_in && row_valid(p.valid, b, C, k) && (!p.causal || k <= q);
      float pv = 0.f, dsv = 0.f;
      if (m) {
        const float vv = vt ? Io<T>::one(vt + q * C + k) : 1.f;
        pv = s4[i] * vv;
        dsv = (d4[i] + dd) * vv * q_inv;
      }
      pt[(4 * lg + i) * kPitch + 16 * w + lr] = pv;
      dt[(4 * lg + i) * kPitch + 16 * w + lr] = dsv;
    }
    uint32_t in_ok = 0, rows_ok = 0;
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int64_t r = qt + 4 * s + lg;
      in_ok |= (uint32_t)(r < C) << s;
      rows_ok |= (uint32_t)row_valid(p.valid, b, C, r) << s;
    }
    __syncthreads();
    rows_acc<float, MAXT>(acc1, pt, dnb, qt, in_ok, D, w, lr, lg);
    rows_acc<T, MAXT>(acc2, dt, zb, qt, rows_ok, D, w, lr, lg);
    __syncthreads();
  }

  // Epilogue: dzhat = key-side + query-side parts; J; row mask.
  const int ntiles = (D + 15) >> 4;
  float rp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    const int tile_i = w + 4 * t;
    if (tile_i >= ntiles) break;
    const int col = 16 * tile_i + lr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t k = k0 + 4 * lg + i;
      if (col < D && row_valid(p.valid, b, C, k)) {
        const float g = acc2[t][i] + ws.dzr[(b * C + k) * D + col];
        acc2[t][i] = g;
        rp[i] += Io<T>::one(zb + k * D + col) * g;
      }
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
      // zhat . dzhat / ||z|| when the norm is not clamped; no radial term otherwise.
      if (n >= neps) r = (red[i] + red[kRows + i] + red[2 * kRows + i] + red[3 * kRows + i]) / n;
    }
    rad[i] = r;
  }
  __syncthreads();
  T* dzb = (T*)p.dz + b * C * D;
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    const int tile_i = w + 4 * t;
    if (tile_i >= ntiles) break;
    const int col = 16 * tile_i + lr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t k = k0 + 4 * lg + i;
      if (col >= D || k >= C) continue;
      float g = 0.f;
      if (row_valid(p.valid, b, C, k)) {
        const float inv = inv_norm(ws.nrm, b * C + k, neps);
        const float zh = Io<T>::one(zb + k * D + col) * inv;
        g = acc1[t][i] + (acc2[t][i] - zh * rad[4 * lg + i]) * inv;
      }
      Io<T>::put(dzb + k * D + col, g);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void bwd_final_kernel(BwdParams p, Ws ws) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x, nt = (int64_t)gridDim.x * blockDim.x;
  if (p.dv)
    for (int64_t i = tid; i < p.C * p.C; i += nt) Io<T>::put((T*)p.dv + i, ws.dv[i]);
  if (p.dbias)
    for (int64_t i = tid; i < p.D; i += nt) Io<T>::put((T*)p.dbias + i, ws.db[i]);
}

// ---------------------------------------------------------------------------
// bf16 path: 16x16x32 bf16 MFMA (fp32 accumulation) on bf16 operands, every
// operand a 16-byte load. Products over features take z rows as stored (the
// similarity is scaled by both inverse norms afterwards, so no operand is
// re-rounded); products over rows take their right operand from transposed
// copies (z^T, dnum^T) so that 8 consecutive rows of one column are adjacent.
// dnum, P and dS are rounded to bf16 as MFMA operands; den, dden, dv, the
// accumulators and the epilogues stay fp32. Needs D % 8 == 0 and a 16-byte
// aligned z_tr.

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

// 16 x 16 block of A B^T over D features (A row lr = a, B row lr = b; a null row
// is zero and not read). Lane group lg feeds features 32s + 8lg .. +7 at step s.
// Loads of 8 steps are issued before their MFMAs. Result: lane holds C[4 lg + i][lr].
__device__ __forceinline__ f32x4 row_dot16(const __bf16* a, const __bf16* b, int D, int lg) {
  f32x4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
  const int steps = (D + 31) >> 5;
  for (int s0 = 0; s0 < steps; s0 += 8) {
    bf16x8 x[8], y[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int d = 32 * (s0 + u) + 8 * lg;
      const bool in = s0 + u < steps && d < D;
      x[u] = (a && in) ? ld8(a + d) : zero8();
      y[u] = (b && in) ? ld8(b + d) : zero8();
    }
#pragma unroll
    for (int u = 0; u < 8; u += 2) {
      c0 = mfma16(x[u], y[u], c0);
      c1 = mfma16(x[u + 1], y[u + 1], c1);
    }
  }
  return c0 + c1;
}

// Two row dots sharing an operand: c1 = a1 b^T and c2 = a2 b^T (b loaded once), or
// with `shared_a`, c1 = a b1^T and c2 = a b2^T (a loaded once). Same lane layout
// as row_dot16; a null row is zero and not read.
template <bool shared_a>
__device__ __forceinline__ void row_dot16x2(const __bf16* a1, const __bf16* a2, const __bf16* b1, const __bf16* b2,
                                            int D, int lg, f32x4& c1, f32x4& c2) {
  c1 = f32x4{0.f, 0.f, 0.f, 0.f};
  c2 = f32x4{0.f, 0.f, 0.f, 0.f};
  const int steps = (D + 31) >> 5;
  for (int s0 = 0; s0 < steps; s0 += 4) {
    bf16x8 x1[4], x2[4], y1[4], y2[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int d = 32 * (s0 + u) + 8 * lg;
      const bool in = s0 + u < steps && d < D;
      if (shared_a) {
        x1[u] = (a1 && in) ? ld8(a1 + d) : zero8();
        y1[u] = (b1 && in) ? ld8(b1 + d) : zero8();
        y2[u] = (b2 && in) ? ld8(b2 + d) : zero8();
      } else {
        x1[u] = (a1 && in) ? ld8(a1 + d) : zero8();
        x2[u] = (a2 && in) ? ld8(a2 + d) : zero8();
        y1[u] = (b1 && in) ? ld8(b1 + d) : zero8();
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (shared_a) {
        c1 = mfma16(x1[u], y1[u], c1);
        c2 = mfma16(x1[u], y2[u], c2);
      } else {
        c1 = mfma16(x1[u], y1[u], c1);
        c2 = mfma16(x2[u], y1[u], c2);
      }
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
    *(bf16x8*)(dst + r * pitch + c) = row_valid(valid, b, C, row) ? ld8(zb + row * D + c) : zero8();
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
      const __bf16* yp = Yt + (int64_t)col * cp + r0 + 8 * lg;
#pragma unroll
      for (int k = 0; k < KS; ++k) y[t][k] = in ? ld8(yp + 32 * k) : zero8();
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
  const __bf16* vt = (const __bf16*)p.v;
  const int64_t qend = q0 + kRows < C ? q0 + kRows : C;
  const int64_t nkt = p.causal ? cdiv(qend, KT) : cdiv(C, KT);

  stage_rows16(qzl, dp, zb, p.valid, b, C, q0, D);
  const __bf16* qa_row = qzl + lr * dp;  // A rows of the row dots (zero when padded)
  float qinv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t q = q0 + 4 * lg + i;
    qinv[i] = row_valid(p.valid, b, C, q) ? inv_norm(ws.nrm, b * C + q, neps) : 0.f;
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
    const float k_inv = k_ok ? inv_norm(ws.nrm, b * C + k, neps) : 0.f;
    const f32x4 s4 = row_dot16(qa_row, k_ok ? zb + k * D : nullptr, D, lg);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t q = q0 + 4 * lg + i;
      const bool m = k_ok && q < C && (!p.causal || k <= q);
      float pv = 0.f;
      if (m) pv = s4[i] * qinv[i] * k_inv * (vt ? (float)vt[q * C + k] : 1.f);
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
  const __bf16* gb = p.gate ? (const __bf16*)p.gate + b * C * D : nullptr;
  const __bf16* ob = (const __bf16*)p.dout + b * C * D;
  __bf16* dgb = p.dgate ? (__bf16*)p.dgate + b * C * D : nullptr;
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
        const bool rq = row_valid(p.valid, b, C, q);
        const float den = stat[row];
        const float y = p.normalize ? acc[t][i] / den : acc[t][i];
        const float u = y + (p.bias ? (float)((const __bf16*)p.bias)[col] : 0.f);
        const float go = rq ? (float)ob[q * D + col] : 0.f;
        const float gt = gb ? (rq ? (float)gb[q * D + col] : 0.f) : 1.f;
        if (dgb) dgb[q * D + col] = (__bf16)(go * activate<float>(u, p.act));
        const float du = go * gt * act_grad(u, p.act);
        dbs += du;
        dn = p.normalize ? du / den : du;
        ddp[i] += du * y;
        ws.dn16[(b * C + q) * D + col] = (__bf16)dn;
      }
      dn4[i] = (__bf16)dn;
      dnl[row * dp + col] = dn4[i];
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
  for (int64_t kt = 0; kt < nkt; ++kt) {
    const int64_t k = kt * KT + 16 * w + lr;
    const bool k_ok = row_valid(p.valid, b, C, k);
    const float k_inv = k_ok ? inv_norm(ws.nrm, b * C + k, neps) : 0.f;
    const __bf16* k_row = k_ok ? zb + k * D : nullptr;
    f32x4 s4, d4;
    row_dot16x2<false>(qa_row, dn_row, k_row, nullptr, D, lg, s4, d4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t q = q0 + 4 * lg + i;
      const bool m = k_ok && q < C && (!p.causal || k <= q);
      float dsv = 0.f;
      if (m) {
        const float dpv = d4[i] + stat[kRows + 4 * lg + i];
        const float vv = vt ? (float)vt[q * C + k] : 1.f;
        dsv = dpv * vv * k_inv;
        if (ws.dv) unsafeAtomicAdd(ws.dv + q * C + k, dpv * s4[i] * qinv[i] * k_inv);
      }
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
  const __bf16* vt = (const __bf16*)p.v;

  stage_rows16(kzl, dp, zb, p.valid, b, C, k0, D);
  const __bf16* ka_row = kzl + lr * dp;  // A rows of the row dots (zero when padded)
  float kinv[4];
  bool kok[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t k = k0 + 4 * lg + i;
    kok[i] = row_valid(p.valid, b, C, k);
    kinv[i] = kok[i] ? inv_norm(ws.nrm, b * C + k, neps) : 0.f;
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
    const float q_inv = q_ok ? inv_norm(ws.nrm, b * C + q, neps) : 0.f;
    f32x4 s4, d4;
    row_dot16x2<true>(ka_row, nullptr, q_ok ? zb + q * D : nullptr, q_in ? dnb + q * D : nullptr, D, lg, s4, d4);
    const float dd = q_in ? ws.dden[b * C + q] : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t k = k0 + 4 * lg + i;
      const bool m = q_in && kok[i] && (!p.causal || k <= q);
      float pv = 0.f, dsv = 0.f;
      if (m) {
        const float vv = vt ? (float)vt[q * C + k] : 1.f;
        pv = s4[i] * kinv[i] * q_inv * vv;
        dsv = (d4[i] + dd) * vv * q_inv;
      }
      pt[(4 * lg + i) * TP + 16 * w + lr] = (__bf16)pv;
      dt[(4 * lg + i) * TP + 16 * w + lr] = (__bf16)dsv;
    }
    __syncthreads();
    rows_acc16<NW, MAXT>(acc1, pt, dntb, qt, D, cp, w, lr, lg);
    rows_acc16<NW, MAXT>(acc2, dt, ztb, qt, D, cp, w, lr, lg);
    __syncthreads();
  }

  const int ntiles = (D + 15) >> 4;
  float rp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    const int tile_i = w + NW * t;
    if (tile_i >= ntiles) break;
    const int col = 16 * tile_i + lr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t k = k0 + 4 * lg + i;
      if (col < D && kok[i]) {
        const float g = acc2[t][i] + ws.dzr[(b * C + k) * D + col];
        acc2[t][i] = g;
        rp[i] += (float)zb[k * D + col] * g;
      }
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
        const float zh = (float)zb[k * D + col] * kinv[i];
        g = acc1[t][i] + (acc2[t][i] - zh * rad[4 * lg + i]) * kinv[i];
      }
      dzb[k * D + col] = (__bf16)g;
    }
  }
}

template <int NW, int MAXT>
hipError_t launch_bwd16_t(const BwdParams& p, hipStream_t s) {
  Ws ws = carve(p.work, p.B, p.C, p.D, p.dv != nullptr, p.dbias != nullptr, true);
  const int64_t rows = p.B * p.C;
  hipLaunchKernelGGL(bwd_prep_kernel<__bf16>, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, s, p, ws);
  hipLaunchKernelGGL(bwd16_transpose_kernel, dim3((unsigned)(ws.cp / 64), (unsigned)cdiv(p.D, 64), (unsigned)p.B),
                     dim3(256), 0, s, p, ws);
  const dim3 grid((unsigned)(cdiv(p.C, kRows) * p.B));  // 1-D, mapped by tile_of_block
  hipLaunchKernelGGL((bwd16_rows_kernel<NW, MAXT>), grid, dim3(64 * NW), 0, s, p, ws);
  hipLaunchKernelGGL((bwd16_cols_kernel<NW, MAXT>), grid, dim3(64 * NW), 0, s, p, ws);
  if (p.dv || p.dbias) {
    const int64_t n = p.dv ? p.C * p.C : p.D;
    const int64_t blocks = cdiv(n, 256) < 1024 ? cdiv(n, 256) : 1024;
    hipLaunchKernelGGL(bwd_final_kernel<__bf16>, dim3((unsigned)blocks), dim3(256), 0, s, p, ws);
  }
  return hipGetLastError();
}

template <typename T, int MAXT>
hipError_t launch_bwd_t(const BwdParams& p, hipStream_t s) {
  Ws ws = carve(p.work, p.B, p.C, p.D, p.dv != nullptr, p.dbias != nullptr, false);
  const int64_t rows = p.B * p.C;
  hipLaunchKernelGGL(bwd_prep_kernel<T>, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, s, p, ws);
  const dim3 grid((unsigned)(cdiv(p.C, kRows) * p.B));  // 1-D, mapped by tile_of_block
  hipLaunchKernelGGL((bwd_rows_kernel<T, MAXT>), grid, dim3(256), 0, s, p, ws);
  hipLaunchKernelGGL((bwd_cols_kernel<T, MAXT>), grid, dim3(256), 0, s, p, ws);
  if (p.dv || p.dbias) {
    const int64_t n = p.dv ? p.C * p.C : p.D;
    const int64_t blocks = cdiv(n, 256) < 1024 ? cdiv(n, 256) : 1024;
    hipLaunchKernelGGL(bwd_final_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, s, p, ws);
  }
  return hipGetLastError();
}

template <typename T>
hipError_t launch_bwd_d(const BwdParams& p, hipStream_t s) {
  const int64_t tiles = cdiv(p.D, 16);
  if (tiles <= 8) return launch_bwd_t<T, 2>(p, s);
  if (tiles <= 16) return launch_bwd_t<T, 4>(p, s);
  if (tiles <= 32) return launch_bwd_t<T, 8>(p, s);
  return launch_bwd_t<T, 16>(p, s);
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

bool bwd_fast_path(int dtype, int64_t D, const void* z) {
  return dtype == AVEY_DTYPE_BF16 && D % 8 == 0 && ((uintptr_t)z & 15) == 0;
}

int64_t bwd_workspace_floats(int64_t B, int64_t C, int64_t D, bool has_v, bool has_bias, bool fast) {
  return ws_floats(B, C, D, has_v, has_bias, fast);
}

hipError_t launch_bwd(const BwdParams& p, int dtype, hipStream_t s) {
  if (bwd_fast_path(dtype, p.D, p.z)) return launch_bwd16(p, s);
  switch (dtype) {
    case AVEY_DTYPE_BF16: return launch_bwd_d<__bf16>(p, s);
    case AVEY_DTYPE_F16: return launch_bwd_d<_Float16>(p, s);
    case AVEY_DTYPE_F32: return launch_bwd_d<float>(p, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace avey
