// Fused forward contextualizer, 16 query rows per workgroup, split by role.
//
// Eight waves, two per SIMD, in two roles that meet at ONE barrier per key tile:
//
//   S-waves 0-3 (similarity). Wave (p, kb) = (wv >> 1, wv & 1) covers feature
//   slices 2p and 2p+1 (two 32*NK-feature slices) for the 16 keys of half kb of a
//   32-key tile: the partial S^T = Z_keys . Q^T over its 64*NK features on
//   v_mfma_f32_16x16x32 (exact 16-bit products, fp32 sums), and the keys' partial
//   sums of squares. It copies into LDS exactly the key rows it reads (its half of
//   its two slices), so its own reads need only its own copy waits; its query
//   fragments stay in registers. It also issues every other copy: the query rows,
//   the gate rows for the epilogue and the cache-line touches of the gate.
//
//   M-waves 4-7 (mixing). Wave h = wv - 4 serves feature slice h: it sums the two
//   pairs' partials of the previous tile, scales by 1/||q|| 1/||k|| (F.normalize,
//   ops.py:68-69), weights by V (ops.py:70-71), masks causality / key padding with
//   selects (ops.py:72-77), adds to the signed row sums (ops.py:79-80) and rounds P
//   to the 16-bit type in the MFMA operand layout, in its own registers (every
//   M-wave forms the whole 16 x 32 P: no exchange of P through LDS). Then the mixing
//   O^T += Z_keys^T P^T (ops.py:78) of its slice, and the transposed reads
//   (ds_read_b64_tr_b16) of the current tile for the next mixing step.
//
// Interval t (ended by the tile's barrier):
//   S: copy tile t+R-1 into the slot tile t-1 left; A(t) from slot t; publish the
//      partials and key norms of t (double-buffered); wait until tile t+1 landed.
//   M: B(t-1) and C(t-1) from the partials published in interval t-1; V words of
//      tile t; T(t), the transposed operands of tile t (read in the same interval
//      as the S-waves read it, so a slot is free one interval after its tile).
// A copy reaches the M-waves through its S-wave's explicit vmcnt wait before the
// barrier that precedes their reads (the same order the query-split variants use
// between partner waves); the S-waves' waits count copies only.
//
// The S-waves keep about 130 registers, so the twelve similarity operands of a
// tile can be in flight at once; the M-waves hold the accumulators and the
// transposed operands (about 170). Splitting the similarity by (feature pair, key
// half) halves the partials the M-waves read per tile and keeps the double-buffered
// partials inside the LDS next to three 48 KB key slots at 768 features.
//
// Epilogue (M-waves): x 1 / (den + eps) (Avey-B), + bias, activation, x gate, a
// select that zeroes padded rows, one rounding (ops.py:79-91). The gate rows are
// copied by the S-waves into slot 0 after the last tile, while the M-waves finish
// the last mixing step.
//
// EG (the enricher's gate half fused): there are no gate rows to copy. The M-waves
// form z_tl = gact(x W_g^T + b_g) for the block's 16 rows: G^T tile t2 = W_g rows
// (features fw + 16 t2 ..) times the x rows, contracted over the model width on the
// similarity's MFMA, lands in exactly the lanes and registers of oacc[t2], so the
// gate never leaves registers. W_g streams through the free key ring after the last
// key tile: chunk c holds model features 32c .. 32c + 31 of all 128 NK rows (64 bytes
// a row, at most TILE bytes), copied by the S-waves like a key tile and read by the
// M-waves after one barrier per chunk. The S-waves also touch the x rows early.
#pragma once

#include "avey_fused.h"

namespace avey {

namespace {

typedef uint32_t u32x4s __attribute__((ext_vector_type(4)));

// Raw buffer descriptor in scalar registers (gfx9: base, stride 0, num_records,
// data format) over rows [row0, rows) of an array whose rows start `stride` bytes
// apart and hold `row_bytes` bytes; num_records 0 (every access reads 0 / is
// dropped) when row0 >= rows. The same resource rows_rsrc builds.
__device__ __forceinline__ u32x4s rows_desc(const char* base, int row0, int rows, uint32_t stride,
                                            uint32_t row_bytes) {
  const int n = rows - row0;
  const uint64_t a = (uint64_t)(base + (int64_t)row0 * stride);
  const uint32_t bytes = n > 0 ? (uint32_t)(n - 1) * stride + row_bytes : 0u;
  return u32x4s{(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a),
                (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xffffu),
                (uint32_t)__builtin_amdgcn_readfirstlane(bytes), (uint32_t)kRsrcWord3};
}

// Buffer-to-LDS copies issued from inline asm (16 or 4 bytes per lane; lane l's
// bytes land at lds + 16 l / 4 l), which the compiler does not track. Its tracking
// of LDS copies makes an LDS read wait for every copy in flight whenever it cannot
// prove the two apart, and it could not here, so a similarity step waited for the
// refill issued for a later tile. The kernel orders these copies with explicit
// vmcnt waits instead: they retire in issue order with every other vector-memory
// operation, so the compiler's own waits for its loads stay correct (they can only
// retire more than they need).
__device__ __forceinline__ uint32_t lds_addr(const char* lds) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) const char*)lds);
}
__device__ __forceinline__ void copy16(const u32x4s& rs, char* lds, uint32_t off) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" : : "v"(off), "s"(rs), "{m0}"(lds_addr(lds)) : "memory");
}
__device__ __forceinline__ void copy4(const u32x4s& rs, char* lds, uint32_t off) {
  asm volatile("buffer_load_dword %0, %1, 0 offen lds" : : "v"(off), "s"(rs), "{m0}"(lds_addr(lds)) : "memory");
}
// P copies of 1 KB (lane l's 16 bytes to lds + 1024 j + 16 l, j < P) when `real`,
// else P 4-byte copies of the same lanes into `sink` (a word no one reads). One inline
// asm block with one branch: every path through it issues exactly P vector-memory
// operations, so a wait counting them holds whichever way the branch went.
#define AVEY_CP(j) "buffer_load_dwordx4 %[o" #j "], %[rs], 0 offen lds\n\ts_add_u32 m0, m0, 0x400\n\t"
#define AVEY_PD(j) "buffer_load_dword %[o" #j "], %[rs], 0 offen lds\n\t"
#define AVEY_HEAD "s_cmp_eq_u32 %[r], 0\n\ts_cbranch_scc1 1f\n\t"
#define AVEY_MID "s_branch 2f\n1:\n\ts_mov_b32 m0, %[sink]\n\t"
template <int P>
__device__ __forceinline__ void copies_or_pads(uint32_t real, const u32x4s& rs, char* lds, char* sink,
                                               const uint32_t (&o)[P]) {
  uint32_t m0 = lds_addr(lds);
  const uint32_t r = __builtin_amdgcn_readfirstlane(real), sk = lds_addr(sink);
  if constexpr (P == 2) {
    asm volatile(AVEY_HEAD AVEY_CP(0) AVEY_CP(1) AVEY_MID AVEY_PD(0) AVEY_PD(1) "2:"
                 : "+{m0}"(m0)
                 : [o0] "v"(o[0]), [o1] "v"(o[1]), [rs] "s"(rs), [r] "s"(r), [sink] "s"(sk)
                 : "memory", "scc");
  } else if constexpr (P == 4) {
    asm volatile(AVEY_HEAD AVEY_CP(0) AVEY_CP(1) AVEY_CP(2) AVEY_CP(3) AVEY_MID AVEY_PD(0) AVEY_PD(1) AVEY_PD(2)
                     AVEY_PD(3) "2:"
                 : "+{m0}"(m0)
                 : [o0] "v"(o[0]), [o1] "v"(o[1]), [o2] "v"(o[2]), [o3] "v"(o[3]), [rs] "s"(rs), [r] "s"(r),
                   [sink] "s"(sk)
                 : "memory", "scc");
  } else if constexpr (P == 6) {
    asm volatile(AVEY_HEAD AVEY_CP(0) AVEY_CP(1) AVEY_CP(2) AVEY_CP(3) AVEY_CP(4) AVEY_CP(5) AVEY_MID AVEY_PD(0)
                     AVEY_PD(1) AVEY_PD(2) AVEY_PD(3) AVEY_PD(4) AVEY_PD(5) "2:"
                 : "+{m0}"(m0)
                 : [o0] "v"(o[0]), [o1] "v"(o[1]), [o2] "v"(o[2]), [o3] "v"(o[3]), [o4] "v"(o[4]), [o5] "v"(o[5]),
                   [rs] "s"(rs), [r] "s"(r), [sink] "s"(sk)
                 : "memory", "scc");
  } else {
    static_assert(P == 8, "copies per slice");
    asm volatile(AVEY_HEAD AVEY_CP(0) AVEY_CP(1) AVEY_CP(2) AVEY_CP(3) AVEY_CP(4) AVEY_CP(5) AVEY_CP(6) AVEY_CP(7)
                     AVEY_MID AVEY_PD(0) AVEY_PD(1) AVEY_PD(2) AVEY_PD(3) AVEY_PD(4) AVEY_PD(5) AVEY_PD(6)
                         AVEY_PD(7) "2:"
                 : "+{m0}"(m0)
                 : [o0] "v"(o[0]), [o1] "v"(o[1]), [o2] "v"(o[2]), [o3] "v"(o[3]), [o4] "v"(o[4]), [o5] "v"(o[5]),
                   [o6] "v"(o[6]), [o7] "v"(o[7]), [rs] "s"(rs), [r] "s"(r), [sink] "s"(sk)
                 : "memory", "scc");
  }
}
#undef AVEY_CP
#undef AVEY_PD
#undef AVEY_HEAD
#undef AVEY_MID

// LDS geometry of the 16-row role-split kernel for slices of 32*NK features.
template <int NK>
struct G16 {
  typedef Geo<16, NK> Gm;
  static constexpr int DS = Gm::DS, NT = Gm::NT, CPR = Gm::CPR, CPRP = Gm::CPRP, G = Gm::G;
  static constexpr int SLICE = Gm::SLICE, TILE = Gm::TILE, P = Gm::P, RPP = Gm::RPP;
  static constexpr int KDW = 2 * P;  // copies per S-wave per key tile (16 rows x 2 slices)
  // Partials of a tile: [pair][kb][lane] f32x4 (S^T of 16 keys x 16 queries).
  static constexpr int SXB = 2 * 2 * 64 * 16;
  static constexpr int SMALL = 2 * SXB + 2 * 2 * 32 * 4 + 2 * 16 * 4 + 32 * 4 + 256;
  static constexpr int kLdsMax = 160 * 1024;
  static constexpr int R = 3 * TILE + SMALL <= kLdsMax ? 3 : 2;
  static_assert(2 * TILE + SMALL <= kLdsMax, "tile does not fit the LDS");
};

template <int NK>
struct Small16 {
  f32x4 sx[2][2][2][64];  // [buffer][pair][kb][lane]: partial S^T of a tile
  float nxp[2][2][32];    // [buffer][pair][key]: partial sums of squares; -1: out of range
  float nq[2][16];        // [pair][row]: partial sums of squares of the queries; -1: out of range
  f32x4 rk[8];            // 1 / max(||k||, norm_eps) of the M-waves' current tile; 0: left out
};

}  // namespace

template <typename T16, int NK, bool FULL, bool STRIDED, bool HILO, bool EG>
__global__ __launch_bounds__(512, 1) void fused16_kernel(FwdParams p) {
  typedef G16<NK> Gx;
  constexpr int DS = Gx::DS, NT = Gx::NT, CPR = Gx::CPR, CPRP = Gx::CPRP, G = Gx::G;
  constexpr int SLICE = Gx::SLICE, TILE = Gx::TILE, R = Gx::R, P = Gx::P, RPP = Gx::RPP, KDW = Gx::KDW;
  __shared__ __attribute__((aligned(16))) char slot0[TILE];
  __shared__ __attribute__((aligned(16))) char slot1[TILE];
  __shared__ __attribute__((aligned(16))) char slot2[R == 3 ? TILE : 16];
  __shared__ Small16<NK> sm;
  __shared__ __attribute__((aligned(16))) char touch_sink[256];
  static_assert(sizeof(Small16<NK>) + 256 <= Gx::SMALL, "small LDS arrays");

  const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int li = lane & 15, lg = lane >> 4;
  const bool swave = wv < 4;
  const int pr = (wv >> 1) & 1, kbs = wv & 1;  // S-wave: feature pair and key half
  const int h = wv & 3;                         // M-wave: feature slice
  const int C = (int)p.C, D = (int)p.D, B = (int)p.B;
  const int n_qt = (C + 15) / 16;
  int b, qt;
  block_item((int)blockIdx.x, B, n_qt, p.causal != 0, b, qt);
  const int q0 = qt * 16;
  const uint32_t row_bytes = (uint32_t)D * 2u;
  const uint32_t zstride = STRIDED ? (uint32_t)p.zrs * 2u : row_bytes;
  const uint32_t gstride = STRIDED ? (uint32_t)p.grs * 2u : row_bytes;
  const char* zb = (const char*)p.z + (STRIDED ? (int64_t)b * p.zbs * 2 : (int64_t)b * C * row_bytes);
  const bool has_valid = p.valid != nullptr, has_v = p.v != nullptr;
  const bool has_gate = p.gate != nullptr, has_bias = p.bias != nullptr;
  const char* gb = has_gate ? (const char*)p.gate + (STRIDED ? (int64_t)b * p.gbs * 2 : (int64_t)b * C * row_bytes)
                             : (const char*)p.z;
  const char* vb = has_valid ? (const char*)p.valid + (int64_t)b * C : (const char*)p.z;
  const int valid_rows = has_valid ? C : 0;
  const uint32_t or_valid = has_valid ? 0u : 1u;
  const uint32_t or_v = has_v ? 0u : Ops<T16>::kOne;
  const bool causal = p.causal != 0;
  const float norm_eps = (float)p.norm_eps;
  const float eps2 = norm_eps * norm_eps;
  const float inv_eps = 1.f / norm_eps;
  const int nkt = (int)key_tiles_for(qt, C, 16, kBN, causal);

  auto slot_ptr = [&](auto slot) -> char* {
    constexpr int I = decltype(slot)::value;
    return I == 0 ? slot0 : (I == 1 ? slot1 : slot2);
  };
  // Global byte offset of slice position pos (row pos / CPRP, chunk swizzle(row, ...))
  // of feature slice `sl`, rows `stride` bytes apart; kNowhere past the slice or D.
  auto goff = [&](int sl, int pos, uint32_t stride) -> uint32_t {
    const int r = pos / CPRP, c = swzc<G>(r, pos % CPRP);
    const int col = sl * DS + 8 * c;
    return (c < CPR && (FULL || col < D)) ? (uint32_t)r * stride + (uint32_t)col * 2u : kNowhere;
  };

  if (swave) {
    // =============================== S-waves ========================================
    const int sl0 = 2 * pr;  // slices sl0, sl0 + 1
    // Lane offsets of the copies of 16 rows of each of the two slices (they repeat
    // every P copies, 16 rows); the rows go into the resource base.
    uint32_t kof[2][P];
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int j = 0; j < P; ++j) kof[e][j] = goff(sl0 + e, 64 * j + lane, zstride);
    uint32_t a1[G / 4];
#pragma unroll
    for (int m = 0; m < G / 4; ++m) a1[m] = 16u * (uint32_t)(li * CPRP + swzc<G>(li, 4 * m + lg));
    auto frag = [&](const char* slice_base, int row16, int s) -> u32x4 {
      return *reinterpret_cast<const u32x4*>(slice_base + a1[s % (G / 4)] + 16 * (16 * row16 * CPRP + G * (s / (G / 4))));
    };
    // Key tile t, rows 16 kbs .. 16 kbs + 15 of both slices, into ring slot I.
    // Tiles at or past nkt (the causal limit, or past the context) are copies of nothing:
    // 4-byte loads through an empty resource into the never-read word, one per copy a
    // tile would take.
    auto copy_tile = [&](int t, auto slot) {
      char* base = slot_ptr(slot);
      const u32x4s r = rows_desc(zb, t * kBN + 16 * kbs, t < nkt ? C : 0, zstride, row_bytes);
      const uint32_t real = t < nkt ? 1u : 0u;
#pragma unroll
      for (int e = 0; e < 2; ++e) copies_or_pads<P>(real, r, base + (sl0 + e) * SLICE + 1024 * kbs * P, touch_sink, kof[e]);
    };
    static_assert(KDW + 2 < 64, "vmcnt holds 6 bits");
    // All but the newest N vector-memory operations retired (they return in order).
    auto wait_keep = [&](auto n) {
      constexpr int N = decltype(n)::value;
      __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
    };
    // The gate rows reach the L2 ahead of the epilogue's copy (one 4-byte touch per
    // 128-byte line into a never-read word). When the whole grid's gate fits the L2s
    // with room to spare, the touches wait until a few tiles of the loop have been
    // issued, so that they do not compete with the prologue's loads, which every
    // workgroup issues at once (C2: touching in the prologue 13.29 us per call,
    // interval 1 13.28, interval 3 for workgroups of more than 4 key tiles and 1 for 3-4
    // tiles 12.53, on one box); light workgroups still touch at the start. Larger grids
    // touch three key tiles before the tail.
    constexpr int kTouchLead = 3;
    const bool gate_fits = (uint64_t)B * (uint64_t)C * row_bytes <= (8ull << 20);
    const int touch_t = gate_fits ? (nkt > 4 ? 3 : (nkt > 2 ? 1 : 0)) : nkt - kTouchLead;
    auto touch_gate = [&]() {
      const u32x4s r = rows_desc(gb, q0, min(C, q0 + 16), gstride, row_bytes);
      constexpr int kLines = 4 * 32 * NK * 2 / 128;
      constexpr int kTouches = (16 * kLines + 255) / 256;
#pragma unroll
      for (int i = 0; i < kTouches; ++i) {
        const uint32_t line = (uint32_t)(i * 256 + tid), c = line % kLines;
        copy4(r, touch_sink, c * 128u < row_bytes ? (line / kLines) * gstride + c * 128u : kNowhere);
      }
    };

    // EG: the block's x rows reach the L2 while the key loop runs (one 4-byte touch per
    // 128-byte line into the never-read word; rows past 4096 features in part).
    auto touch_x = [&]() {
      const uint32_t xrb = (uint32_t)p.dm * 2u, lines = (xrb + 127u) / 128u;
      const u32x4s r = rows_desc((const char*)p.xg + (int64_t)b * C * xrb, q0, min(C, q0 + 16), xrb, xrb);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t line = (uint32_t)(i * 256 + tid);
        copy4(r, touch_sink, line < 16u * lines ? (line / lines) * xrb + (line % lines) * 128u : kNowhere);
      }
    };

    // ---- prologue: the 16 query rows into slot R-1 (the two waves of a pair split
    // the P copies of each of their slices, even / odd), key tiles 0 .. R-2 ----------
    {
      char* qbase = slot_ptr(IC<R - 1>{});
      const u32x4s r = rows_desc(zb, q0, C, zstride, row_bytes);
#pragma unroll
      for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int j = kbs; j < P; j += 2) copy16(r, qbase + (sl0 + e) * SLICE + 1024 * j, kof[e][j]);
    }
    // Order: tile 0 and the gate touches, then tile 1, so that waiting for everything
    // but tile 1's copies is one count.
    copy_tile(0, IC<0>{});
    if (has_gate && touch_t < 1) touch_gate();
    if constexpr (EG) touch_x();
    if constexpr (R == 3) {
      // Without a tile 1, copies of nothing stand in for it (copy_tile), so that one
      // wait count holds on every path.
      copy_tile(1, IC<1>{});
      wait_keep(IC<KDW>{});  // the query rows and tile 0 landed; tile 1 may stay in flight
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F70);
    }
    lds_barrier();  // P0: query rows and tile 0 visible to every wave
    // Query fragments of both slices; partial norms (pair p: both key halves compute
    // them, the kb = 0 wave publishes).
    u32x4 qf[2 * NK];
    {
      const char* qbase = slot_ptr(IC<R - 1>{});
      // Rows past the context read as zeros and are marked -1. Padded rows (valid ==
      // False, possibly NaN) go through: their similarities and norms are selected
      // away by the M-waves.
      const bool ok = li < C - q0;
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int s = 0; s < NK; ++s) {
          const u32x4 x = frag(qbase + (sl0 + e) * SLICE, 0, s);
          qf[e * NK + s] = x;
          ss = Ops<T16>::sumsq(qf[e * NK + s], ss);
        }
      ss = sum_over_groups(ss);
      if (kbs == 0 && lg == 0) sm.nq[pr][li] = ok ? ss : -1.f;
    }
    lds_barrier();  // P1: the query rows are consumed (slot R-1 may be refilled)

    // ---- A(t): partial S^T of this wave's 16 keys from slot I ---------------------
    auto stage_a = [&](int t, auto slot) {
      const int k0 = t * kBN;
      const char* base = slot_ptr(slot);
      f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
      float ss = 0.f;
      u32x4 a[2 * NK];
#pragma unroll
      for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int s = 0; s < NK; ++s) a[e * NK + s] = frag(base + (sl0 + e) * SLICE, kbs, s);
#pragma unroll
      for (int m = 0; m < 2 * NK; ++m) {
        sacc = Ops<T16>::mfma32(a[m], qf[m], sacc);
        ss = Ops<T16>::sumsq(a[m], ss);
      }
      ss = sum_over_groups(ss);
      const bool ok = 16 * kbs + li < C - k0;  // keys past the context read as zeros; -1 marks them
      const int buf = t & 1;
      sm.sx[buf][pr][kbs][lane] = sacc;
      if (lg == 0) sm.nxp[buf][pr][16 * kbs + li] = ok ? ss : -1.f;
    };
    // Interval t: refill, A(t), wait for tile t+1, barrier. Unrolled by R so that
    // every slot index is a constant.
    auto interval = [&](int t, auto cur) {
      constexpr int I = decltype(cur)::value, F = (I + R - 1) % R;
      if (has_gate && touch_t >= 1 && t == touch_t) touch_gate();
      // The refill goes into the slot tile t-1 left (every wave's reads of it ended
      // at the previous barrier). Once no tile is left, copies of nothing take its
      // place, so that every interval issues the same count and one wait holds on every
      // path. Nothing else of this wave goes to memory in the loop, so the wait below
      // counts these copies exactly.
      copy_tile(t + R - 1, IC<F>{});
      stage_a(t, cur);
      // Tile t+1 must have landed before the barrier after which the M-waves read it;
      // the refill just issued (R = 3) may stay in flight.
      if constexpr (R == 3)
        wait_keep(IC<KDW>{});
      else
        __builtin_amdgcn_s_waitcnt(0x0F70);
      lds_barrier();
    };
    {
      int t = 0;
      if constexpr (R == 2) {
        for (; t + 1 < nkt; t += 2) {
          interval(t, IC<0>{});
          interval(t + 1, IC<1>{});
        }
        if (t < nkt) interval(t, IC<0>{});
      } else {
        for (; t + 2 < nkt; t += 3) {
          interval(t, IC<0>{});
          interval(t + 1, IC<1>{});
          interval(t + 2, IC<2>{});
        }
        if (t < nkt) interval(t, IC<0>{});
        if (t + 1 < nkt) interval(t + 1, IC<1>{});
      }
    }
    if constexpr (EG) {
      // ---- tail: W_g chunk by chunk through the ring (every slot is free). Chunk c
      // goes to slot c % R; S-wave wv copies rows 32 NK wv .. + 32 NK - 1 (16 rows per
      // 1 KB copy: lane l, row l / 4, bytes 16 (l % 4) of the row's 64). A chunk past
      // the last is copies of nothing, so every step issues the same count.
      constexpr int CW = 2 * NK, CH = CW <= 8 ? 1 : 2, CP = CW / CH;
      const uint32_t xrb = (uint32_t)p.dm * 2u;
      const int ks = (int)((p.dm + 31) / 32);
      const u32x4s rw = rows_desc((const char*)p.wg, 0, D, xrb, xrb);
      auto slot_rt = [&](int c) -> char* {
        const int i = c % R;
        return i == 0 ? slot0 : (i == 1 ? slot1 : slot2);
      };
      auto copy_chunk = [&](int c) {
        const uint32_t real = c < ks ? 1u : 0u;
        const uint32_t kb = 64u * (uint32_t)c + 16u * (uint32_t)(lane & 3);
        char* dst = slot_rt(c) + 1024 * wv * CW;
#pragma unroll
        for (int hh = 0; hh < CH; ++hh) {
          uint32_t o[CP];
#pragma unroll
          for (int i = 0; i < CP; ++i) {
            const uint32_t row = (uint32_t)(16 * (wv * CW + hh * CP + i) + (lane >> 2));
            o[i] = kb < xrb ? row * xrb + kb : kNowhere;
          }
          copies_or_pads<CP>(real, rw, dst + 1024 * CP * hh, touch_sink, o);
        }
      };
      // Chunk c must have landed by barrier c; with three slots chunk c + 1 may still be
      // in flight there (its slot held chunk c - 2, read before barrier c - 1).
      auto wait_chunk = [&]() {
        if constexpr (R == 3)
          wait_keep(IC<CW>{});
        else
          __builtin_amdgcn_s_waitcnt(0x0F70);
      };
      copy_chunk(0);
      if constexpr (R == 3) copy_chunk(1);
      wait_chunk();
      lds_barrier();  // chunk 0 (E)
      for (int c = 1; c < ks; ++c) {
        copy_chunk(R == 3 ? c + 1 : c);
        wait_chunk();
        lds_barrier();  // chunk c
      }
      __builtin_amdgcn_s_waitcnt(0x0F70);
      lds_barrier();  // the M-waves' reads of the last chunk ended (they reuse slot 0)
      return;
    }
    // ---- tail: the gate rows of slice 2p + kbs into slot 0 (every slot is free)
    if (has_gate) {
      const int sl = sl0 + kbs;
      const u32x4s r = rows_desc(gb, q0, C, gstride, row_bytes);
#pragma unroll
      for (int j = 0; j < P; ++j) copy16(r, slot0 + sl * SLICE + 1024 * j, goff(sl, 64 * j + lane, gstride));
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);
    lds_barrier();  // E: the gate rows are visible to the M-waves
    return;
  }

  // ================================= M-waves =========================================
  // Transposed mixing operands: row 4 lg + li / 4, chunk 2 t + (li & 3) / 2, half li & 1.
  uint32_t a2[G / 2];
  {
    const int r0 = 4 * lg + (li >> 2);
#pragma unroll
    for (int m = 0; m < G / 2; ++m)
      a2[m] = 16u * (uint32_t)(r0 * CPRP + swzc<G>(r0, 2 * m + ((li & 3) >> 1))) + 8u * (uint32_t)(li & 1);
  }
  u32x4 ztr[NT];
  auto stage_t = [&](auto slot) {
    const char* base = slot_ptr(slot) + h * SLICE;
#pragma unroll
    for (int t2 = 0; t2 < NT; ++t2) {
      const uint32_t o = a2[t2 % (G / 2)] + 16u * (uint32_t)(G * (t2 / (G / 2)));
      const u32x2 lo = __builtin_bit_cast(u32x2, lds_read_tr((const uint16_t*)(base + o)));
      const u32x2 hi = __builtin_bit_cast(u32x2, lds_read_tr((const uint16_t*)(base + o + 16 * 16 * CPRP)));
      ztr[t2] = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
  };
  // key - query for the lane's keys 16 kb + 4 lg + i of a tile, i = 0..3, is
  // ud[kb] + i - (q0 - k0); V[q0 + li][k0 + 16 kb + 4 lg + i] starts at voff[kb].
  float ud[2];
  uint32_t voff[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    ud[kb] = (float)(16 * kb + 4 * lg - li);
    voff[kb] = ((uint32_t)(q0 + li) * (uint32_t)C + (uint32_t)(16 * kb + 4 * lg)) * 2u;
  }
  const uint32_t vbytes = has_v ? (uint32_t)C * (uint32_t)C * 2u : 0u;
  // Padding: the validity bytes of the lane's query row and of key lane & 31 of a tile.
  // Padded rows reach the products as they are (possibly NaN) and are selected away
  // here: P is a bitwise select (an exact +0), and padded keys are cleared in the
  // transposed operands.
  const uint32_t qvalid = ld8(rows_rsrc(vb, q0, valid_rows, 1u, 1u), (uint32_t)li);
  const bool qok = (qvalid | or_valid) != 0u;
  uint32_t kvb = 1u;  // validity byte of key lane & 31 of the next tile (used an interval later)
  auto load_kvalid = [&](int k0) {
    if (has_valid) kvb = ld8(rows_rsrc(vb, k0, valid_rows, 1u, 1u), (uint32_t)(lane & 31));
  };
  u32x2 vv[2];
  auto load_v = [&](int k0) {
    const uint32_t skip = (uint32_t)k0 * 2u;
    const rsrc_t r = make_rsrc((const char*)(has_v ? p.v : p.z) + skip, vbytes > skip ? vbytes - skip : 0u);
    if ((C & 1) == 0) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) vv[kb] = ld64(r, voff[kb]);
    } else {
      // Odd context: a row may start mid-dword and V's last dword is half past its end.
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
        vv[kb] = u32x2{ld16(r, voff[kb]) | (ld16(r, voff[kb] + 2u) << 16),
                       ld16(r, voff[kb] + 4u) | (ld16(r, voff[kb] + 6u) << 16)};
    }
  };
  f32x4 oacc[NT];
#pragma unroll
  for (int t2 = 0; t2 < NT; ++t2) oacc[t2] = f32x4{0.f, 0.f, 0.f, 0.f};
  float den = 0.f;
  float rq = 0.f;
  // ---- B(t) and C(t): P of tile t in registers, then the mixing product ------------
  // P = S^T * (1/||k|| 1/||q||) * V, the causal and padding masks as bitwise selects.
  // Lane l finds 1/||k|| of key l & 31 (0 for padded or out-of-range keys) and
  // publishes it; each lane reads back its eight keys. `diag`: the tile holds keys
  // past some of the block's queries (causal only), so the causal compare runs.
  auto form_p = [&](const f32x4 (&sv)[2], const f32x4 (&rk4)[2], float lim, auto diag, uint32_t (&ph)[4],
                    uint32_t (&pl)[4]) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      float pv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float rkq = rk4[kb][i] * rq;
        bool ok = rkq > 0.f;  // false for padded / out-of-range keys and padded queries (NaN-safe)
        if constexpr (decltype(diag)::value) ok = ok && (ud[kb] + (float)i <= lim);
        const uint32_t vw = vv[kb][i >> 1];
        const float x = sv[kb][i] * rkq * Ops<T16>::to_f_or((i & 1) ? vw >> 16 : vw & 0xffffu, or_v);
        pv[i] = __uint_as_float(__float_as_uint(x) & (ok ? 0xffffffffu : 0u));
        den += pv[i];
      }
      ph[2 * kb] = pack2<T16>(pv[0], pv[1]);
      ph[2 * kb + 1] = pack2<T16>(pv[2], pv[3]);
      if constexpr (HILO) {
        pl[2 * kb] = pack2<T16>(pv[0] - Ops<T16>::to_f(ph[2 * kb] & 0xffffu), pv[1] - Ops<T16>::hi_f(ph[2 * kb]));
        pl[2 * kb + 1] =
            pack2<T16>(pv[2] - Ops<T16>::to_f(ph[2 * kb + 1] & 0xffffu), pv[3] - Ops<T16>::hi_f(ph[2 * kb + 1]));
      }
    }
  };
  auto stage_bc = [&](int t) {
    const int k0 = t * kBN;
    const int buf = t & 1;
    {
      const int k = lane & 31;
      const float n = sm.nxp[buf][0][k] + sm.nxp[buf][1][k];
      const bool kok = (kvb | or_valid) != 0u;
      const float r = (n < 0.f || !kok) ? 0.f : (n > eps2 ? __builtin_amdgcn_rsqf(n) : inv_eps);
      if (lane < 32) reinterpret_cast<float*>(sm.rk)[k] = r;
    }
    f32x4 sv[2], rk4[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      sv[kb] = sm.sx[buf][0][kb][lane] + sm.sx[buf][1][kb][lane];
      rk4[kb] = sm.rk[4 * kb + lg];
    }
    uint32_t ph[4], pl[4];
    if (causal && k0 + kBN - 1 > q0)
      form_p(sv, rk4, (float)(q0 - k0), std::true_type{}, ph, pl);
    else
      form_p(sv, rk4, 0.f, std::false_type{}, ph, pl);
    if (has_valid) {
      // Word w of a transposed operand holds keys 16 (w / 2) + 4 lg + 2 (w % 2) + {0, 1}.
      u32x4 km;
#pragma unroll
      for (int w2 = 0; w2 < 4; ++w2)
        km[w2] = (rk4[w2 >> 1][2 * (w2 & 1)] > 0.f ? 0x0000ffffu : 0u) |
                 (rk4[w2 >> 1][2 * (w2 & 1) + 1] > 0.f ? 0xffff0000u : 0u);
#pragma unroll
      for (int t2 = 0; t2 < NT; ++t2) ztr[t2] &= km;
    }
    const u32x4 pf = u32x4{ph[0], ph[1], ph[2], ph[3]};
#pragma unroll
    for (int t2 = 0; t2 < NT; ++t2) oacc[t2] = Ops<T16>::mfma32(ztr[t2], pf, oacc[t2]);
    if constexpr (HILO) {
      const u32x4 pfl = u32x4{pl[0], pl[1], pl[2], pl[3]};
#pragma unroll
      for (int t2 = 0; t2 < NT; ++t2) oacc[t2] = Ops<T16>::mfma32(ztr[t2], pfl, oacc[t2]);
    }
  };

  lds_barrier();  // P0: query rows and tile 0 landed
  load_v(0);
  load_kvalid(0);
  lds_barrier();  // P1: query norms published
  {
    // Two partials (-1 each for padded / out-of-range rows); F.normalize divides by
    // max(||q||, norm_eps); 0 marks the rows that are left out.
    const float ss = sm.nq[0][li] + sm.nq[1][li];
    rq = (ss < 0.f || !qok) ? 0.f : (ss > eps2 ? __builtin_amdgcn_rsqf(ss) : inv_eps);
  }
  auto m_interval = [&](int t, auto cur) {
    if (t > 0) {
      stage_bc(t - 1);
      // V and validity of tile t for B(t) in the next interval (B(t-1) consumed the
      // previous ones).
      load_v(t * kBN);
      load_kvalid(t * kBN);
    }
    __builtin_amdgcn_sched_barrier(0);
    stage_t(cur);
    lds_barrier();
  };
  {
    int t = 0;
    if constexpr (R == 2) {
      for (; t + 1 < nkt; t += 2) {
        m_interval(t, IC<0>{});
        m_interval(t + 1, IC<1>{});
      }
      if (t < nkt) m_interval(t, IC<0>{});
    } else {
      for (; t + 2 < nkt; t += 3) {
        m_interval(t, IC<0>{});
        m_interval(t + 1, IC<1>{});
        m_interval(t + 2, IC<2>{});
      }
      if (t < nkt) m_interval(t, IC<0>{});
      if (t + 1 < nkt) m_interval(t + 1, IC<1>{});
    }
  }
  // ---- tail: bias words and the row's validity byte, the last tile's B and C ------
  const int fw = h * DS;
  u32x2 bw[NT];
  {
    const rsrc_t rbias = make_rsrc(has_bias ? p.bias : p.z, has_bias ? row_bytes : 0u);
#pragma unroll
    for (int t2 = 0; t2 < NT; ++t2) {
      const int f = fw + 16 * t2 + 4 * lg;
      bw[t2] = ld64(rbias, (FULL || f < D) ? (uint32_t)f * 2u : kNowhere);
    }
  }
  stage_bc(nkt - 1);
  if constexpr (!EG) lds_barrier();  // E: gate rows copied by the S-waves (EG: the chunk barriers)
  const float dtot = sum_over_groups(den);
  const float rden = p.normalize ? 1.f / (dtot + (float)p.eps) : 1.f;  // signed sum + eps, no clamp
  // ---- epilogue: lane holds query li, features fw + 16 t2 + 4 lg .. +3 --------------
  uint32_t a3[G / 2];
#pragma unroll
  for (int m = 0; m < G / 2; ++m)
    a3[m] = 16u * (uint32_t)(li * CPRP + swzc<G>(li, 2 * m + (lg >> 1))) + 8u * (uint32_t)(lg & 1);
  char* const ebase = slot0 + h * SLICE;
  auto efrag = [&](int t2) -> char* { return ebase + a3[t2 % (G / 2)] + 16 * G * (t2 / (G / 2)); };
  const uint32_t one2 = Ops<T16>::kOne | (Ops<T16>::kOne << 16);
  constexpr int GB = NT <= 12 ? NT : 8;
  // Own loads (bias, validity) retired; the gate rows were waited for by their S-wave.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // EG: G^T = W_g x^T of this wave's slice, chunk by chunk (32 model features) as
  // the S-waves publish them; the x fragment of the next chunk loads meanwhile. Then
  // z_tl = gact(G + b_g), in place.
  f32x4 gacc[EG ? NT : 1];
  if constexpr (EG) {
    const uint32_t xrb = (uint32_t)p.dm * 2u;
    const rsrc_t rx = rows_rsrc((const char*)p.xg + (int64_t)b * C * xrb, q0, C, xrb, xrb);
    const int ks = (int)((p.dm + 31) / 32);
    auto xoff = [&](int c) -> uint32_t {
      const uint32_t kb = 64u * (uint32_t)c + 16u * (uint32_t)lg;
      return kb < xrb ? (uint32_t)li * xrb + kb : kNowhere;
    };
#pragma unroll
    for (int t2 = 0; t2 < NT; ++t2) gacc[t2] = f32x4{0.f, 0.f, 0.f, 0.f};
    u32x4 xf = ld128(rx, xoff(0));
    const uint32_t wrow = (uint32_t)(fw + li) * 64u + 16u * (uint32_t)lg;
    for (int c = 0; c < ks; ++c) {
      lds_barrier();  // chunk c landed (c = 0: also E)
      const u32x4 xn = ld128(rx, xoff(c + 1 < ks ? c + 1 : c));
      const int si = c % R;
      const char* base = (si == 0 ? slot0 : (si == 1 ? slot1 : slot2)) + wrow;
#pragma unroll
      for (int t2 = 0; t2 < NT; ++t2)
        gacc[t2] = Ops<T16>::mfma32(*reinterpret_cast<const u32x4*>(base + 1024 * t2), xf, gacc[t2]);
      xf = xn;
    }
    // The output staging below writes slot 0 in slices laid out apart from the chunk
    // rows: every wave's chunk reads end first.
    lds_barrier();
    const rsrc_t rbg = make_rsrc(p.bg ? p.bg : p.z, p.bg ? row_bytes : 0u);
#pragma unroll
    for (int t2 = 0; t2 < NT; ++t2) {
      const int f = fw + 16 * t2 + 4 * lg;
      const u32x2 bgw = ld64(rbg, (FULL || f < D) ? (uint32_t)f * 2u : kNowhere);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t w = bgw[k >> 1];
        gacc[t2][k] = activate<float>(gacc[t2][k] + ((k & 1) ? Ops<T16>::hi_f(w) : Ops<T16>::to_f(w & 0xffffu)),
                                      p.gact);
      }
    }
  }
  auto finish = [&](auto act_tag) {
    constexpr int ACT = decltype(act_tag)::value;
#pragma unroll
    for (int tb = 0; tb < NT; tb += GB) {
      u32x2 gw[GB];
      if constexpr (!EG) {
#pragma unroll
        for (int i = 0; i < GB; ++i) gw[i] = *reinterpret_cast<const u32x2*>(efrag(tb + i));
        if (!has_gate) {
#pragma unroll
          for (int i = 0; i < GB; ++i) gw[i] = u32x2{one2, one2};
        }
      }
#pragma unroll
      for (int i = 0; i < GB; ++i) {
        const int t2 = tb + i;
        float y[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t bword = bw[t2][k >> 1], gword = EG ? 0u : gw[i][k >> 1];
          float x = oacc[t2][k] * rden;
          x += (k & 1) ? Ops<T16>::hi_f(bword) : Ops<T16>::to_f(bword & 0xffffu);
          x = activate<float>(x, ACT);
          if constexpr (EG)
            x *= gacc[t2][k];
          else
            x *= (k & 1) ? Ops<T16>::hi_f(gword) : Ops<T16>::to_f(gword & 0xffffu);
          y[k] = qok ? x : 0.f;
        }
        *reinterpret_cast<u32x2*>(efrag(t2)) = u32x2{pack2<T16>(y[0], y[1]), pack2<T16>(y[2], y[3])};
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
  // The rows of slice h leave in 16-byte row-contiguous stores; rows past the context
  // fall outside the resource and are dropped.
  const char* ob = (const char*)p.out + (int64_t)b * C * row_bytes;
  const rsrc_t ro = rows_rsrc(ob, q0, C, row_bytes, row_bytes);
#pragma unroll
  for (int j = 0; j < P; ++j) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(ebase + 1024 * j + 16 * lane);
    st128(v, ro, goff(h, 64 * j + lane, row_bytes));
  }
}

template <typename T16, int NK, bool STRIDED, bool EG>
hipError_t launch_fused16_one(const FwdParams& p, int64_t grid, hipStream_t s) {
  const dim3 g((unsigned)grid), t(512);
  const bool full = p.D == 4 * 32 * NK;
  if (p.normalize != 0) {
    if (full)
      fused16_kernel<T16, NK, true, STRIDED, true, EG><<<g, t, 0, s>>>(p);
    else
      fused16_kernel<T16, NK, false, STRIDED, true, EG><<<g, t, 0, s>>>(p);
  } else {
    if (full)
      fused16_kernel<T16, NK, true, STRIDED, false, EG><<<g, t, 0, s>>>(p);
    else
      fused16_kernel<T16, NK, false, STRIDED, false, EG><<<g, t, 0, s>>>(p);
  }
  return hipGetLastError();
}

// EG: the enricher gate formed in the epilogue (avey_fwd_enriched); compiled apart
// from the plain variants (avey_fused_bm16_*_eg.hip).
template <typename T16, bool STRIDED, bool EG = false>
hipError_t launch_fused16(const FwdParams& p, int nk, int64_t grid, hipStream_t s) {
  switch (nk) {
    case 1: return launch_fused16_one<T16, 1, STRIDED, EG>(p, grid, s);
    case 2: return launch_fused16_one<T16, 2, STRIDED, EG>(p, grid, s);
    case 3: return launch_fused16_one<T16, 3, STRIDED, EG>(p, grid, s);
    case 4: return launch_fused16_one<T16, 4, STRIDED, EG>(p, grid, s);
    case 6: return launch_fused16_one<T16, 6, STRIDED, EG>(p, grid, s);
    case 8: return launch_fused16_one<T16, 8, STRIDED, EG>(p, grid, s);
    default: return hipErrorInvalidConfiguration;
  }
}

}  // namespace avey
