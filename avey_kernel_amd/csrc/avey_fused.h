// Fused forward contextualizer for bf16 / fp16 on gfx950 MFMA.
//
// One workgroup owns BM query rows of one batch item and streams key tiles of
// BN = 32 rows over them. The feature axis is split four ways: feature slice w,
// [w*DS, (w+1)*DS), is served by wave w for every product (by two waves in the
// 8-wave variants below). Per key tile t there are three stages:
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
// partials; the key tiles sit in a ring of 2 or 3 LDS slots, refilled by
// buffer-to-LDS copies a tile or two ahead.
//
// Waves per workgroup (fused_threads in avey_common.h; 16-row blocks run the
// role-split kernel of avey_fused16.h instead):
//   * 32-row variants and 64-row ones up to 128 features per slice, 8 waves ("query
//     split"): waves w and w+4 serve slice w, each for half of the query blocks, so
//     each holds half the accumulators. Each copies half of a key tile's rows and
//     orders them for its partner by an explicit wait before the iteration's last
//     barrier.
//   * 64-row variants with 192 features per slice, 4 waves of 512 registers (their
//     state does not fit 256).
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
// mode (the diagonal tile is kept and masked elementwise). The block order
// (block_item in avey_common.h) puts all query tiles of one batch item on the same
// XCD whenever the batch is a multiple of 8 (its L2 then serves the repeated key
// reads): heaviest query tile first in causal mode, and the tiles of an item
// dispatched together otherwise.
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

// Resource over rows [row0, rows) of an array whose rows start `stride` bytes apart
// and hold `row_bytes` bytes; empty when row0 >= rows.
__device__ __forceinline__ rsrc_t rows_rsrc(const char* base, int row0, int rows, uint32_t stride,
                                            uint32_t row_bytes) {
  const int n = rows - row0;
  return make_rsrc(base + (int64_t)row0 * stride, n > 0 ? (uint32_t)(n - 1) * stride + row_bytes : 0u);
}

__device__ __forceinline__ u32x4 ld128(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ uint32_t ld16(rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
__device__ __forceinline__ u32x2 ld64(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
__device__ __forceinline__ uint32_t ld8(rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, off, 0, 0);
}
__device__ __forceinline__ void st64(u32x2 v, rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, 0);
}

__device__ __forceinline__ u32x4 zero4() { return u32x4{0u, 0u, 0u, 0u}; }

template <int I>
using IC = std::integral_constant<int, I>;

// Hides a value from the optimizer, so that a select feeding a load's offset stays
// a select instead of becoming a branch around two loads.
__device__ __forceinline__ uint32_t opaque(uint32_t x) {
  asm("" : "+v"(x));
  return x;
}

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
};

typedef float f32x2 __attribute__((ext_vector_type(2)));

// Two floats rounded (to nearest even) into one word, lo in the low half: a single
// v_cvt_pk_{bf16,f16}_f32.
template <typename T16>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  typedef T16 h2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), h2));
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

// Workgroup barrier for the LDS exchanges between waves (partial similarities,
// P, norms): the wave's own LDS accesses complete first (lgkmcnt(0)), and memory
// clobbers keep the compiler from moving LDS accesses across it. Global loads and
// the buffer-to-LDS copies stay in flight: a workgroup-scope LDS fence would
// also wait for every copy (they write LDS), but each wave only ever reads the
// copies it issued itself, and the compiler's own wait before those reads covers
// them.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// LDS-geometry of one (BM, NK) variant. Key tiles, the query rows and the gate
// rows live in LDS as per-wave "slices": wave w's 32 * NK features of a row,
// stored as CPRP 16-byte chunks (CPR real ones, padded to whole 128-byte groups).
// Chunk c of row r sits at position r * CPRP + swizzle(r, c), an XOR of c's low
// bits with a permutation of r's low bits, within groups of G chunks. With it the
// similarity operand reads (16 rows, one chunk), the transposed mixing reads (4
// rows, two chunks) and the epilogue reads all hit distinct LDS banks, while every
// 128-byte group still arrives from one 128-byte run of global memory.
template <int BM, int NK>
struct Geo {
  static constexpr int QB = BM / 16, DS = 32 * NK, NT = DS / 16;
  static constexpr int CPR = 4 * NK;
  static constexpr int CPRP = (CPR + 7) / 8 * 8;
  static constexpr int G = CPRP % 16 == 0 ? 16 : 8;
  static constexpr int SLICE = kBN * CPRP * 16;  // bytes of one wave's rows of a key tile
  static constexpr int TILE = kWaves * SLICE;    // bytes of one ring slot
  static constexpr int KDMA = kBN * CPRP / 64;   // DMA instructions per wave per key tile
  // Lane offsets of consecutive DMA instructions repeat every P instructions, which
  // cover RPP = 16 rows (the swizzle's period): only P offsets are kept, and the
  // rows they advance go into the resource base.
  static constexpr int P = CPRP / 4;
  static constexpr int RPP = 16;
  static constexpr int SX = kWaves * 2 * QB * 64 * 16;
  // One plane of P (16-bit MFMA operands, a sink row for idle units); the
  // normalised variants keep a second plane for the low part of P.
  static constexpr int PX = (QB + 1) * 64 * 16;
  // The query rows of the prologue take ring slot R-1 and, for BM = 64, this
  // region too, which later holds the partial similarities and both planes of P.
  static constexpr int OVF = (BM > 32 && TILE > SX + 2 * PX) ? TILE : SX + 2 * PX;
  static constexpr int SMALL = 4 * (kWaves * kBN + kBN + kWaves * BM + BM + (QB + 1) * 2 * 4 * 16 + BM);
  static constexpr int kLdsMax = 160 * 1024;
  // Ring depth: three slots where they fit, else two.
  static constexpr int R = 3 * TILE + OVF + SMALL <= kLdsMax ? 3 : 2;
  static_assert(2 * TILE + OVF + SMALL <= kLdsMax, "tile does not fit the LDS");
  static_assert(BM <= 32 * R, "query rows must fit the ring");
  // Query split (the 32- and 64-row variants whose halved state fits 256 registers):
  // 8 waves, waves w and w + 4 both serve feature slice w, each for half of the query
  // blocks. Every wave runs every stage on its half (the key rows of a slice are read
  // by both), so a wave holds half the accumulators and each SIMD holds two waves
  // whose stalls the other fills. The others keep 4 waves of 512 registers.
  static constexpr bool QS = fused_query_split(BM, NK);
  static constexpr int THREADS = (QS ? 2 : 1) * kThreads;
  static constexpr int QBW = QS ? QB / 2 : QB;        // query blocks per wave
  static constexpr int KD = QS ? KDMA / 2 : KDMA;     // refill copies per wave per tile
};

template <int G>
__device__ __forceinline__ int swz(int r) {
  const int h = G == 8 ? (r & 15) >> 1 : (r & 15);
  return G == 8 ? (((h << 1) & 7) | (h >> 2)) : (((h << 1) & 15) | (h >> 3));
}
template <int G>
__device__ __forceinline__ int swzc(int r, int c) {
  return (c & ~(G - 1)) | ((c ^ swz<G>(r)) & (G - 1));
}

template <int BM>
struct SmallLds {
  float nxp[kWaves][kBN];            // per-wave partial sums of squares of the keys; -1: padded key
  // 1 / max(||k||, norm_eps) of key 4 i + j in rk[i][j]; 0 for padded or out-of-range
  // keys. Stored as 16-byte vectors so the four a lane reads are one aligned load: an
  // under-aligned vector load is split, and the split accesses lose the alias scopes
  // that tell the compiler they cannot overlap a buffer-to-LDS copy in flight (it
  // would then wait for every copy before them).
  f32x4 rk[kBN / 4];
  float nq[kWaves][BM];              // per-wave partial sums of squares of the queries
  float rq[BM];                      // 1 / max(||q||, norm_eps); 0 for padded or out-of-range rows
  float dx[BM / 16 + 1][2][4][16];   // signed row-sum partials; last row: sink of idle waves
  float dq[BM];                      // 1 / (full signed row sum + eps)
};

// Global -> LDS copy of 16 bytes per lane: lane l's bytes land at lds + 16 l.
__device__ __forceinline__ void dma16(rsrc_t r, char* lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, off, 0, 0, 0);
}
// Global -> LDS copy of 4 bytes per lane (lane l's word lands at lds + 4 l).
__device__ __forceinline__ void dma4(rsrc_t r, char* lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 4, off, 0, 0, 0);
}
__device__ __forceinline__ void st128(u32x4 v, rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 0);
}
// s_waitcnt lgkmcnt(0), leaving the vector-memory counters alone: the wave's LDS
// reads of a ring slot have finished before a DMA refills it.
__device__ __forceinline__ void wait_lds_reads() { __builtin_amdgcn_s_waitcnt(0xC07F); }

}  // namespace

// FULL: D == 4 * 32 * NK, so every chunk a wave touches lies inside the row.
// Otherwise chunks at or past D are redirected to kNowhere (D % 8 == 0 makes a
// chunk wholly in or out). STRIDED: z_tr / z_tl rows and batch items are apart by
// the strides in FwdParams; otherwise contiguous (a separate instantiation: the
// runtime strides cost registers, and the 64-row variants then spill more).
// HILO (the normalised, Avey-B calls): the mixing product takes P as two 16-bit
// parts, P_hi = rnd(P) and P_lo = rnd(P - P_hi), in two MFMAs into the same fp32
// accumulator. P then enters the numerator to about 2^-17 (bf16) of itself, as
// the denominator's fp32 sum does; with P_hi alone, rows whose signed sum cancels
// amplify the 2^-9 rounding of each term past the bf16 bound.
template <typename T16, int BM, int NK, bool FULL, bool STRIDED, bool HILO>
__global__ __launch_bounds__((Geo<BM, NK>::THREADS), 1) void fused_fwd_kernel(FwdParams p) {
  typedef Geo<BM, NK> Gm;
  static_assert(BM > 16 && Gm::THREADS == fused_threads(BM, NK), "16-row blocks run fused16_kernel");
  constexpr bool QS = Gm::QS;
  constexpr int QB = Gm::QB, DS = Gm::DS, NT = Gm::NT, CPR = Gm::CPR, CPRP = Gm::CPRP, G = Gm::G;
  constexpr int SLICE = Gm::SLICE, TILE = Gm::TILE, R = Gm::R, KDMA = Gm::KDMA;
  constexpr int QBW = Gm::QBW, KD = Gm::KD;
  // Reduction units (query block, key half) are shared by RW waves.
  constexpr int RW = QS ? 2 * kWaves : kWaves;
  constexpr int UNITS = 2 * QB, UPW = (UNITS + RW - 1) / RW;
  // One LDS object per ring slot: the compiler's wait for a slot's DMA then covers
  // that slot only, not the refills in flight for the others.
  __shared__ __attribute__((aligned(16))) char slot0[TILE];
  __shared__ __attribute__((aligned(16))) char slot1[TILE];
  __shared__ __attribute__((aligned(16))) char slot2[R == 3 ? TILE : 16];
  __shared__ __attribute__((aligned(16))) char ovf[Gm::OVF];
  __shared__ SmallLds<BM> sm;
  // Landing place of the cache-line touches below; never read.
  __shared__ __attribute__((aligned(16))) char touch_sink[256];
  static_assert(sizeof(SmallLds<BM>) <= Gm::SMALL, "small LDS arrays");
  f32x4(*const sx)[2][QB][64] = reinterpret_cast<f32x4(*)[2][QB][64]>(ovf);           // [wave][kb][qb][lane]
  u32x4(*const px)[64] = reinterpret_cast<u32x4(*)[64]>(ovf + Gm::SX);                // [qb (QB: sink)][lane]
  u32x4(*const pxl)[64] = reinterpret_cast<u32x4(*)[64]>(ovf + Gm::SX + Gm::PX);      // P_lo, as px (HILO)

  // The wave index is read into a scalar register, so that LDS addresses built
  // from it (DMA destinations go through M0) stay scalar.
  const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int li = lane & 15, lg = lane >> 4;
  // w: the feature slice this wave serves; h: the query half of a query-split wave,
  // whose query blocks are qb0 .. qb0+QBW-1.
  const int w = QS ? (wv & (kWaves - 1)) : wv;
  const int h = QS ? (wv >> 2) : 0;
  const int qb0 = h * QBW;
  const int C = (int)p.C, D = (int)p.D, B = (int)p.B;
  const int n_qt = (C + BM - 1) / BM;
  int b, qt;
  block_item((int)blockIdx.x, B, n_qt, p.causal != 0, b, qt);
  const int q0 = qt * BM;
  const uint32_t row_bytes = (uint32_t)D * 2u;
  // z_tr and z_tl may be strided views (rows and batch items `*stride` apart).
  const uint32_t zstride = STRIDED ? (uint32_t)p.zrs * 2u : row_bytes;
  const uint32_t gstride = STRIDED ? (uint32_t)p.grs * 2u : row_bytes;
  const char* zb = (const char*)p.z + (STRIDED ? (int64_t)b * p.zbs * 2 : (int64_t)b * C * row_bytes);
  const bool has_valid = p.valid != nullptr, has_v = p.v != nullptr;
  const bool has_gate = p.gate != nullptr, has_bias = p.bias != nullptr;
  const char* gb = has_gate ? (const char*)p.gate + (STRIDED ? (int64_t)b * p.gbs * 2 : (int64_t)b * C * row_bytes)
                             : (const char*)p.z;
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
  const int nkt = (int)key_tiles_for(qt, C, BM, kBN, causal);

  // ---- addressing -------------------------------------------------------------------
  // This wave's part of ring slot I, and row group j (32 rows) of the query region
  // (prologue) and of the gate / output region (epilogue). Key tile t sits in slot
  // t % R.
  auto slot_base = [&](auto slot) -> char* {
    constexpr int I = decltype(slot)::value;
    char* s = I == 0 ? slot0 : (I == 1 ? slot1 : slot2);
    return s + w * SLICE;
  };
  auto qrows_base = [&](int j) -> char* { return j == 0 ? ((R == 3 ? slot2 : slot1) + w * SLICE) : (ovf + w * SLICE); };
  auto erows_base = [&](int j) -> char* { return (j == 0 ? slot0 : slot1) + w * SLICE; };

  // Global byte offset (from a region's first row; rows `stride` bytes apart) of
  // slice position pos, i.e. row pos / CPRP, chunk swizzle(row, pos % CPRP);
  // kNowhere past the slice or past D.
  auto goff = [&](int pos, uint32_t stride) -> uint32_t {
    const int r = pos / CPRP, c = swzc<G>(r, pos % CPRP);
    const int col = fw + 8 * c;
    return (c < CPR && (FULL || col < D)) ? (uint32_t)r * stride + (uint32_t)col * 2u : kNowhere;
  };
  constexpr int P = Gm::P, RPP = Gm::RPP;
  // The DMA lane offsets stay in registers unless the variant's registers are
  // full (BM = 64 with 768-feature rows), where they are recomputed per tile.
  constexpr bool KOF_LIVE = !QS && QB * NK < 24;
  uint32_t kof_live[P];
  if constexpr (KOF_LIVE) {
#pragma unroll
    for (int j = 0; j < P; ++j) kof_live[j] = goff(64 * j + lane, zstride);
  }
  // LDS byte offsets of this lane's fragments inside a slice (see Geo):
  //   a1: similarity operands, row li, chunk 4 s + lg          (s % (G / 4) picks the entry)
  //   a2: transposed mixing operands, row 4 lg + li / 4, chunk 2 t + (li & 3) / 2, half li & 1
  //   a3: epilogue, row li, chunk 2 t + lg / 2, half lg & 1     (t % (G / 2) picks the entry)
  uint32_t a1[G / 4], a2[G / 2];
#pragma unroll
  for (int m = 0; m < G / 4; ++m) a1[m] = 16u * (uint32_t)(li * CPRP + swzc<G>(li, 4 * m + lg));
  {
    const int r0 = 4 * lg + (li >> 2);
#pragma unroll
    for (int m = 0; m < G / 2; ++m)
      a2[m] = 16u * (uint32_t)(r0 * CPRP + swzc<G>(r0, 2 * m + ((li & 3) >> 1))) + 8u * (uint32_t)(li & 1);
  }
  auto frag_a = [&](const char* base, int row16, int s) -> u32x4 {
    return *reinterpret_cast<const u32x4*>(base + a1[s % (G / 4)] + 16 * (16 * row16 * CPRP + G * (s / (G / 4))));
  };

  // Reduction units: unit u = r + RW j -> (query block u/2, key half u%2), r the
  // wave's rank among the RW reducing waves. Waves with fewer real units than UPW
  // run a copy of unit 0 whose results go to the sink rows, so every wave executes
  // the same branch-free code.
  const int rr = QS ? wv : w;
  int uq[UPW], uk[UPW], pq[UPW];
  float ud[UPW];
  uint32_t voff[UPW];
#pragma unroll
  for (int j = 0; j < UPW; ++j) {
    const bool real = (UNITS % RW == 0) || (rr + RW * j < UNITS);
    const int u = real ? rr + RW * j : 0;
    uq[j] = u >> 1;
    uk[j] = u & 1;
    pq[j] = real ? uq[j] : QB;
    // key - query = ud + i - (q0 - k0) for the lane's keys i = 0..3
    ud[j] = (float)(16 * uk[j] + 4 * lg - 16 * uq[j] - li);
    // V[q][k0 + 16 uk + 4 lg + i] relative to V + k0: row q = q0 + 16 uq + li
    voff[j] = ((uint32_t)(q0 + 16 * uq[j] + li) * (uint32_t)C + (uint32_t)(16 * uk[j] + 4 * lg)) * 2u;
  }
  const uint32_t vbytes = has_v ? (uint32_t)C * (uint32_t)C * 2u : 0u;

  // ---- loads ------------------------------------------------------------------------
  // Key tile t (its 32 rows, this wave's slice) into ring slot I, with the validity
  // bytes of its two 16-row blocks (rows past the context read 0 and are told apart
  // by their index). Tiles past the last are not fetched.
  uint32_t zv[R][2];
  auto key_offsets = [&](uint32_t (&kof)[P]) {
    if constexpr (KOF_LIVE) {
#pragma unroll
      for (int j = 0; j < P; ++j) kof[j] = kof_live[j];
    } else {
      // Recomputed from an opaque lane index, so the compiler cannot keep them live.
      const int ln = (int)opaque((uint32_t)lane);
#pragma unroll
      for (int j = 0; j < P; ++j) kof[j] = goff(64 * j + ln, zstride);
    }
  };
  // DMA instruction j (of KDMA) of key tile t into this wave's part of a ring slot.
  // The refills sit under uniform branches (`if (refill)`), not issued through an
  // empty resource when there is nothing to fetch: unconditional copies into a
  // free slot have been seen to make the compiler drop the wait that a later read
  // of the other slot needs (it read a tile whose copies were still in flight).
  auto fetch_key_part = [&](int t, char* dst, int j, const uint32_t (&kof)[P]) {
    dma16(rows_rsrc(zb, t * kBN + RPP * (j / P), C, zstride, row_bytes), dst + 1024 * j, kof[j % P]);
  };
  auto fetch_valid = [&](int t, auto slot, bool live = true) {
    constexpr int I = decltype(slot)::value;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
      zv[I][kb] = ld8(rows_rsrc(vb, t * kBN + 16 * kb, live ? valid_rows : 0, 1u, 1u), (uint32_t)li);
  };
  // This wave's share of a key tile's copies: all KDMA, or (query split) the half
  // jj + h KD of them, KD = P, so the lane offsets are indexed by jj alone.
  // Query split: the copies go out whether or not there is a tile to fetch (`live`;
  // otherwise through an empty resource, writing zeros into the free slot), so that
  // every iteration issues the same number of copies and the waits that order them
  // for the partner wave can count them (see wait_next_tile).
  constexpr bool UNCOND = QS;
  // A refilled tile's validity bytes: loaded after its copies by the 4-wave variants
  // (they are then live for less of the iteration, which the 64-row variants'
  // registers need), before them by the others (the query-split waits count the
  // copies as the newest loads).
  constexpr bool VALID_LATE = !QS;
  auto fetch_key_share = [&](int t, char* dst, int jj, const uint32_t (&kof)[P], bool live) {
    if constexpr (QS)
      dma16(rows_rsrc(zb, t * kBN + RPP * h, live ? C : 0, zstride, row_bytes), dst + 1024 * (h * KD + jj), kof[jj]);
    else
      fetch_key_part(t, dst, jj, kof);
  };
  auto fetch_keys = [&](int t, auto slot) {
    uint32_t kof[P];
    key_offsets(kof);
#pragma unroll
    for (int j = 0; j < KD; ++j) fetch_key_share(t, slot_base(slot), j, kof, true);
    fetch_valid(t, slot);
  };
  // BM rows (`stride` bytes apart) of a batch item from row q0 into a row region
  // (prologue: the queries; tail: the gate).
  // (Query split: the wave's half of the rows, copies h JR .. h JR + JR - 1.)
  constexpr int JR = BM * CPRP / 64 / (QS ? 2 : 1);  // copies of a wave's row share
  auto fetch_rows = [&](const char* src, uint32_t stride, auto region) {
    uint32_t kof[P];
#pragma unroll
    for (int j = 0; j < P; ++j) kof[j] = goff(64 * j + lane, stride);
#pragma unroll
    for (int jj = 0; jj < JR; ++jj) {
      const int j = h * JR + jj;  // JR is a multiple of P: j % P == jj % P
      dma16(rows_rsrc(src, q0 + RPP * (j / P), C, stride, row_bytes), region(j / KDMA) + 1024 * (j % KDMA),
            kof[jj % P]);
    }
  };
  // V entries of tile k0 for this wave's units (raw 16-bit words, two per dword): the
  // lane's four keys are adjacent, so with an even context one dword-aligned 8-byte
  // load fetches them. With an odd one a row may start mid-dword, and V's last dword
  // is half past its end (a buffer load reads such a dword as 0), so the entries are
  // then read one by one. Entries past the end of V read 0; their keys are masked.
  auto load_v = [&](int k0, u32x2 (&vv)[UPW]) {
    const uint32_t skip = (uint32_t)k0 * 2u;
    const rsrc_t r = make_rsrc((const char*)(has_v ? p.v : p.z) + skip, vbytes > skip ? vbytes - skip : 0u);
    if ((C & 1) == 0) {
#pragma unroll
      for (int j = 0; j < UPW; ++j) vv[j] = ld64(r, voff[j]);
    } else {
#pragma unroll
      for (int j = 0; j < UPW; ++j)
        vv[j] = u32x2{ld16(r, voff[j]) | (ld16(r, voff[j] + 2u) << 16), ld16(r, voff[j] + 4u) | (ld16(r, voff[j] + 6u) << 16)};
    }
  };

  // ---- prologue: the query rows, the first R-1 key tiles, the query norms ------------
  fetch_rows((const char*)zb, zstride, qrows_base);
  fetch_keys(0, IC<0>{});
  if constexpr (R == 3) {
    if (1 < nkt) fetch_keys(1, IC<1>{});
  }
  // The gate rows are first read in the tail; one touch per 128-byte line ahead of
  // that brings them into the L2, so that their fetch does not wait on HBM. When the
  // whole grid's gate rows fit the L2s with room to spare (8 MB over 8 XCDs) the
  // touch goes out now; otherwise three key tiles before the tail, as touching them
  // all at once would push the key tiles out of the L2.
  constexpr int kTouchLead = 3;
  const bool gate_fits = (uint64_t)B * (uint64_t)C * row_bytes <= (8ull << 20);
  const int touch_t = gate_fits ? 0 : nkt - kTouchLead;  // the iteration that touches; < 1: here
  constexpr int kTouchLanes = QS ? Gm::THREADS : kThreads;  // lanes of the touching waves
  auto touch_gate = [&]() {
    const rsrc_t r = rows_rsrc(gb, q0, min(C, q0 + BM), gstride, row_bytes);
    constexpr int kLines = 4 * 32 * NK * 2 / 128;                              // 128-byte lines per row
    constexpr int kTouches = (BM * kLines + kTouchLanes - 1) / kTouchLanes;  // lines over the lanes
#pragma unroll
    for (int i = 0; i < kTouches; ++i) {
      const uint32_t line = (uint32_t)(i * kTouchLanes + tid), c = line % kLines;
      dma4(r, touch_sink, c * 128u < row_bytes ? (line / kLines) * gstride + c * 128u : kNowhere);
    }
  };
  // (Query split: after the first barrier, which waits for every copy before it.)
  if (!QS && has_gate && touch_t < 1) touch_gate();
  // Query fragments of this wave's query blocks (local index qb: block qb0 + qb).
  u32x4 qf[QBW][NK];
  {
  uint32_t qv[QBW];
#pragma unroll
  for (int qb = 0; qb < QBW; ++qb)
    qv[qb] = ld8(rows_rsrc(vb, q0 + 16 * (qb0 + qb), valid_rows, 1u, 1u), (uint32_t)li);
#pragma unroll
  for (int qb = 0; qb < QBW; ++qb) {
    const int qg = qb0 + qb;
    const bool ok = (16 * qg + li < C - q0) && ((qv[qb] | or_valid) != 0u);
    float ss = 0.f;
#pragma unroll
    for (int s = 0; s < NK; ++s) {
      const u32x4 x = frag_a(qrows_base(qg >> 1), qg & 1, s);
      qf[qb][s] = ok ? x : zero4();  // select, so NaN in padded rows never enters
      ss = Ops<T16>::sumsq(qf[qb][s], ss);
    }
    ss = sum_over_groups(ss);
    if (lg == 0) sm.nq[w][16 * qg + li] = ok ? ss : -1.f;
  }
  }

  f32x4 oacc[NT][QBW];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int qb = 0; qb < QBW; ++qb) oacc[t][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float den[UPW];
#pragma unroll
  for (int j = 0; j < UPW; ++j) den[j] = 0.f;
  f32x4 sacc[2][QBW];
  u32x2 vv[UPW];
  u32x4 ztr[NT];  // transposed mixing operands of the previous tile

  // ---- T(t): the mixing operands of tile t, read transposed from its slot -------------
  auto stage_t = [&](auto slot) {
    const char* base = slot_base(slot);
#pragma unroll
    for (int t2 = 0; t2 < NT; ++t2) {
      const uint32_t o = a2[t2 % (G / 2)] + 16u * (uint32_t)(G * (t2 / (G / 2)));
      const u32x2 lo = __builtin_bit_cast(u32x2, lds_read_tr((const uint16_t*)(base + o)));
      const u32x2 hi = __builtin_bit_cast(u32x2, lds_read_tr((const uint16_t*)(base + o + 16 * 16 * CPRP)));
      ztr[t2] = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
  };

  // ---- A(t): partial similarity from slot I, key partial norms. When `refill`, the
  // refill of slot F with key tile tf goes out interleaved with MFMAs, so that the
  // memory queue drains behind them instead of stalling the wave: with at most 32
  // query rows it is spread thinly over A and C (one DMA every other MFMA; A issues
  // [0, KA), C the rest), while the 64-row variants, whose registers are full, keep
  // it in A, one DMA per step. A issues DMAs [0, JE). The DMAs sit under their own
  // uniform branches, so the MFMA code is not duplicated.
  // (Query split: the 64-row variants take this order too. Their halved
  // accumulators leave room for the mixing operands across the barrier, and the other
  // order would let one wave's refill overwrite rows its partner is still reading.)
  constexpr bool SPLIT = BM <= 32 || QS;
  constexpr int KA = SPLIT ? (KD + 1) / 2 : KD;
  constexpr int SP = SPLIT ? 2 : 1;  // MFMA steps per DMA in A
  auto stage_a = [&](int t, auto slot, int tf, auto fslot, bool refill, auto je) {
    constexpr int I = decltype(slot)::value;
    constexpr int JE = decltype(je)::value;
    const int k0 = t * kBN;
    char* base = slot_base(slot);
    uint32_t kof[P];
    key_offsets(kof);
    if (has_valid) {
      // Padded rows may hold NaN: once the tile has landed, zero them in this wave's
      // slice before they reach the products, the norms or the mixing operands.
      const uint64_t bad0 = __builtin_amdgcn_ballot_w64(lg == 0 && zv[I][0] == 0u);
      const uint64_t bad1 = __builtin_amdgcn_ballot_w64(lg == 0 && zv[I][1] == 0u);
      uint32_t bad = ((uint32_t)bad0 & 0xffffu) | (((uint32_t)bad1 & 0xffffu) << 16);
      if (bad != 0u) {
        __builtin_amdgcn_s_waitcnt(0);
        while (bad != 0u) {
          const int r = __builtin_ctz(bad);
          bad &= bad - 1u;
          if (lane < CPRP) *reinterpret_cast<u32x4*>(base + 16 * (r * CPRP + lane)) = zero4();
        }
      }
    }
    float nkey[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const bool ok = (16 * kb + li < C - k0) && ((zv[I][kb] | or_valid) != 0u);
#pragma unroll
      for (int qb = 0; qb < QBW; ++qb) sacc[kb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
      float ss = 0.f;
#pragma unroll
      for (int s = 0; s < NK; ++s) {
        const u32x4 a = frag_a(base, kb, s);
#pragma unroll
        for (int qb = 0; qb < QBW; ++qb) sacc[kb][qb] = Ops<T16>::mfma32(a, qf[qb][s], sacc[kb][qb]);
        ss = Ops<T16>::sumsq(a, ss);
        const int step = kb * NK + s;
        if (step % SP == 0 && step / SP < JE && (UNCOND || refill))
          fetch_key_share(tf, slot_base(fslot), step / SP, kof, refill);
      }
      ss = sum_over_groups(ss);
      nkey[kb] = ok ? ss : -1.f;
    }
    if (UNCOND || refill) {
#pragma unroll
      for (int j = (2 * NK + SP - 1) / SP; j < JE; ++j) fetch_key_share(tf, slot_base(fslot), j, kof, refill);
      if constexpr (VALID_LATE && JE == KD) fetch_valid(tf, fslot);
    }
    // Lane groups 0 / 1 write the two key halves (groups 2 / 3 repeat them).
    sm.nxp[w][16 * (lg & 1) + li] = (lg & 1) ? nkey[1] : nkey[0];
  };

  // ---- B(t): reduce partials, scale, weight, mask, publish P; then V of tile t+1 ------
  auto stage_b = [&](int t) {
    const int k0 = t * kBN;
    // causal: keep key <= query, i.e. ud + i <= q0 - k0
    const float lim = causal ? (float)(q0 - k0) : 1e30f;
#pragma unroll
    for (int j = 0; j < UPW; ++j) {
      const int qb = uq[j], kb = uk[j];
      f32x4 sv = sx[0][kb][qb][lane];
#pragma unroll
      for (int x = 1; x < kWaves; ++x) sv += sx[x][kb][qb][lane];
      const f32x4 rk4 = sm.rk[4 * kb + lg];
      const float rqv = sm.rq[16 * qb + li];  // 0 for padded / out-of-range queries
      float pv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // Causal and key-padding masks (padded / out-of-range keys have rk == 0) as
        // bitwise selects: whatever V holds there, the entry is an exact +0.
        const uint32_t keep = ((ud[j] + (float)i <= lim) & (rk4[i] > 0.f)) ? 0xffffffffu : 0u;
        const uint32_t vw = vv[j][i >> 1];
        const float x = sv[i] * (rk4[i] * rqv) * Ops<T16>::to_f_or((i & 1) ? vw >> 16 : vw & 0xffffu, or_v);
        pv[i] = __uint_as_float(__float_as_uint(x) & keep);
        den[j] += pv[i];
      }
      const uint32_t h01 = pack2<T16>(pv[0], pv[1]), h23 = pack2<T16>(pv[2], pv[3]);
      reinterpret_cast<u32x2*>(&px[pq[j]][lane])[kb] = u32x2{h01, h23};
      if constexpr (HILO) {
        // P - P_hi is exact in fp32 (P_hi holds P's leading bits); its rounding is P_lo.
        const float l0 = pv[0] - Ops<T16>::to_f(h01 & 0xffffu), l1 = pv[1] - Ops<T16>::hi_f(h01);
        const float l2 = pv[2] - Ops<T16>::to_f(h23 & 0xffffu), l3 = pv[3] - Ops<T16>::hi_f(h23);
        reinterpret_cast<u32x2*>(&pxl[pq[j]][lane])[kb] = u32x2{pack2<T16>(l0, l1), pack2<T16>(l2, l3)};
      }
    }
    load_v(t + 1 < nkt ? (t + 1) * kBN : C, vv);
  };

  // ---- C: mixing of the previous tile from the transposed operands in registers; with
  // FETCH, the second part of the refill A started (one DMA every other MFMA) ------------
  // FETCH: this variant issues (part of) the refill here; `refill`: it is a real one.
  auto stage_c = [&](int tf, auto fslot, bool refill, auto fetch) {
    constexpr bool FETCH = SPLIT && decltype(fetch)::value;
    uint32_t kof[P];
    if constexpr (FETCH) key_offsets(kof);
    u32x4 pf[QBW];
#pragma unroll
    for (int qb = 0; qb < QBW; ++qb) pf[qb] = px[qb0 + qb][lane];
#pragma unroll
    for (int t2 = 0; t2 < NT; ++t2)
#pragma unroll
      for (int qb = 0; qb < QBW; ++qb) {
        oacc[t2][qb] = Ops<T16>::mfma32(ztr[t2], pf[qb], oacc[t2][qb]);
        const int m = t2 * QBW + qb;
        if (m % 2 == 0 && KA + m / 2 < KD && FETCH && (UNCOND || refill))
          fetch_key_share(tf, slot_base(fslot), KA + m / 2, kof, refill);
      }
    if constexpr (HILO) {
      // The low part of P, one query block at a time (its operand is live for one
      // block only: the 64-row variants' registers are full).
#pragma unroll
      for (int qb = 0; qb < QBW; ++qb) {
        const u32x4 pl = pxl[qb0 + qb][lane];
#pragma unroll
        for (int t2 = 0; t2 < NT; ++t2) oacc[t2][qb] = Ops<T16>::mfma32(ztr[t2], pl, oacc[t2][qb]);
      }
    }
    if (FETCH && (UNCOND || refill)) {
#pragma unroll
      for (int j = KA + (NT * QBW + 1) / 2; j < KD; ++j) fetch_key_share(tf, slot_base(fslot), j, kof, refill);
      if constexpr (VALID_LATE) fetch_valid(tf, fslot);
    }
  };

  // ---- interval-2 publication: A(t)'s partial S^T and the tile's key reciprocals
  // (every wave computes the same reciprocals, lanes 32..63 repeating 0..31, so no
  // wave waits on a branch here) ---------------------------------------------------
  auto publish = [&]() {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int qb = 0; qb < QBW; ++qb) sx[w][kb][qb0 + qb][lane] = sacc[kb][qb];
    const int k = lane & (kBN - 1);
    const float n = (sm.nxp[0][k] + sm.nxp[1][k]) + (sm.nxp[2][k] + sm.nxp[3][k]);
    // A float store: an element assignment to the vector would be a read-modify-
    // write of all 16 bytes, racing with the lanes that own the other three keys.
    reinterpret_cast<float*>(sm.rk)[k] = n < 0.f ? 0.f : (n > eps2 ? __builtin_amdgcn_rsqf(n) : inv_eps);
  };

  // s_waitcnt encodings (gfx9: vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt at
  // their maxima, i.e. not waited for).
  static_assert(KDMA + 2 < 64, "vmcnt holds 6 bits");
  auto wait_all = [&]() { __builtin_amdgcn_s_waitcnt(0x0F70); };  // vmcnt(0)
  // All but the newest N vector-memory operations retired (they return in issue order).
  auto wait_keep = [&](auto n) {
    constexpr int N = decltype(n)::value;
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
  };
  // Query split: each wave of a slice copies half of a key tile's rows and reads them
  // all, so a wave's copies are ordered before its partner's reads by its own wait and
  // a barrier. Before the barrier that closes iteration t, key tile t+1 has landed:
  // with two slots it is this iteration's refill (all of it retires); with three it
  // is the previous one, and this iteration's stays in flight: its KD copies, which
  // every iteration issues (see fetch_key_share) after its other loads (the tile's
  // validity bytes go out first), and which come after everything of the previous
  // iteration (nothing moves across a barrier). Anything of this iteration issued
  // after them only makes the wait retire more. After the last iteration everything
  // retires: the tail's gate rows then land in slots that the partner's last (empty)
  // copies also write.
  auto wait_next_tile = [&](bool last) {
    if constexpr (R == 3) {
      wait_keep(IC<KD>{});
      if (last) wait_all();
    } else {
      wait_all();
    }
  };

  // t = 0: A only (with the whole fetch of the last tile of the ring's first round);
  // the query norms, A(0)'s publication and tile 0's mixing operands. The query rows
  // share slot R-1 with that tile; their reads into qf are complete (the norms above
  // consumed them) before the refill is issued (after the wave's LDS reads retired;
  // query split: after a barrier, as the partner read them too).
  // Steady-state iterations run over t = 1 .. nkt-1, unrolled by R so that every slot
  // index is a constant.
  auto run_loop = [&](auto iter) {
    int t = 1;
    if constexpr (R == 2) {
      for (; t + 1 < nkt; t += 2) {
        iter(t, IC<1>{});
        iter(t + 1, IC<0>{});
      }
      if (t < nkt) iter(t, IC<1>{});
    } else {
      for (; t + 2 < nkt; t += 3) {
        iter(t, IC<1>{});
        iter(t + 1, IC<2>{});
        iter(t + 2, IC<0>{});
      }
      if (t < nkt) iter(t, IC<1>{});
      if (t + 1 < nkt) iter(t + 1, IC<2>{});
    }
  };
  using TT = std::true_type;
  using FF = std::false_type;
  if constexpr (QS) {
    // Key tile 0 (and 1) from both waves of the slice; the partner's query reads done
    // before this wave's refill overwrites slot R-1.
    wait_all();
    lds_barrier();
    if (has_gate && touch_t < 1) touch_gate();
  }
  load_v(0, vv);
  wait_lds_reads();
  if constexpr (!VALID_LATE) fetch_valid(R - 1, IC<R - 1>{}, R - 1 < nkt);
  stage_a(0, IC<0>{}, R - 1, IC<R - 1>{}, R - 1 < nkt, IC<KD>{});
  lds_barrier();
  if (tid < BM) {
    float ss = 0.f;
#pragma unroll
    for (int x = 0; x < kWaves; ++x) ss += sm.nq[x][tid];
    // F.normalize divides by max(||q||, norm_eps); 0 marks padded / out-of-range rows.
    sm.rq[tid] = ss < 0.f ? 0.f : (ss > eps2 ? __builtin_amdgcn_rsqf(ss) : inv_eps);
  }
  publish();
  if constexpr (SPLIT) stage_t(IC<0>{});
  if constexpr (QS) wait_next_tile(nkt == 1);
  lds_barrier();
  // Steady state, unrolled by R so that every slot index is a constant. Iteration
  // t runs B(t-1), then A(t); then C(t-1) and A(t)'s publication, and refills tile
  // t-1's slot with tile t+R-1. With SPLIT, T(t) (tile t's mixing operands) closes
  // the iteration, so tile t-1's slot is free all along and its refill spreads over
  // A(t) and C(t-1); otherwise T(t-1) opens it and the refill waits for its reads.
  auto iteration = [&](int t, auto cur) {
    constexpr int I = decltype(cur)::value, PREV = (I + R - 1) % R;
    const bool refill = t + R - 1 < nkt;
    if constexpr (!SPLIT) stage_t(IC<PREV>{});
    // The V words B consumes were loaded an iteration ago.
    stage_b(t - 1);
    if (has_gate && t == touch_t) touch_gate();
    if constexpr (!VALID_LATE) fetch_valid(t + R - 1, IC<PREV>{}, refill);
    if constexpr (!SPLIT) wait_lds_reads();  // the refill overwrites what T read
    stage_a(t, cur, t + R - 1, IC<PREV>{}, refill, IC<KA>{});
    lds_barrier();
    stage_c(t + R - 1, IC<PREV>{}, refill, TT{});
    publish();
    if constexpr (SPLIT) {
      // T(t) overwrites the operands C just used: keep the scheduler from hoisting
      // its reads above C's MFMAs (two live copies would not fit the registers).
      __builtin_amdgcn_sched_barrier(0);
      stage_t(cur);
    }
    if constexpr (QS) wait_next_tile(t + 1 == nkt);
    lds_barrier();
  };
  run_loop(iteration);
  // Tail: the last tile's mixing operands (SPLIT: already in registers); every slot
  // is then free, so the gate rows (already in the L2) stream into this wave's part
  // of slots 0 / 1 while the last reduction and mixing product run.
  if constexpr (!SPLIT) {
    switch ((nkt - 1) % R) {
      case 0: stage_t(IC<0>{}); break;
      case 1: stage_t(IC<1>{}); break;
      default: stage_t(IC<(R == 3 ? 2 : 0)>{}); break;
    }
    wait_lds_reads();
  }
  if (has_gate) fetch_rows(gb, gstride, erows_base);
  // The epilogue's bias words and validity bytes, now that the query fragments are
  // dead: their latency hides behind the last reduction and mixing product.
  u32x2 bw[NT];
  uint32_t qv2[QBW];
  {
    const rsrc_t rbias = make_rsrc(has_bias ? p.bias : p.z, has_bias ? row_bytes : 0u);
#pragma unroll
    for (int t2 = 0; t2 < NT; ++t2) {
      const int f = fw + 16 * t2 + 4 * lg;
      bw[t2] = ld64(rbias, (FULL || f < D) ? (uint32_t)f * 2u : kNowhere);
    }
#pragma unroll
    for (int qb = 0; qb < QBW; ++qb)
      qv2[qb] = ld8(rows_rsrc(vb, q0 + 16 * (qb0 + qb), valid_rows, 1u, 1u), (uint32_t)li);
  }
  stage_b(nkt - 1);
  lds_barrier();
  stage_c(0, IC<0>{}, false, FF{});

  // ---- epilogue: lane holds query 16*(qb0+qb)+li, features fw+16t+4*lg .. +3 ----------
  uint32_t a3[G / 2];
#pragma unroll
  for (int m = 0; m < G / 2; ++m)
    a3[m] = 16u * (uint32_t)(li * CPRP + swzc<G>(li, 2 * m + (lg >> 1))) + 8u * (uint32_t)(lg & 1);
  auto efrag = [&](int qb, int t2) -> char* {
    return erows_base(qb >> 1) + a3[t2 % (G / 2)] + 16 * (16 * (qb & 1) * CPRP + G * (t2 / (G / 2)));
  };
  float rden[QBW];
  if (p.normalize) {
#pragma unroll
    for (int j = 0; j < UPW; ++j) sm.dx[pq[j]][uk[j]][lg][li] = den[j];
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
    for (int qb = 0; qb < QBW; ++qb) rden[qb] = sm.dq[16 * (qb0 + qb) + li];
  } else {
#pragma unroll
    for (int qb = 0; qb < QBW; ++qb) rden[qb] = 1.f;
  }
  const uint32_t one2 = Ops<T16>::kOne | (Ops<T16>::kOne << 16);
  // The result goes back into this wave's gate slots, then out in 16-byte runs. The
  // gate words of up to 12 fragments are read before any result is written: the
  // compiler cannot tell the reads from the writes apart, and interleaved they
  // would pay one LDS round trip each.
  constexpr int GB = NT <= 12 ? NT : 8;
  // The gate rows' DMAs must have landed before the reads below. The compiler's
  // LDS-DMA wait tracking has been seen to drop this wait (the 8-wave variant read
  // gate words still in flight), so it is explicit, and a compiler memory barrier
  // keeps the reads after it; the bias and validity loads it also drains are
  // consumed right away.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  auto finish = [&](auto act_tag) {
    constexpr int ACT = decltype(act_tag)::value;
#pragma unroll
    for (int qb = 0; qb < QBW; ++qb) {
      const bool qok = (qv2[qb] | or_valid) != 0u;
#pragma unroll
      for (int tb = 0; tb < NT; tb += GB) {
        u32x2 gw[GB];
#pragma unroll
        for (int i = 0; i < GB; ++i)
          gw[i] = has_gate ? *reinterpret_cast<const u32x2*>(efrag(qb0 + qb, tb + i)) : u32x2{one2, one2};
#pragma unroll
        for (int i = 0; i < GB; ++i) {
          const int t2 = tb + i;
          float y[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const uint32_t bword = bw[t2][k >> 1], gword = gw[i][k >> 1];
            float x = oacc[t2][qb][k] * rden[qb];
            x += (k & 1) ? Ops<T16>::hi_f(bword) : Ops<T16>::to_f(bword & 0xffffu);
            x = activate<float>(x, ACT);
            x *= (k & 1) ? Ops<T16>::hi_f(gword) : Ops<T16>::to_f(gword & 0xffffu);
            y[k] = qok ? x : 0.f;
          }
          *reinterpret_cast<u32x2*>(efrag(qb0 + qb, t2)) = u32x2{pack2<T16>(y[0], y[1]), pack2<T16>(y[2], y[3])};
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
  // Rows past the context fall outside the resources and are dropped. A wave writes
  // out the rows it wrote above (query split: its half, as in fetch_rows).
  const char* ob = (const char*)p.out + (int64_t)b * C * row_bytes;
  uint32_t kof[P];
#pragma unroll
  for (int j = 0; j < P; ++j) kof[j] = goff(64 * j + lane, row_bytes);
#pragma unroll
  for (int jj = 0; jj < JR; ++jj) {
    const int j = h * JR + jj;
    const u32x4 v = *reinterpret_cast<const u32x4*>(erows_base(j / KDMA) + 1024 * (j % KDMA) + 16 * lane);
    st128(v, rows_rsrc(ob, q0 + RPP * (j / P), C, row_bytes, row_bytes), kof[jj % P]);
  }
}

// Instantiates and launches fused_fwd_kernel<T16, BM, NK, FULL, STRIDED> for one
// BM, type and stride kind; defined in avey_fused_bm{16,32,64}_{bf16,f16}[_strided].hip
// so the variants compile in parallel.
template <typename T16, int BM, bool STRIDED>
hipError_t launch_fused_bm(const FwdParams& p, int nk, int64_t grid, hipStream_t s);
// The 16-row variants with the enricher gate in the epilogue; defined in
// avey_fused_bm16_{bf16,f16}[_strided]_eg.hip.
template <typename T16, bool STRIDED>
hipError_t launch_fused16_enriched(const FwdParams& p, int nk, int64_t grid, hipStream_t s);

template <typename T16, int BM, int NK, bool STRIDED>
hipError_t launch_fused_one(const FwdParams& p, int64_t grid, hipStream_t s) {
  const dim3 g((unsigned)grid), t(Geo<BM, NK>::THREADS);
  const bool full = p.D == 4 * 32 * NK;
  if (p.normalize != 0) {
    if (full)
      fused_fwd_kernel<T16, BM, NK, true, STRIDED, true><<<g, t, 0, s>>>(p);
    else
      fused_fwd_kernel<T16, BM, NK, false, STRIDED, true><<<g, t, 0, s>>>(p);
  } else {
    if (full)
      fused_fwd_kernel<T16, BM, NK, true, STRIDED, false><<<g, t, 0, s>>>(p);
    else
      fused_fwd_kernel<T16, BM, NK, false, STRIDED, false><<<g, t, 0, s>>>(p);
  }
  return hipGetLastError();
}

template <typename T16, int BM, bool STRIDED>
hipError_t launch_fused_nk(const FwdParams& p, int nk, int64_t grid, hipStream_t s) {
  switch (nk) {
    case 1: return launch_fused_one<T16, BM, 1, STRIDED>(p, grid, s);
    case 2: return launch_fused_one<T16, BM, 2, STRIDED>(p, grid, s);
    case 3: return launch_fused_one<T16, BM, 3, STRIDED>(p, grid, s);
    case 4: return launch_fused_one<T16, BM, 4, STRIDED>(p, grid, s);
    case 6: return launch_fused_one<T16, BM, 6, STRIDED>(p, grid, s);
    case 8:
      // 1024-feature rows take the 16-row variant only (the plan's choice for them).
      if constexpr (BM == 16) return launch_fused_one<T16, BM, 8, STRIDED>(p, grid, s);
      return hipErrorInvalidConfiguration;
    default: return hipErrorInvalidConfiguration;
  }
}

}  // namespace avey
