// C ABI of libavey_hip.so: argument checks, the static tile table, dispatch.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "avey_common.h"
#include "avey_internal.h"

namespace avey {

namespace {

constexpr int kMaxDevices = 64;
std::atomic<int> g_device_ok[kMaxDevices];  // 0 unknown, 1 gfx950, 2 other

// Scratch of the allocation-free entry point (avey_fwd_noalloc): one copy of this
// array per GPU, for the life of the process. Host code never uses its name as an
// address (on the host it is only a stand-in for the symbol); the device address of
// each GPU's copy comes from hipGetSymbolAddress, once per device, with that device
// current, and is kept in g_scratch.
static __device__ __align__(256) char scratch[AVEY_NOALLOC_SCRATCH_BYTES];
struct ScratchSlot {
  std::once_flag once;
  void* ptr = nullptr;
  hipError_t err = hipSuccess;
};
ScratchSlot g_scratch[kMaxDevices];

// Device address of `dev`'s copy of the scratch array; `dev` must be current.
hipError_t device_scratch(int dev, void** ptr) {
  ScratchSlot& slot = g_scratch[dev];
  std::call_once(slot.once, [&slot] { slot.err = hipGetSymbolAddress(&slot.ptr, HIP_SYMBOL(scratch)); });
  *ptr = slot.err == hipSuccess ? slot.ptr : nullptr;
  return slot.err;
}

size_t elem_size(int dtype) {
  switch (dtype) {
    case AVEY_DTYPE_F32: return 4;
    case AVEY_DTYPE_F64: return 8;
    case AVEY_DTYPE_BF16:
    case AVEY_DTYPE_F16: return 2;
    default: return 0;
  }
}

// Row and batch strides (elements) of a [B][C][D] operand: row stride 0 means
// contiguous.
struct Strides {
  int64_t row, batch;
};
Strides resolve(int64_t row, int64_t batch, const avey_fwd_args& a) {
  if (row == 0) return {a.features, a.context * a.features};
  return {row, batch};
}
// Elements from the first to one past the last element of a strided operand.
double span_elems(const Strides& st, const avey_fwd_args& a) {
  return (double)(a.batch - 1) * (double)st.batch + (double)(a.context - 1) * (double)st.row + (double)a.features;
}

bool overlaps(const void* a, size_t an, const void* b, size_t bn) {
  if (!a || !b) return false;
  const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
  return x < y + bn && y < x + an;
}

int validate(const avey_fwd_args* a) {
  if (!a || !a->z_tr || !a->out) return AVEY_ERR_NULL_POINTER;
  const size_t es = elem_size(a->dtype);
  if (!es) return AVEY_ERR_DTYPE;
  if (a->batch < 1 || a->context < 1 || a->features < 1) return AVEY_ERR_SHAPE;
  // Keep every element offset and the 1-D grid inside 63 / 31 bits.
  if (a->context > (1 << 24) || a->features > (1 << 24) || a->batch > (1 << 24)) return AVEY_ERR_SHAPE;
  const double n = (double)a->batch * (double)a->context * (double)a->features;
  if (n * (double)es > 9.0e18) return AVEY_ERR_SHAPE;
  if (a->activation < AVEY_ACT_IDENTITY || a->activation > AVEY_ACT_GELU) return AVEY_ERR_ACTIVATION;
  if (!(isfinite(a->eps) && a->eps > 0) || !(isfinite(a->norm_eps) && a->norm_eps > 0)) return AVEY_ERR_EPS;
  if ((a->causal != 0 && a->causal != 1) || (a->normalize != 0 && a->normalize != 1)) return AVEY_ERR_FLAGS;
  const Strides zs = resolve(a->z_tr_row_stride, a->z_tr_batch_stride, *a);
  const Strides gs = resolve(a->z_tl_row_stride, a->z_tl_batch_stride, *a);
  for (const Strides& st : {zs, gs})
    if (st.row < a->features || st.batch < 0 || st.row > (int64_t(1) << 40) || st.batch > (int64_t(1) << 50))
      return AVEY_ERR_STRIDE;
  const double zspan = span_elems(zs, *a), gspan = span_elems(gs, *a);
  if (zspan * (double)es > 9.0e18 || gspan * (double)es > 9.0e18) return AVEY_ERR_SHAPE;
  const size_t nb = (size_t)n * es;
  const size_t vb = (size_t)a->context * (size_t)a->context * es;
  if (overlaps(a->out, nb, a->z_tr, (size_t)zspan * es) || overlaps(a->out, nb, a->z_tl, (size_t)gspan * es) ||
      overlaps(a->out, nb, a->v, vb) ||
      overlaps(a->out, nb, a->bias, (size_t)a->features * es) ||
      overlaps(a->out, nb, a->valid, (size_t)a->batch * (size_t)a->context))
    return AVEY_ERR_ALIAS;
  return AVEY_OK;
}

// Wave slices of the fused kernel come in multiples of 32 features; only these
// slice widths are compiled.
int slice_steps(int64_t D) {
  const int64_t nk = cdiv(D, 128);
  if (nk <= 4) return (int)nk;
  if (nk <= 6) return 6;
  if (nk <= 8) return 8;
  return 0;
}

// Profiling override of the table's row-block height (environment variable
// AVEY_PLAN_BM = 16, 32 or 64), read once. It exists to measure the alternatives
// the table rejects with the same counters as its choices; a height that is not
// compiled for the row width (32 / 64 rows with more than 768 features) is ignored.
int forced_bm() {
  static const int bm = [] {
    const char* s = getenv("AVEY_PLAN_BM");
    const int v = s ? atoi(s) : 0;
    return (v == 16 || v == 32 || v == 64) ? v : 0;
  }();
  return bm;
}

bool device_ok(int dev) {
  if (dev < 0 || dev >= kMaxDevices) return false;
  int st = g_device_ok[dev].load(std::memory_order_relaxed);
  if (st == 0) {
    hipDeviceProp_t prop;
    st = 2;
    if (hipGetDeviceProperties(&prop, dev) == hipSuccess && strncmp(prop.gcnArchName, "gfx950", 6) == 0) st = 1;
    g_device_ok[dev].store(st, std::memory_order_relaxed);
  }
  return st == 1;
}

}  // namespace

// The static tile table (replaces the reference's runtime autotuner,
// avey_kernels/_triton.py:131-150). For the fused kernel:
//   * slice width DS = 32 * ceil(D / 128) features per wave (4 waves cover D);
//   * BM = 64 query rows up to DS = 192 (the key-slice ring and the partial
//     similarity tiles fit the 160 KB of LDS), else 16;
//   * BM halves (down to 16) while the grid would leave CUs of the 256 idle;
//   * waves per workgroup as fused_threads (avey_common.h) gives them.
// The fused kernel addresses memory with 16-byte row chunks and 32-bit buffer
// offsets, so it also needs D % 8 == 0, 16-byte aligned z_tr / z_tl / out, row
// and batch strides of z_tr / z_tl that are multiples of 8 elements, an 8-byte
// aligned bias, batch items spanning under 2^30 elements and C <= 32768 (V under
// 2 GiB); other shapes take the generic kernel.
Plan make_plan(const avey_fwd_args& a) {
  Plan pl{};
  const bool low = a.dtype == AVEY_DTYPE_BF16 || a.dtype == AVEY_DTYPE_F16;
  const int nk = slice_steps(a.features);
  const auto al = [](const void* x, uintptr_t n) { return x == nullptr || ((uintptr_t)x & (n - 1)) == 0; };
  const Strides zs = resolve(a.z_tr_row_stride, a.z_tr_batch_stride, a);
  const Strides gs = resolve(a.z_tl_row_stride, a.z_tl_batch_stride, a);
  const bool strides8 = zs.row % 8 == 0 && zs.batch % 8 == 0 && (a.z_tl == nullptr || (gs.row % 8 == 0 && gs.batch % 8 == 0));
  const bool layout = a.features % 8 == 0 && al(a.z_tr, 16) && al(a.z_tl, 16) && al(a.out, 16) && al(a.bias, 8) && strides8;
  const auto item = [&](const Strides& st) { return (a.context - 1) * st.row + a.features; };
  const bool small_item = item(zs) < (int64_t(1) << 30) && item(gs) < (int64_t(1) << 30) && a.context <= 32768 &&
                          a.batch < (int64_t(1) << 31);
  if (low && nk > 0 && layout && small_item) {
    pl.kernel = 1;
    pl.bn = 32;
    pl.bd = 32 * nk;
    // Row block: 64 rows up to 192 features per slice (768-feature rows), halved
    // while the grid would not cover the 256 CUs. Wider rows take the 16-row warp-
    // specialized variant: the 32-row one for 1024-feature rows keeps 4 waves (its
    // state does not fit 256 registers) and was 1.23x slower on B4 N2048 causal.
    int bm = nk <= 6 ? 64 : 16;
    while (bm > 16 && cdiv(a.context, bm) * a.batch < 256) bm /= 2;
    if (forced_bm() != 0 && (forced_bm() == 16 || nk <= 6)) bm = forced_bm();
    pl.bm = bm;
    pl.threads = fused_threads(bm, nk);
    const int64_t nqt = cdiv(a.context, bm);
    pl.grid = nqt * a.batch;
    pl.work_bytes = 0;
    int64_t steps = 0;
    for (int64_t qt = 0; qt < nqt; ++qt) steps += key_tiles_for(qt, a.context, bm, 32, a.causal != 0);
    pl.key_tile_steps = steps * a.batch;
  } else {
    pl.kernel = 2;
    pl.bm = 16;
    pl.bn = 16;
    pl.bd = 64;
    pl.threads = 256;
    const int64_t nqt = cdiv(a.context, 16);
    pl.grid = nqt * cdiv(a.features, 64) * a.batch;
    pl.work_bytes = a.batch * a.context * (a.dtype == AVEY_DTYPE_F64 ? 8 : 4);
    int64_t steps = 0;
    for (int64_t qt = 0; qt < nqt; ++qt) steps += key_tiles_for(qt, a.context, 16, 16, a.causal != 0);
    pl.key_tile_steps = steps * cdiv(a.features, 64) * a.batch;
  }
  return pl;
}

}  // namespace avey

using namespace avey;

namespace {
// Test helper: fills a workgroup's whole LDS (160 KB) with words that are NaN both
// as fp32 and as two bf16 / fp16 halves. A grid of 4 workgroups per CU, one at a
// time (the LDS holds one), leaves every CU's LDS poisoned.
constexpr int kPoisonWords = 160 * 1024 / 4;
__global__ __launch_bounds__(1024) void poison_lds_kernel() {
  __shared__ uint32_t buf[kPoisonWords];
  volatile uint32_t* v = buf;
  for (int i = threadIdx.x; i < kPoisonWords; i += 1024) v[i] = 0x7fc07fc0u;
}
}  // namespace

extern "C" {

int avey_debug_poison_lds(void* stream) {
  poison_lds_kernel<<<dim3(1024), dim3(1024), 0, (hipStream_t)stream>>>();
  return (int)hipGetLastError();
}

int avey_abi_version(void) { return AVEY_ABI_VERSION; }

const char* avey_status_string(int status) {
  switch (status) {
    case AVEY_OK: return "ok";
    case AVEY_ERR_NULL_POINTER: return "null pointer: args, z_tr and out are required";
    case AVEY_ERR_SHAPE: return "batch, context and features must be >= 1 and within the supported range";
    case AVEY_ERR_DTYPE: return "unknown dtype code";
    case AVEY_ERR_ACTIVATION: return "unknown activation id";
    case AVEY_ERR_EPS: return "eps and norm_eps must be finite and positive";
    case AVEY_ERR_WORKSPACE: return "workspace smaller than avey_fwd_workspace_bytes";
    case AVEY_ERR_DEVICE: return "current HIP device is not a gfx950 (MI355X) GPU";
    case AVEY_ERR_FLAGS: return "causal and normalize must be 0 or 1";
    case AVEY_ERR_ALIAS: return "out overlaps an input buffer";
    case AVEY_ERR_STRIDE: return "z_tr / z_tl row stride below features, or a negative stride";
    case AVEY_ERR_SCRATCH:
      return "the call needs more scratch than avey_fwd_noalloc holds (AVEY_NOALLOC_SCRATCH_BYTES)";
    case AVEY_ERR_ENRICHED:
      return "enriched forward: needs z_tl NULL, aligned x / w_gate (/ b_gate), model_dim a multiple of 8 in "
             "[8, 65536], a known gate activation and a call the fused bf16 / fp16 kernel covers";
    case AVEY_ERR_UNSUPPORTED:
      return "backward needs bf16 / fp16 / fp32, features <= 1024, batch <= 65535 and contiguous operands";
    default: return status > 0 ? hipGetErrorString((hipError_t)status) : "unknown status";
  }
}

int64_t avey_key_tile_count(int64_t query_tile, int64_t context, int32_t block_m, int32_t block_n, int32_t causal,
                            int32_t skip) {
  if (query_tile < 0 || context < 1 || block_m < 1 || block_n < 1) return -1;
  if (query_tile * (int64_t)block_m >= context) return -1;
  return key_tiles_for(query_tile, context, block_m, block_n, causal != 0 && skip != 0);
}

int64_t avey_fwd_workspace_bytes(const avey_fwd_args* args) {
  if (validate(args) != AVEY_OK) return -1;
  return make_plan(*args).work_bytes;
}

int avey_fwd_plan(const avey_fwd_args* args, avey_fwd_plan_t* out) {
  const int st = validate(args);
  if (st != AVEY_OK) return st;
  if (!out) return AVEY_ERR_NULL_POINTER;
  const Plan pl = make_plan(*args);
  out->kernel = pl.kernel;
  out->block_m = pl.bm;
  out->block_n = pl.bn;
  out->block_d = pl.bd;
  out->threads = pl.threads;
  out->waves_per_simd = pl.threads / 256;
  out->grid = pl.grid;
  out->workspace_bytes = pl.work_bytes;
  out->key_tile_steps = pl.key_tile_steps;
  return AVEY_OK;
}

int avey_device_supported(int device) { return device_ok(device) ? 1 : 0; }

namespace {
// Checks of avey_bwd's arguments; on success fills the kernel parameters.
int validate_bwd(const avey_bwd_args* a, BwdParams* p) {
  if (!a || !a->dout || !a->dz_tr) return AVEY_ERR_NULL_POINTER;
  avey_fwd_args f = a->fwd;
  f.out = a->dz_tr;  // the forward's checks, with dz_tr as the output that must not alias an input
  int st = validate(&f);
  if (st != AVEY_OK) return st;
  if (f.dtype == AVEY_DTYPE_F64 || f.features > kBwdMaxFeatures || f.batch > 65535 || f.z_tr_row_stride != 0 ||
      f.z_tl_row_stride != 0)
    return AVEY_ERR_UNSUPPORTED;
  const size_t es = elem_size(f.dtype);
  const size_t nb = (size_t)f.batch * (size_t)f.context * (size_t)f.features * es;
  const size_t vb = (size_t)f.context * (size_t)f.context * es;
  void* dv = f.v ? a->dv : nullptr;
  void* dg = f.z_tl ? a->dz_tl : nullptr;
  void* db = f.bias ? a->dbias : nullptr;
  const struct { const void* p; size_t n; } outs[] = {{a->dz_tr, nb}, {dv, vb}, {dg, nb}, {db, f.features * es}};
  const struct { const void* p; size_t n; } ins[] = {{f.z_tr, nb}, {f.v, vb}, {f.z_tl, nb}, {f.bias, f.features * es},
                                                     {f.valid, (size_t)f.batch * (size_t)f.context}, {a->dout, nb}};
  for (size_t i = 0; i < 4; ++i) {
    for (const auto& in : ins)
      if (overlaps(outs[i].p, outs[i].n, in.p, in.n)) return AVEY_ERR_ALIAS;
    for (size_t j = 0; j < i; ++j)
      if (overlaps(outs[i].p, outs[i].n, outs[j].p, outs[j].n)) return AVEY_ERR_ALIAS;
  }
  if (p) {
    *p = BwdParams{};
    p->z = f.z_tr;
    p->v = f.v;
    p->gate = f.z_tl;
    p->bias = f.bias;
    p->valid = f.valid;
    p->dout = a->dout;
    p->dz = a->dz_tr;
    p->dv = dv;
    p->dgate = dg;
    p->dbias = db;
    p->B = f.batch;
    p->C = f.context;
    p->D = f.features;
    p->causal = f.causal;
    p->normalize = f.normalize;
    p->act = f.activation;
    p->eps = f.eps;
    p->norm_eps = f.norm_eps;
  }
  return AVEY_OK;
}
}  // namespace

int64_t avey_bwd_workspace_bytes(const avey_bwd_args* args) {
  BwdParams p;
  const int st = validate_bwd(args, &p);
  if (st != AVEY_OK) return st;
  return bwd_workspace_bytes(p.B, p.C, p.D, p.dv != nullptr, p.dbias != nullptr,
                             bwd_path(args->fwd.dtype, p.D, p.z, p.normalize != 0));
}

int avey_bwd(const avey_bwd_args* a, void* workspace, size_t workspace_bytes, void* stream) {
  BwdParams p;
  const int st = validate_bwd(a, &p);
  if (st != AVEY_OK) return st;
  const size_t need = (size_t)bwd_workspace_bytes(p.B, p.C, p.D, p.dv != nullptr, p.dbias != nullptr,
                                                  bwd_path(a->fwd.dtype, p.D, p.z, p.normalize != 0));
  if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255) != 0) return AVEY_ERR_WORKSPACE;
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (!device_ok(dev)) return AVEY_ERR_DEVICE;
  p.work = workspace;
  e = launch_bwd(p, a->fwd.dtype, (hipStream_t)stream);
  return e == hipSuccess ? AVEY_OK : (int)e;
}

}  // extern "C"

namespace {
// Launches the planned kernels of a validated call with `work` as their scratch;
// with `en`, the 16-row fused kernel that forms the enricher gate.
int run_fwd(const avey_fwd_args* a, const Plan& pl, void* work, hipStream_t s,
            const avey_enriched_args* en = nullptr) {
  FwdParams p{};
  p.z = a->z_tr;
  p.v = a->v;
  p.gate = a->z_tl;
  p.bias = a->bias;
  p.valid = a->valid;
  p.out = a->out;
  p.work = work;
  p.B = a->batch;
  p.C = a->context;
  p.D = a->features;
  const Strides zs = resolve(a->z_tr_row_stride, a->z_tr_batch_stride, *a);
  const Strides gs = resolve(a->z_tl_row_stride, a->z_tl_batch_stride, *a);
  p.zrs = zs.row;
  p.zbs = zs.batch;
  p.grs = gs.row;
  p.gbs = gs.batch;
  p.causal = a->causal;
  p.normalize = a->normalize;
  p.act = a->activation;
  p.eps = a->eps;
  p.norm_eps = a->norm_eps;
  if (en) {
    p.xg = en->x;
    p.wg = en->w_gate;
    p.bg = en->b_gate;
    p.dm = en->model_dim;
    p.gact = en->gate_activation;
    const hipError_t e = launch_fused_enriched(p, a->dtype, pl, s);
    return e == hipSuccess ? AVEY_OK : (int)e;
  }
  const hipError_t e = pl.kernel == 1 ? launch_fused(p, a->dtype, pl, s) : launch_generic(p, a->dtype, pl, s);
  return e == hipSuccess ? AVEY_OK : (int)e;
}

// Checks of avey_fwd_enriched beyond validate(); fills the 16-row plan.
int validate_enriched(const avey_enriched_args* en, Plan* pl) {
  const avey_fwd_args& a = en->fwd;
  const auto al = [](const void* x, uintptr_t n) { return ((uintptr_t)x & (n - 1)) == 0; };
  if (a.z_tl || !en->x || !en->w_gate || !al(en->x, 16) || !al(en->w_gate, 16) || !al(en->b_gate, 8))
    return AVEY_ERR_ENRICHED;
  if (en->model_dim < 8 || en->model_dim > 65536 || en->model_dim % 8 != 0) return AVEY_ERR_ENRICHED;
  if (en->gate_activation < AVEY_ACT_IDENTITY || en->gate_activation > AVEY_ACT_GELU) return AVEY_ERR_ENRICHED;
  *pl = make_plan(a);
  if (pl->kernel != 1) return AVEY_ERR_ENRICHED;
  // Every row block of 16: only the 16-row variant forms the gate.
  pl->bm = 16;
  pl->threads = fused_threads(16, pl->bd / 32);
  const int64_t nqt = cdiv(a.context, 16);
  pl->grid = nqt * a.batch;
  int64_t steps = 0;
  for (int64_t qt = 0; qt < nqt; ++qt) steps += key_tiles_for(qt, a.context, 16, 32, a.causal != 0);
  pl->key_tile_steps = steps * a.batch;
  const size_t es = elem_size(a.dtype);
  const size_t nb = (size_t)a.batch * (size_t)a.context * (size_t)a.features * es;
  const size_t xb = (size_t)a.batch * (size_t)a.context * (size_t)en->model_dim * es;
  const size_t wb = (size_t)a.features * (size_t)en->model_dim * es;
  if (overlaps(a.out, nb, en->x, xb) || overlaps(a.out, nb, en->w_gate, wb) ||
      overlaps(a.out, nb, en->b_gate, (size_t)a.features * es))
    return AVEY_ERR_ALIAS;
  return AVEY_OK;
}

// The current device, checked to be a gfx950 GPU.
int current_device(int* dev) {
  const hipError_t e = hipGetDevice(dev);
  if (e != hipSuccess) return (int)e;
  return device_ok(*dev) ? AVEY_OK : AVEY_ERR_DEVICE;
}
}  // namespace

extern "C" {

int avey_fwd(const avey_fwd_args* a, void* workspace, size_t workspace_bytes, void* stream) {
  const int st = validate(a);
  if (st != AVEY_OK) return st;
  const Plan pl = make_plan(*a);
  if (pl.work_bytes > 0 && (!workspace || workspace_bytes < (size_t)pl.work_bytes)) return AVEY_ERR_WORKSPACE;
  int dev = -1;
  const int ds = current_device(&dev);
  if (ds != AVEY_OK) return ds;
  return run_fwd(a, pl, workspace, (hipStream_t)stream);
}

int avey_fwd_enriched(const avey_enriched_args* en, void* stream) {
  if (!en) return AVEY_ERR_NULL_POINTER;
  const int st = validate(&en->fwd);
  if (st != AVEY_OK) return st;
  Plan pl;
  const int se = validate_enriched(en, &pl);
  if (se != AVEY_OK) return se;
  int dev = -1;
  const int ds = current_device(&dev);
  if (ds != AVEY_OK) return ds;
  return run_fwd(&en->fwd, pl, nullptr, (hipStream_t)stream, en);
}

int avey_fwd_noalloc(const avey_fwd_args* a, void* stream) {
  const int st = validate(a);
  if (st != AVEY_OK) return st;
  const Plan pl = make_plan(*a);
  if (pl.work_bytes > (int64_t)AVEY_NOALLOC_SCRATCH_BYTES) return AVEY_ERR_SCRATCH;
  int dev = -1;
  const int ds = current_device(&dev);
  if (ds != AVEY_OK) return ds;
  // The first call on a device looks up that device's copy of the scratch array.
  void* work = nullptr;
  const hipError_t e = device_scratch(dev, &work);
  if (e != hipSuccess) return (int)e;
  return run_fwd(a, pl, work, (hipStream_t)stream);
}

}  // extern "C"
