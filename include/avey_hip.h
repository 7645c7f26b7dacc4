/*
 * avey_hip.h -- C ABI of libavey_hip.so, the MI355X (gfx950) forward
 * contextualizer for Avey and Avey-B.
 *
 * The library replaces the reference's device path for this op
 * (HusamettinYilmazz/avey_kernel):
 *   - avey_fwd            replaces the custom op `mix` and its launch of the
 *                         Triton kernel `_mix_kernel` (avey_kernels/_triton.py:153-188,
 *                         kernel at :53-128) together with the separate
 *                         F.normalize pass in `_dispatch` (avey_kernels/ops.py:107-108):
 *                         one call computes out = gate * act(mix / den + bias).
 *   - avey_fwd_plan       replaces the Triton autotuner and its 84-entry
 *                         candidate table (avey_kernels/_triton.py:131-150) with a
 *                         static, documented tile table; host-only, no GPU needed.
 *   - avey_key_tile_count replaces `_key_tile_count` (avey_kernels/_triton.py:38-50),
 *                         the causal tile-skip rule; host-only.
 *   - avey_fwd_noalloc    avey_fwd without allocation; no reference counterpart
 *                         (for callers that cannot allocate device memory).
 *   - avey_fwd_enriched   avey_fwd with the enricher's gate half fused: replaces the
 *                         caller's enricher GEMM for z_tl and the z_tl tensor the op
 *                         receives (the static layers around the op, ops.py:4-7;
 *                         the reference takes z_tl as stored, ops.py:109-113).
 *   - avey_bwd            replaces autograd over the eager path for the
 *                         gradients (avey_kernels/ops.py:96-106 and :61-91).
 *   - avey_fwd_workspace_bytes, avey_bwd_workspace_bytes, avey_status_string, avey_abi_version,
 *     avey_device_supported: plumbing for the Python binding
 *     (avey_kernel_amd/_hip.py), no reference counterpart beyond the op's
 *     argument checks (avey_kernels/_triton.py:165-166).
 *
 * Conventions
 *   - All tensor pointers are device pointers owned by the caller. The
 *     library never allocates, frees or keeps pointers after a call returns.
 *   - z_tr, z_tl, out: [batch][context][features], features contiguous.
 *     z_tr and z_tl may be strided views (row and batch strides in the
 *     arguments; e.g. the two halves of the enricher output, which the
 *     reference copies with .contiguous(), ops.py:109-113); out is contiguous.
 *     v: [context][context] indexed [query][key], shared by the batch.
 *     bias: [features]. valid: [batch][context] bytes (0 = padded row).
 *     z_tr, z_tl, v, bias and out share one element type (ops.py:39-43).
 *   - Launches are asynchronous on the caller's HIP stream; no host sync.
 *   - Errors are returned as status codes; nothing throws or aborts across
 *     the ABI. Negative = invalid argument, positive = hipError_t value.
 */
#ifndef AVEY_HIP_H
#define AVEY_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AVEY_ABI_VERSION 5

/* Element type of z_tr / z_tl / v / bias / out. */
enum avey_dtype {
  AVEY_DTYPE_F32 = 0,
  AVEY_DTYPE_F16 = 1,
  AVEY_DTYPE_BF16 = 2,
  AVEY_DTYPE_F64 = 3,
};

/* Activation ids, same numbering as the reference's kernel (avey_kernels/_triton.py:169). */
enum avey_activation {
  AVEY_ACT_IDENTITY = 0,
  AVEY_ACT_RELU = 1,
  AVEY_ACT_RELU2 = 2,
  AVEY_ACT_SILU = 3,
  AVEY_ACT_GELU = 4, /* tanh approximation, ops.py:57 */
};

enum avey_status {
  AVEY_OK = 0,
  AVEY_ERR_NULL_POINTER = -1,     /* args, z_tr or out is NULL */
  AVEY_ERR_SHAPE = -2,            /* batch, context or features < 1, or too large */
  AVEY_ERR_DTYPE = -3,            /* unknown dtype code */
  AVEY_ERR_ACTIVATION = -4,       /* unknown activation id */
  AVEY_ERR_EPS = -5,              /* eps or norm_eps not finite and > 0 */
  AVEY_ERR_WORKSPACE = -6,        /* workspace smaller than avey_fwd_workspace_bytes */
  AVEY_ERR_DEVICE = -7,           /* current device is not gfx950 */
  AVEY_ERR_FLAGS = -8,            /* causal / normalize not 0 or 1 */
  AVEY_ERR_ALIAS = -9,            /* out overlaps an input */
  AVEY_ERR_STRIDE = -10,          /* a row stride below features, or a negative stride */
  AVEY_ERR_UNSUPPORTED = -11,     /* backward: fp64, features > 1024, batch > 65535 or strided operands */
  AVEY_ERR_SCRATCH = -12,         /* avey_fwd_noalloc: the call needs more than AVEY_NOALLOC_SCRATCH_BYTES */
  AVEY_ERR_ENRICHED = -13,        /* avey_fwd_enriched: see avey_enriched_args */
};

typedef struct avey_fwd_args {
  const void* z_tr;     /* required */
  const void* v;        /* optional (NULL: no learned weights, Avey-B) */
  const void* z_tl;     /* optional gate */
  const void* bias;     /* optional */
  const uint8_t* valid; /* optional key/query padding mask */
  void* out;            /* required */
  int64_t batch;
  int64_t context;      /* C: tokens (query and key positions) */
  int64_t features;     /* d': feature width */
  int32_t dtype;        /* enum avey_dtype */
  int32_t causal;       /* 1: keys j <= query i only (diagonal kept) */
  int32_t normalize;    /* 1: divide by the signed row sum + eps (Avey-B) */
  int32_t activation;   /* enum avey_activation */
  double eps;           /* denominator epsilon (used when normalize = 1) */
  double norm_eps;      /* F.normalize clamp of the row norm */
  /* Strides of z_tr and z_tl in elements (ABI 2). A row stride of 0 means
   * contiguous (row stride = features, batch stride = context * features) and
   * the batch stride is then ignored; otherwise the row stride must be at least
   * `features` and the batch stride is used as given (>= 0). The fused MFMA
   * kernel needs both strides to be multiples of 8 (16-byte rows); other
   * strides take the generic kernel. */
  int64_t z_tr_row_stride;
  int64_t z_tr_batch_stride;
  int64_t z_tl_row_stride;
  int64_t z_tl_batch_stride;
} avey_fwd_args;

/* Arguments of the backward (ABI 3). `fwd` holds the forward call's inputs and
 * flags; fwd.out is ignored, and z_tr / z_tl must be contiguous (strides 0).
 * dout and every gradient share fwd.dtype and the shape of their input. */
typedef struct avey_bwd_args {
  avey_fwd_args fwd;
  const void* dout;     /* required: gradient of out, [batch][context][features] */
  void* dz_tr;          /* required */
  void* dv;             /* optional: [context][context]; NULL or fwd.v NULL: not computed */
  void* dz_tl;          /* optional: NULL or fwd.z_tl NULL: not computed */
  void* dbias;          /* optional: [features]; NULL or fwd.bias NULL: not computed */
} avey_bwd_args;

/* Kernel choice and launch geometry for one call; filled by avey_fwd_plan. */
typedef struct avey_fwd_plan_t {
  int32_t kernel;        /* 1 = fused MFMA (bf16/fp16), 2 = generic VALU (fp32/fp64/wide) */
  int32_t block_m;       /* query rows per workgroup */
  int32_t block_n;       /* key rows per pipeline step */
  int32_t block_d;       /* features per output tile (generic) or per wave slice (MFMA) */
  int32_t threads;       /* threads per workgroup */
  int32_t waves_per_simd;
  int64_t grid;          /* workgroups launched by the main kernel */
  int64_t workspace_bytes;
  int64_t key_tile_steps;   /* sum over workgroups of key tiles visited */
} avey_fwd_plan_t;

/* Launch the forward contextualizer on `stream` (a hipStream_t; NULL = default stream). */
int avey_fwd(const avey_fwd_args* args, void* workspace, size_t workspace_bytes, void* stream);

/* The forward without allocation (ABI 4). No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP-graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). Same arguments, kernels
 * and results as avey_fwd; the scratch the kernels need (the generic fp32 / fp64
 * kernel's per-row inverse norms, 4 or 8 bytes per batch x context row; the fused
 * bf16 / fp16 kernels need none) comes from a static device array of
 * AVEY_NOALLOC_SCRATCH_BYTES that each GPU holds until the process ends. It calls
 * no hipMalloc / hipFree. Larger needs return AVEY_ERR_SCRATCH. Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU (other streams, other
 * host threads) race and must be serialised by the caller. */
#define AVEY_NOALLOC_SCRATCH_BYTES (4u << 20)
int avey_fwd_noalloc(const avey_fwd_args* args, void* stream);
/* The forward with the enricher's gate half fused (ABI 5). In Avey the enricher
 * z = act_e(x W_e^T + b_e) produces the op's two inputs as halves of its tail,
 * z_tl and z_tr. Here the caller still computes z_tr (every row block reads all of
 * it as keys); z_tl = gate_activation(x w_gate^T + b_gate) is formed for each block of
 * 16 query rows inside the fused kernel and never stored, which saves the enricher
 * writing it and the op reading it (2 * batch * context * features elements).
 * Requirements (else AVEY_ERR_ENRICHED): fwd.z_tl NULL; x and w_gate non-NULL and
 * 16-byte aligned, b_gate NULL or 8-byte aligned, all of fwd.dtype; model_dim a
 * multiple of 8 in [8, 65536]; gate_activation an avey_activation id; and a call the
 * fused kernel covers (bf16 / fp16, features <= 1024 and a multiple of 8, the
 * layout rules of avey_fwd_plan). Needs no workspace. */
typedef struct avey_enriched_args {
  avey_fwd_args fwd;       /* as for avey_fwd, with z_tl NULL */
  const void* x;           /* [batch][context][model_dim], contiguous: the enricher's input */
  const void* w_gate;      /* [features][model_dim]: the enricher weight rows of z_tl */
  const void* b_gate;      /* [features] or NULL: their bias */
  int64_t model_dim;
  int32_t gate_activation; /* enum avey_activation, the enricher's activation */
} avey_enriched_args;
int avey_fwd_enriched(const avey_enriched_args* args, void* stream);

/* Device scratch bytes avey_fwd needs for these arguments (0 when none). Host-only. */
int64_t avey_fwd_workspace_bytes(const avey_fwd_args* args);

/* Describe the launch avey_fwd would make, without touching a GPU. Returns a status. */
int avey_fwd_plan(const avey_fwd_args* args, avey_fwd_plan_t* plan);

/* Key tiles visited by query tile `query_tile` (the causal skip rule keeps the
 * diagonal tile). Host-only. Returns -1 on invalid input. */
int64_t avey_key_tile_count(int64_t query_tile, int64_t context, int32_t block_m, int32_t block_n,
                            int32_t causal, int32_t skip);

/* Gradients of the forward w.r.t. z_tr, v, z_tl and bias on `stream`. Replaces
 * the reference's backward, which is PyTorch autograd over the eager path
 * (avey_kernels/ops.py:96-106 selects it whenever an input requires grad; the
 * math is ops.py:61-91) and materialises [batch, context, context] tensors; this
 * one stores no context x context tile except the fp32 dv accumulator. bf16,
 * fp16 and fp32; features <= 1024. Arithmetic in fp32. The workspace holds
 * avey_bwd_workspace_bytes bytes; dv and dbias are summed with atomics, so their
 * low bits may differ from call to call. */
int avey_bwd(const avey_bwd_args* args, void* workspace, size_t workspace_bytes, void* stream);

/* Device scratch bytes avey_bwd needs for these arguments, or a negative status. Host-only. */
int64_t avey_bwd_workspace_bytes(const avey_bwd_args* args);

/* 1 if `device` is a gfx950 GPU this library can run on, else 0. */
int avey_device_supported(int device);

const char* avey_status_string(int status);
int avey_abi_version(void);

/* Test helper, no reference counterpart: fills the LDS of every CU with NaN bit
 * patterns (fp32 and 16-bit alike) on `stream` (a hipStream_t; NULL: the null
 * stream), so that a test can show a kernel's results do not depend on LDS it did
 * not write. Returns a HIP status (0 on success). */
int avey_debug_poison_lds(void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AVEY_HIP_H */
