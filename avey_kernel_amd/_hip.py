"""ctypes binding of libavey_hip.so and the ``avey_kernels::contextualize`` op.

The op is functional: it allocates and returns a fresh output, as the
reference's ``avey_kernels::mix`` does (``avey_kernels/_triton.py:153-188``),
and has a fake implementation so fake-tensor tracing and
``torch.compile(fullgraph=True)`` see an opaque call. Unlike ``mix`` it takes
the raw ``z_tr`` only: row normalisation happens inside the fused kernel. z_tr
and z_tl may be strided views whose last dimension is contiguous (e.g. the two
halves of the enricher output): their row and batch strides go to the library
instead of a copy (the reference copies them, ``avey_kernels/ops.py:109-113``).

Its gradient is ``avey_kernels::contextualize_backward``, the library's fused
backward (the reference differentiates its eager path with autograd instead,
``avey_kernels/ops.py:96-106``).

Nothing here falls back to another implementation: if the shared library is
missing or refuses the call, the error surfaces to the caller.
"""

import ctypes
import os
from typing import Optional

import torch

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'libavey_hip.so')

DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.float64: 3}
ACTIVATION_IDS = {'identity': 0, 'relu': 1, 'relu2': 2, 'silu': 3, 'gelu': 4}
KERNEL_NAMES = {1: 'fused_mfma', 2: 'generic_valu'}


class HipUnavailable(RuntimeError):
    """libavey_hip.so is missing or cannot be loaded."""


class AveyFwdArgs(ctypes.Structure):
    _fields_ = [
        ('z_tr', ctypes.c_void_p), ('v', ctypes.c_void_p), ('z_tl', ctypes.c_void_p),
        ('bias', ctypes.c_void_p), ('valid', ctypes.c_void_p), ('out', ctypes.c_void_p),
        ('batch', ctypes.c_int64), ('context', ctypes.c_int64), ('features', ctypes.c_int64),
        ('dtype', ctypes.c_int32), ('causal', ctypes.c_int32), ('normalize', ctypes.c_int32),
        ('activation', ctypes.c_int32), ('eps', ctypes.c_double), ('norm_eps', ctypes.c_double),
        ('z_tr_row_stride', ctypes.c_int64), ('z_tr_batch_stride', ctypes.c_int64),
        ('z_tl_row_stride', ctypes.c_int64), ('z_tl_batch_stride', ctypes.c_int64),
    ]


class AveyBwdArgs(ctypes.Structure):
    _fields_ = [
        ('fwd', AveyFwdArgs), ('dout', ctypes.c_void_p), ('dz_tr', ctypes.c_void_p), ('dv', ctypes.c_void_p),
        ('dz_tl', ctypes.c_void_p), ('dbias', ctypes.c_void_p),
    ]


class AveyEnrichedArgs(ctypes.Structure):
    _fields_ = [
        ('fwd', AveyFwdArgs), ('x', ctypes.c_void_p), ('w_gate', ctypes.c_void_p), ('b_gate', ctypes.c_void_p),
        ('model_dim', ctypes.c_int64), ('gate_activation', ctypes.c_int32),
    ]


class AveyFwdPlan(ctypes.Structure):
    _fields_ = [
        ('kernel', ctypes.c_int32), ('block_m', ctypes.c_int32), ('block_n', ctypes.c_int32),
        ('block_d', ctypes.c_int32), ('threads', ctypes.c_int32), ('waves_per_simd', ctypes.c_int32),
        ('grid', ctypes.c_int64), ('workspace_bytes', ctypes.c_int64), ('key_tile_steps', ctypes.c_int64),
    ]


# Symbols of include/avey_hip.h with their ctypes signatures.
EXPORTS = {
    'avey_fwd': (ctypes.c_int, [ctypes.POINTER(AveyFwdArgs), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    'avey_fwd_noalloc': (ctypes.c_int, [ctypes.POINTER(AveyFwdArgs), ctypes.c_void_p]),
    'avey_fwd_enriched': (ctypes.c_int, [ctypes.POINTER(AveyEnrichedArgs), ctypes.c_void_p]),
    'avey_fwd_workspace_bytes': (ctypes.c_int64, [ctypes.POINTER(AveyFwdArgs)]),
    'avey_fwd_plan': (ctypes.c_int, [ctypes.POINTER(AveyFwdArgs), ctypes.POINTER(AveyFwdPlan)]),
    'avey_key_tile_count': (ctypes.c_int64, [ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                             ctypes.c_int32, ctypes.c_int32]),
    'avey_bwd': (ctypes.c_int, [ctypes.POINTER(AveyBwdArgs), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    'avey_bwd_workspace_bytes': (ctypes.c_int64, [ctypes.POINTER(AveyBwdArgs)]),
    'avey_device_supported': (ctypes.c_int, [ctypes.c_int]),
    'avey_status_string': (ctypes.c_char_p, [ctypes.c_int]),
    'avey_abi_version': (ctypes.c_int, []),
    'avey_debug_poison_lds': (ctypes.c_int, [ctypes.c_void_p]),
}
ABI_VERSION = 5
NOALLOC_SCRATCH_BYTES = 4 << 20  # AVEY_NOALLOC_SCRATCH_BYTES of include/avey_hip.h

_lib = None


def library_path():
    return _LIB_PATH


def load():
    """Load libavey_hip.so once; raise HipUnavailable if it is absent or stale."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        raise HipUnavailable(f'{_LIB_PATH} is not built; run `python -m avey_kernel_amd._build`')
    try:
        lib = ctypes.CDLL(_LIB_PATH)
    except OSError as exc:
        raise HipUnavailable(f'cannot load {_LIB_PATH}: {exc}') from exc
    for name, (restype, argtypes) in EXPORTS.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if lib.avey_abi_version() != ABI_VERSION:
        raise HipUnavailable(f'{_LIB_PATH} has ABI {lib.avey_abi_version()}, expected {ABI_VERSION}')
    _lib = lib
    return lib


def status_string(code):
    return load().avey_status_string(code).decode()


def _ptr(t):
    return None if t is None else t.data_ptr()


def readable_in_place(t):
    """Whether the library can read a [B, C, D] operand at its own strides: the
    features contiguous and the rows of a batch item apart by at least D elements
    (a broadcast row stride of 0, or rows that overlap, need a contiguous copy; the
    C ABI reads a row stride of 0 as "contiguous"). Dimensions of size 1 have no
    meaningful stride and are not checked."""
    batch, context, features = t.shape
    if t.is_contiguous():
        return True
    return (features == 1 or t.stride(2) == 1) and (context == 1 or t.stride(1) >= features) \
        and (batch == 1 or t.stride(0) >= 0)


def row_strides(t):
    """(row stride, batch stride) in elements of a [B, C, D] operand the library
    reads in place; (0, 0) for a contiguous tensor or None. Size-1 dimensions get
    the strides of a contiguous layout."""
    if t is None or t.is_contiguous():
        return 0, 0
    if not readable_in_place(t):
        raise ValueError('z_tr / z_tl need contiguous features and rows at least D elements apart')
    batch, context, features = t.shape
    row = t.stride(1) if context > 1 else features
    return row, (t.stride(0) if batch > 1 else context * row)


def make_args(z_tr, v, z_tl, bias, valid, out, eps, norm_eps, causal, normalize, activation):
    batch, context, features = z_tr.shape
    return AveyFwdArgs(
        _ptr(z_tr), _ptr(v), _ptr(z_tl), _ptr(bias), _ptr(valid), _ptr(out),
        batch, context, features, DTYPE_CODES[z_tr.dtype], int(bool(causal)), int(bool(normalize)),
        ACTIVATION_IDS[activation], float(eps), float(norm_eps), *row_strides(z_tr), *row_strides(z_tl))


def plan(shape, dtype, *, causal, normalize, activation='identity', eps=1e-6, norm_eps=1e-12,
         has_v=False, has_gate=False, has_bias=False, has_valid=False, z_tr_strides=(0, 0),
         z_tl_strides=(0, 0)):
    """Static tile-table entry for a call, computed on the host (no GPU needed).
    Strides are (row, batch) in elements; (0, 0) means contiguous."""
    batch, context, features = shape
    # Distinct non-null placeholders: the plan never dereferences pointers.
    base = 1 << 40
    step = 1 << 36
    args = AveyFwdArgs(base, base + step if has_v else None, base + 2 * step if has_gate else None,
                       base + 3 * step if has_bias else None, base + 4 * step if has_valid else None,
                       base + 5 * step, batch, context, features, DTYPE_CODES[dtype], int(causal),
                       int(normalize), ACTIVATION_IDS[activation], float(eps), float(norm_eps),
                       *z_tr_strides, *z_tl_strides)
    out = AveyFwdPlan()
    st = load().avey_fwd_plan(ctypes.byref(args), ctypes.byref(out))
    if st != 0:
        raise ValueError(status_string(st))
    return {
        'kernel': KERNEL_NAMES.get(out.kernel, str(out.kernel)), 'block_m': out.block_m,
        'block_n': out.block_n, 'block_d': out.block_d, 'threads': out.threads, 'grid': out.grid,
        'workspace_bytes': out.workspace_bytes, 'key_tile_steps': out.key_tile_steps,
    }


def device_supported(device):
    """True if ``device`` (a CUDA/ROCm torch device) is a gfx950 GPU."""
    idx = torch.device(device).index
    if idx is None:
        idx = torch.cuda.current_device()
    return bool(load().avey_device_supported(idx))


def launch(z_tr, v, z_tl, bias, valid, out, eps, norm_eps, causal, normalize, activation):
    """Launch the forward pass into ``out`` on the current stream of z_tr's device."""
    lib = load()
    valid_u8 = valid.view(torch.uint8) if valid is not None else None
    args = make_args(z_tr, v, z_tl, bias, valid_u8, out, eps, norm_eps, causal, normalize, activation)
    need = lib.avey_fwd_workspace_bytes(ctypes.byref(args))
    if need < 0:
        raise ValueError('libavey_hip rejected the arguments')
    work = torch.empty(max(int(need), 1), dtype=torch.uint8, device=z_tr.device) if need > 0 else None
    with torch.cuda.device(z_tr.device):
        stream = torch.cuda.current_stream(z_tr.device).cuda_stream
        st = lib.avey_fwd(ctypes.byref(args), _ptr(work), int(need), stream)
    if st < 0:
        raise ValueError(f'avey_fwd: {status_string(st)}')
    if st > 0:
        raise RuntimeError(f'avey_fwd: HIP error {st}: {status_string(st)}')
    return out


def enriched_supported(x, z_tr, w_gate):
    """True when avey_fwd_enriched covers the call (checked on the host; the library
    checks again and reports a status otherwise)."""
    batch, context, features = z_tr.shape
    d = x.shape[-1]
    return (z_tr.dtype in (torch.bfloat16, torch.float16) and x.dtype == z_tr.dtype
            and w_gate.dtype == z_tr.dtype and features % 8 == 0 and features <= 1024
            and d % 8 == 0 and 8 <= d <= 65536)


def launch_enriched(x, w_gate, b_gate, z_tr, v, bias, valid, out, eps, norm_eps, causal, normalize, activation,
                    gate_activation):
    """avey_fwd_enriched into ``out`` on the current stream of z_tr's device."""
    lib = load()
    valid_u8 = valid.view(torch.uint8) if valid is not None else None
    fwd = make_args(z_tr, v, None, bias, valid_u8, out, eps, norm_eps, causal, normalize, activation)
    args = AveyEnrichedArgs(fwd, _ptr(x), _ptr(w_gate), _ptr(b_gate), x.shape[-1],
                            ACTIVATION_IDS[gate_activation])
    with torch.cuda.device(z_tr.device):
        stream = torch.cuda.current_stream(z_tr.device).cuda_stream
        st = lib.avey_fwd_enriched(ctypes.byref(args), stream)
    if st < 0:
        raise ValueError(f'avey_fwd_enriched: {status_string(st)}')
    if st > 0:
        raise RuntimeError(f'avey_fwd_enriched: HIP error {st}: {status_string(st)}')
    return out


@torch.library.custom_op('avey_kernels::contextualize_enriched', mutates_args=())
def contextualize_enriched(x: torch.Tensor, w_gate: torch.Tensor, b_gate: Optional[torch.Tensor],
                           z_tr: torch.Tensor, v: Optional[torch.Tensor], bias: Optional[torch.Tensor],
                           valid: Optional[torch.Tensor], eps: float, norm_eps: float, causal: bool,
                           normalize: bool, activation: str, gate_activation: str) -> torch.Tensor:
    """contextualize with z_tl = gate_activation(x w_gate^T + b_gate) formed inside the
    fused kernel (never stored). Forward only; x, w_gate, b_gate are made contiguous."""
    z_tr = z_tr if readable_in_place(z_tr) else z_tr.contiguous()
    x, w_gate = x.contiguous(), w_gate.contiguous()
    b_gate, v, bias, valid = (None if t is None else t.contiguous() for t in (b_gate, v, bias, valid))
    out = torch.empty_like(z_tr, memory_format=torch.contiguous_format)
    return launch_enriched(x, w_gate, b_gate, z_tr, v, bias, valid, out, eps, norm_eps, causal, normalize,
                           activation, gate_activation)


@contextualize_enriched.register_fake
def _contextualize_enriched_fake(x, w_gate, b_gate, z_tr, v, bias, valid, eps, norm_eps, causal, normalize,
                                 activation, gate_activation):
    return torch.empty_like(z_tr, memory_format=torch.contiguous_format)


@torch.library.custom_op('avey_kernels::contextualize', mutates_args=())
def contextualize(z_tr: torch.Tensor, v: Optional[torch.Tensor], z_tl: Optional[torch.Tensor],
                  bias: Optional[torch.Tensor], valid: Optional[torch.Tensor], eps: float,
                  norm_eps: float, causal: bool, normalize: bool, activation: str) -> torch.Tensor:
    """out = z_tl * act(mix(z_tr) / den + bias), fused on the GPU. z_tr and z_tl may be
    strided views with a contiguous last dimension; out is contiguous."""
    # Callers such as Inductor hand over whatever layouts their graph chose: views
    # the library reads in place go through as they are, anything else is made so.
    z_tr = z_tr if readable_in_place(z_tr) else z_tr.contiguous()
    if z_tl is not None and not readable_in_place(z_tl):
        z_tl = z_tl.contiguous()
    v, bias, valid = (None if t is None else t.contiguous() for t in (v, bias, valid))
    out = torch.empty_like(z_tr, memory_format=torch.contiguous_format)
    return launch(z_tr, v, z_tl, bias, valid, out, eps, norm_eps, causal, normalize, activation)


@contextualize.register_fake
def _contextualize_fake(z_tr, v, z_tl, bias, valid, eps, norm_eps, causal, normalize, activation):
    return torch.empty_like(z_tr, memory_format=torch.contiguous_format)


# Limits of the fused backward (avey_bwd); other inputs take autograd over the eager path.
BWD_DTYPES = (torch.bfloat16, torch.float16, torch.float32)
BWD_MAX_FEATURES = 1024
BWD_MAX_BATCH = 65535


def backward_supported(z_tr):
    """True when avey_bwd covers gradients of a call on ``z_tr`` (dtype and shape only)."""
    return (z_tr.dtype in BWD_DTYPES and z_tr.shape[2] <= BWD_MAX_FEATURES
            and z_tr.shape[0] <= BWD_MAX_BATCH)


def launch_backward(dout, z_tr, v, z_tl, bias, valid, dz_tr, dv, dz_tl, dbias, eps, norm_eps, causal,
                    normalize, activation):
    """Launch the backward into the given gradient buffers (None: not computed) on
    the current stream of z_tr's device. Every [B, C, D] operand is contiguous."""
    lib = load()
    valid_u8 = valid.view(torch.uint8) if valid is not None else None
    fwd = make_args(z_tr, v, z_tl, bias, valid_u8, None, eps, norm_eps, causal, normalize, activation)
    args = AveyBwdArgs(fwd, _ptr(dout), _ptr(dz_tr), _ptr(dv), _ptr(dz_tl), _ptr(dbias))
    need = lib.avey_bwd_workspace_bytes(ctypes.byref(args))
    if need < 0:
        raise ValueError(f'avey_bwd: {status_string(int(need))}')
    work = torch.empty(int(need), dtype=torch.uint8, device=z_tr.device)
    with torch.cuda.device(z_tr.device):
        stream = torch.cuda.current_stream(z_tr.device).cuda_stream
        st = lib.avey_bwd(ctypes.byref(args), _ptr(work), int(need), stream)
    if st < 0:
        raise ValueError(f'avey_bwd: {status_string(st)}')
    if st > 0:
        raise RuntimeError(f'avey_bwd: HIP error {st}: {status_string(st)}')


def _nothing(t):
    return t.new_empty((0,))


@torch.library.custom_op('avey_kernels::contextualize_backward', mutates_args=())
def contextualize_backward(dout: torch.Tensor, z_tr: torch.Tensor, v: Optional[torch.Tensor],
                           z_tl: Optional[torch.Tensor], bias: Optional[torch.Tensor],
                           valid: Optional[torch.Tensor], eps: float, norm_eps: float, causal: bool,
                           normalize: bool, activation: str, need_v: bool, need_z_tl: bool,
                           need_bias: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dz_tr, dv, dz_tl, dbias) of ``contextualize``; a gradient that is not
    needed (or whose input is absent) comes back as an empty tensor."""
    z_tr, dout = z_tr.contiguous(), dout.contiguous()
    z_tl = z_tl.contiguous() if z_tl is not None else None
    v, bias, valid = (None if t is None else t.contiguous() for t in (v, bias, valid))
    dz_tr = torch.empty_like(z_tr)
    dv = torch.empty_like(v) if (v is not None and need_v) else None
    dz_tl = torch.empty_like(z_tl) if (z_tl is not None and need_z_tl) else None
    dbias = torch.empty_like(bias) if (bias is not None and need_bias) else None
    launch_backward(dout, z_tr, v, z_tl, bias, valid, dz_tr, dv, dz_tl, dbias, eps, norm_eps, causal,
                    normalize, activation)
    return (dz_tr, _nothing(z_tr) if dv is None else dv, _nothing(z_tr) if dz_tl is None else dz_tl,
            _nothing(z_tr) if dbias is None else dbias)


@contextualize_backward.register_fake
def _contextualize_backward_fake(dout, z_tr, v, z_tl, bias, valid, eps, norm_eps, causal, normalize, activation,
                                 need_v, need_z_tl, need_bias):
    def grad_like(t, need):
        return torch.empty_like(t, memory_format=torch.contiguous_format) if (t is not None and need) \
            else z_tr.new_empty((0,))
    return (torch.empty_like(z_tr, memory_format=torch.contiguous_format), grad_like(v, need_v),
            grad_like(z_tl, need_z_tl), grad_like(bias, need_bias))


def _setup_context(ctx, inputs, output):
    z_tr, v, z_tl, bias, valid, eps, norm_eps, causal, normalize, activation = inputs
    ctx.save_for_backward(z_tr, v, z_tl, bias, valid)
    ctx.flags = (eps, norm_eps, causal, normalize, activation)


def _backward(ctx, grad):
    z_tr, v, z_tl, bias, valid = ctx.saved_tensors
    need = ctx.needs_input_grad
    dz_tr, dv, dz_tl, dbias = torch.ops.avey_kernels.contextualize_backward(
        grad, z_tr, v, z_tl, bias, valid, *ctx.flags, bool(need[1]), bool(need[2]), bool(need[3]))
    return (dz_tr if need[0] else None, dv if (v is not None and need[1]) else None,
            dz_tl if (z_tl is not None and need[2]) else None,
            dbias if (bias is not None and need[3]) else None, None, None, None, None, None, None)


contextualize.register_autograd(_backward, setup_context=_setup_context)
