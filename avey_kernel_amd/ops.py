"""Avey / Avey-B forward contextualizer: public entry points (MI355X build).

Drop-in for ``avey_kernels.ops`` of HusamettinYilmazz/avey_kernel: ``avey`` and
``avey_b`` keep the reference's positional/keyword layout, defaults, input
contract (the same ``ValueError`` conditions, ``avey_kernels/ops.py:23-46``) and
output dtype (``ops.py:91``). Notation follows the reference: ``z_tr`` is
Z_tr [batch, C, d'], ``z_tl`` the gate Z_tl, ``v`` the learned [query, key]
weights V shared across the batch (``ops.py:1-7``).

Backends (``backend=``):

* ``'auto'``   the fused HIP kernel for ROCm tensors on a gfx950 GPU, with the
  fused HIP backward when gradients are needed (bf16 / fp16 / fp32 and at most
  1024 features); otherwise the eager PyTorch path below (CPU tensors, other
  GPUs, fp64 or wider rows under autograd). The reference sends every
  gradient-requiring call to ``_reference`` (``ops.py:96-106``). On a gfx950 device a
  missing or broken ``libavey_hip.so`` raises instead of falling back.
* ``'triton'`` raises ``ValueError`` with the reference's message, as the
  reference does on every ROCm build (``ops.py:98-103``: its Triton path needs
  ``torch.version.hip is None``), with or without gradients.
* ``'torch'``  the eager PyTorch path (differentiable).
* ``'hip'``    an extension of this build (not in the reference): the fused HIP
  kernel, or ``ValueError`` when it cannot run. The validation message for an
  unknown backend stays the reference's.

``output_tile`` and ``autotune`` are validated exactly as the reference does
(``ops.py:30-33``) and are otherwise advisory: tiles come from the library's
static table and never change the arithmetic.
"""

import math

import torch
import torch.nn.functional as F

from . import _hip

_BACKENDS = ('auto', 'torch', 'triton', 'hip')
_ACTIVATIONS = ('identity', 'relu', 'relu2', 'silu', 'gelu')
_FLOAT_DTYPES = (torch.float16, torch.bfloat16, torch.float32, torch.float64)


def _validate(z_tr, v, z_tl, bias, valid, eps, norm_eps, activation, backend, output_tile, autotune):
    """Input contract of ``avey_kernels/ops.py:23-46`` (same conditions, same exception type)."""
    if z_tr.ndim != 3 or 0 in z_tr.shape:
        raise ValueError('z_tr must have nonempty shape [batch, context, features]')
    if z_tr.dtype not in _FLOAT_DTYPES:
        raise ValueError('z_tr must be floating point')
    if backend not in _BACKENDS:
        # The reference's message ('hip' is this build's extension, accepted as well).
        raise ValueError('backend must be auto, torch, or triton')
    # `type(...) is int` rejects bool and float tile widths, as the reference does.
    if type(output_tile) is not int or output_tile not in (32, 64, 128):
        raise ValueError('output_tile must be 32, 64, or 128')
    if type(autotune) is not bool:
        raise ValueError('autotune must be boolean')
    if activation not in _ACTIVATIONS:
        raise ValueError('unsupported activation')
    if not (math.isfinite(eps) and eps > 0 and math.isfinite(norm_eps) and norm_eps > 0):
        raise ValueError('eps and norm_eps must be finite and positive')
    context, features = z_tr.shape[1], z_tr.shape[2]
    expected = {'v': (context, context), 'z_tl': tuple(z_tr.shape), 'bias': (features,)}
    for name, tensor in (('v', v), ('z_tl', z_tl), ('bias', bias)):
        if tensor is None:
            continue
        if (tuple(tensor.shape) != expected[name] or tensor.device != z_tr.device
                or tensor.dtype != z_tr.dtype):
            raise ValueError(f'{name} must have shape {expected[name]}, z_tr.dtype, and z_tr.device')
    if valid is not None and (tuple(valid.shape) != tuple(z_tr.shape[:2]) or valid.dtype != torch.bool
                              or valid.device != z_tr.device):
        raise ValueError('valid must be boolean [batch, context] on z_tr.device')


def _activate(x, activation):
    """``avey_kernels/ops.py:49-58``; GELU is PyTorch's tanh approximation."""
    if activation == 'relu':
        return F.relu(x)
    if activation == 'relu2':
        return torch.square(F.relu(x))
    if activation == 'silu':
        return F.silu(x)
    if activation == 'gelu':
        return F.gelu(x, approximate='tanh')
    return x


def _eager(z_tr, v, z_tl, bias, valid, eps, norm_eps, causal, normalize, activation):
    """Eager PyTorch contextualizer (CPU, autograd, non-gfx950 devices).

    Same arithmetic as the reference's ``_reference`` (``ops.py:61-91``): fp32
    accumulation for 16/32-bit inputs and fp64 kept; padded rows selected to zero
    before any arithmetic so NaN padding cannot reach values or gradients; dense
    C x C similarity; signed row sum; one rounding back to ``z_tr.dtype``.
    """
    acc_dtype = torch.float64 if z_tr.dtype == torch.float64 else torch.float32
    z = z_tr.to(acc_dtype)
    row_mask = None if valid is None else valid.unsqueeze(-1)
    if row_mask is not None:
        z = z.masked_fill(~row_mask, 0.0)
    zn = F.normalize(z, p=2.0, dim=-1, eps=norm_eps)
    sim = torch.matmul(zn, zn.transpose(1, 2))
    if v is not None:
        sim = sim * v.to(acc_dtype)
    if causal:
        n = z.shape[1]
        future = torch.ones(n, n, dtype=torch.bool, device=z.device).triu(1)
        sim = sim.masked_fill(future, 0.0)
    if valid is not None:
        sim = sim.masked_fill(~valid.unsqueeze(1), 0.0)
    mixed = torch.matmul(sim, z)
    if normalize:
        mixed = mixed / (sim.sum(dim=-1, keepdim=True) + eps)
    if bias is not None:
        mixed = mixed + bias.to(acc_dtype)
    y = _activate(mixed, activation)
    if z_tl is not None:
        gate = z_tl.to(acc_dtype)
        if row_mask is not None:
            gate = gate.masked_fill(~row_mask, 0.0)
        y = y * gate
    if row_mask is not None:
        y = y.masked_fill(~row_mask, 0.0)
    return y.to(z_tr.dtype)


def _fused_device(t):
    """True for a ROCm tensor on a gfx950 GPU (the only target of libavey_hip.so)."""
    if not t.is_cuda or torch.version.hip is None:
        return False
    props = torch.cuda.get_device_properties(t.device)
    return getattr(props, 'gcnArchName', '').startswith('gfx950')


def _rows(t):
    """t itself when the library can read it in place, else a contiguous copy."""
    return t if _hip.readable_in_place(t) else t.contiguous()


def _dispatch(z_tr, v, z_tl, bias, valid, eps, norm_eps, causal, normalize, activation, backend,
              output_tile, autotune):
    _validate(z_tr, v, z_tl, bias, valid, eps, norm_eps, activation, backend, output_tile, autotune)
    needs_grad = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (z_tr, v, z_tl, bias))
    # With gradients the fused forward runs when the fused backward (avey_bwd) covers
    # the inputs; otherwise autograd differentiates the eager path, which is what the
    # reference always does for gradients (ops.py:96-106).
    if backend == 'triton':
        # The reference's Triton path requires a CUDA (non-ROCm) PyTorch build
        # (ops.py:98-103); on ROCm it always raises, and so does this build.
        raise ValueError('Triton requires Triton installed, NVIDIA SM80+, and CUDA '
                         'FP16/BF16/FP32 inference inputs; use backend="torch" for autograd')
    fused_ok = _fused_device(z_tr) and (not needs_grad or _hip.backward_supported(z_tr))
    if backend == 'hip' and not fused_ok:
        raise ValueError('the fused HIP kernel needs ROCm tensors on a gfx950 (MI355X) GPU; with '
                         'gradients also bf16 / fp16 / fp32 and at most 1024 features; use '
                         'backend="torch" for other inputs')
    if backend == 'torch' or not fused_ok:
        return _eager(z_tr, v, z_tl, bias, valid, eps, norm_eps, causal, normalize, activation)
    # The fused path, one launch. z_tr / z_tl go in as they are when their features
    # are contiguous and their rows do not overlap (strided views such as the halves
    # of the enricher output: the library takes their row and batch strides), where
    # ops.py:109-113 copies them; other layouts (broadcast or overlapping rows) and
    # the other operands are made contiguous as there.
    return torch.ops.avey_kernels.contextualize(
        _rows(z_tr), v.contiguous() if v is not None else None,
        _rows(z_tl) if z_tl is not None else None,
        bias.contiguous() if bias is not None else None,
        valid.contiguous() if valid is not None else None,
        float(eps), float(norm_eps), bool(causal), bool(normalize), activation)


def avey(z_tr: torch.Tensor, v: torch.Tensor, *, z_tl=None, bias=None,
         valid=None, causal=True, norm_eps=1e-12, activation='identity', backend='auto',
         output_tile=32, autotune=False):
    """Avey contextualizer: z_tl * act(((v * cos(z_tr, z_tr)) masked) @ z_tr + bias).

    Signature and defaults of ``avey_kernels/ops.py:117-133``. Causal masking keeps
    the diagonal; ``valid`` masks padded query and key rows, whose outputs are zero
    even after bias and gating. ``eps`` is fixed at 1e-6 and unused (no
    normalisation), as in the reference.
    """
    if v is None:
        raise ValueError('Avey requires the learned V matrix (v)')
    return _dispatch(z_tr, v, z_tl, bias, valid, 1e-6, norm_eps, causal, False, activation,
                     backend, output_tile, autotune)


def avey_b(z_tr: torch.Tensor, *, z_tl=None, bias=None, valid=None, eps=1e-6,
           norm_eps=1e-12, activation='identity', backend='auto', output_tile=32, autotune=False):
    """Avey-B dynamic mixing: z_tl * act((S @ z_tr) / (sum(S) + eps) + bias).

    Signature and defaults of ``avey_kernels/ops.py:136-147``. S is the cosine
    similarity with padded keys zeroed; the row sum keeps its sign (no clamp,
    abs or softmax).
    """
    return _dispatch(z_tr, None, z_tl, bias, valid, eps, norm_eps, False, True, activation,
                     backend, output_tile, autotune)


def _enriched(x, w_gate, b_gate, gate_activation, z_tr, v, bias, valid, eps, norm_eps, causal, normalize,
              activation, backend):
    if backend not in ('auto', 'hip', 'torch'):
        raise ValueError("backend must be 'auto', 'hip' or 'torch' for the enriched forward")
    if gate_activation not in _ACTIVATIONS:
        raise ValueError(f'unknown gate_activation {gate_activation!r}')
    if x.dim() != 3 or x.shape[:2] != z_tr.shape[:2] or w_gate.shape != (z_tr.shape[2], x.shape[2]):
        raise ValueError('x must be [batch, context, d] and w_gate [features, d] for z_tr [batch, context, features]')
    if b_gate is not None and b_gate.shape != (z_tr.shape[2],):
        raise ValueError('b_gate must have shape [features]')
    needs_grad = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (x, w_gate, b_gate, z_tr, v, bias))
    fused_ok = (backend in ('auto', 'hip') and not needs_grad and _fused_device(z_tr)
                and _hip.enriched_supported(x, z_tr, w_gate))
    if backend == 'auto' and fused_ok:
        # The enriched kernel is the 16-row one, and each of its workgroups streams all
        # of the gate weights. It pays where the plan runs 16-row workgroups in one
        # round over the 256 CUs (C2: 26.1 against 31.8 us); with 32- or 64-row
        # workgroups (which read the weights a half / quarter as often) or a second
        # round (C4) the composition is faster, so 'auto' takes it there.
        pl = _hip.plan(tuple(z_tr.shape), z_tr.dtype, causal=causal, normalize=normalize, activation=activation,
                       has_v=v is not None, has_bias=bias is not None, has_valid=valid is not None)
        fused_ok = pl['kernel'] == 'fused_mfma' and pl['block_m'] == 16 and pl['grid'] <= 256
    if backend == 'hip' and not fused_ok:
        raise ValueError('the fused enriched kernel needs bf16 / fp16 ROCm tensors on a gfx950 GPU, '
                         'features <= 1024 and multiples of 8, and no gradients; use backend="torch"')
    if not fused_ok:
        # The composition it replaces: the enricher's gate half, then the op.
        gate = _activate(F.linear(x.float(), w_gate.float(), None if b_gate is None else b_gate.float()),
                         gate_activation).to(z_tr.dtype)
        return _dispatch(z_tr, v, gate, bias, valid, eps, norm_eps, causal, normalize, activation,
                         'torch' if backend == 'torch' else 'auto', 32, False)
    _validate(z_tr, v, None, bias, valid, eps, norm_eps, activation, 'auto', 32, False)
    return torch.ops.avey_kernels.contextualize_enriched(
        x, w_gate, b_gate, _rows(z_tr), v, bias, valid, float(eps), float(norm_eps), bool(causal),
        bool(normalize), activation, gate_activation)


def avey_enriched(x: torch.Tensor, w_gate: torch.Tensor, z_tr: torch.Tensor, v: torch.Tensor, *, b_gate=None,
                  gate_activation='relu', bias=None, valid=None, causal=True, norm_eps=1e-12,
                  activation='identity', backend='auto'):
    """``avey(z_tr, v, z_tl=gate_activation(x @ w_gate.T + b_gate), ...)`` with the gate
    formed inside the fused kernel, one [16, features] tile per row block, and never
    stored. In Avey the enricher's output tail splits into z_tl and z_tr; the static
    layers around the op (ops.py:4-7 of the reference) stay the caller's, except the
    gate half of the enricher, which this call takes over from it: the caller passes
    the enricher's input x and the weight rows (and bias) that produce z_tl.
    Inference only: with gradients, where the fused kernel does not apply, or (with
    ``backend='auto'``) where the plan runs 32- or 64-row workgroups or more than one
    round of them, it runs the composition (the gate in fp32, rounded to z_tr's type, then ``avey``);
    ``backend='hip'`` always runs the enriched kernel."""
    if v is None:
        raise ValueError('Avey requires the learned V matrix (v)')
    return _enriched(x, w_gate, b_gate, gate_activation, z_tr, v, bias, valid, 1e-6, norm_eps, causal, False,
                     activation, backend)


def avey_b_enriched(x: torch.Tensor, w_gate: torch.Tensor, z_tr: torch.Tensor, *, b_gate=None,
                    gate_activation='relu', bias=None, valid=None, eps=1e-6, norm_eps=1e-12,
                    activation='identity', backend='auto'):
    """``avey_b`` with the enricher's gate half fused, as ``avey_enriched``."""
    return _enriched(x, w_gate, b_gate, gate_activation, z_tr, None, bias, valid, eps, norm_eps, False, True,
                     activation, backend)
