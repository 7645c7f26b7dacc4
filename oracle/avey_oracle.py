"""CPU oracle for the Avey / Avey-B forward contextualizer (numpy).

TEST INFRASTRUCTURE ONLY. This module is the parity checker. Only code under
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it. The product package ``avey_kernel_amd`` never
imports, links or calls anything under ``oracle/``.

It restates the reference's eager algorithm (``avey_kernels/ops.py:61-91``)
step for step in numpy, at a selectable accumulation precision:

* ``acc=np.float32`` follows the reference's own arithmetic type for
  fp16/bf16/fp32 inputs (``ops.py:62-63``: low-precision input is upcast to
  fp32, fp64 stays fp64);
* ``acc=np.float64`` is the high-precision oracle used to bound the error of
  both the reference-precision path and the HIP kernels.

Inputs are numpy arrays. bf16/fp16 tensors must be upcast to fp32 by the
caller first (exact), e.g. ``t.float().numpy()``; numpy has no bfloat16.

Pinning (each check lives in ``tests/test_oracle.py``):

* ``activate``: closed forms of ReLU / ReLU^2 / SiLU / tanh-GELU at chosen
  points, and ``torch.nn.functional`` on random points.
* ``contextualize``: the reference's hand-computed known answers
  (``tests/test_contextualizer.py:13-39``, ``tests/test_profiling.py:46-61``,
  ``tests/test_triton.py:162-169``), transcribed into
  ``tests/golden/kats.json``; the independent C restatement
  ``oracle/avey_oracle.c`` (a per-query streaming loop, no N x N matrix) on
  random inputs with every flag combination; invariants (causal output rows
  depend only on earlier rows; permuting keys in the bidirectional case
  leaves outputs unchanged; NaN in masked rows never reaches valid outputs).
* ``contextualize_backward``: central finite differences of ``contextualize``
  in fp64 on small inputs, and PyTorch autograd over the product's eager path
  (a restatement of ``_reference`` that autograd differentiates on its own).
* ``key_tile_count``: the reference's closed-form table
  (``tests/test_causal_skip.py:52-60``) and a brute-force count of tiles
  holding at least one allowed (query, key) pair.
* ``enricher_gate``: ``torch.nn.functional.linear`` in fp64 followed by the
  activations above, and a hand-computed 2 x 2 case.
* ``row_condition`` (a diagnostic printed next to Avey-B results; no test
  bound depends on it except the fp32 subset of rows held to 1e-5): closed
  forms on rows with similarities +-1 / 0 (cancelling sums, eps inside the
  absolute value, padded keys dropped) and an explicit loop over keys.
"""

import math

import numpy as np

ACTIVATIONS = ('identity', 'relu', 'relu2', 'silu', 'gelu')

# sqrt(2/pi), the tanh-GELU constant (ops.py:57 selects PyTorch's tanh form).
_GELU_K = math.sqrt(2.0 / math.pi)


def _sigmoid(x):
    # Evaluated without overflow for large |x|: exp of a non-positive number only.
    e = np.exp(-np.abs(x))
    return np.where(x >= 0, 1.0 / (1.0 + e), e / (1.0 + e))


def activate(x, activation):
    """Elementwise activation, ``avey_kernels/ops.py:49-58``.

    identity; relu = max(x, 0); relu2 = max(x, 0)^2; silu = x * sigmoid(x);
    gelu = 0.5 * x * (1 + tanh(sqrt(2/pi) * (x + 0.044715 x^3))).
    """
    if activation == 'identity':
        return x
    if activation == 'relu':
        return np.maximum(x, 0)
    if activation == 'relu2':
        r = np.maximum(x, 0)
        return r * r
    if activation == 'silu':
        return x * _sigmoid(x)
    if activation == 'gelu':
        inner = _GELU_K * (x + 0.044715 * x * x * x)
        return 0.5 * x * (1.0 + np.tanh(inner))
    raise ValueError(f'unknown activation {activation!r}')


def enricher_gate(x, w_gate, b_gate=None, activation='relu'):
    """z_tl as the enricher produces it: activation(x @ w_gate^T + b_gate).

    The static layer just before the op (the reference leaves it to the caller,
    ``avey_kernels/ops.py:4-7``): in Avey the enricher's output tail splits into
    z_tl and z_tr, so z_tl is the product of x with the enricher weight rows of
    that half. ``x``: [..., d]; ``w_gate``: [features, d] (nn.Linear layout).
    """
    y = np.matmul(x, np.swapaxes(w_gate, -1, -2))
    if b_gate is not None:
        y = y + b_gate
    return activate(y, activation)


def normalize_rows(z, norm_eps):
    """F.normalize along the feature axis: z / max(||z||_2, norm_eps) (ops.py:68)."""
    norms = np.sqrt(np.sum(z * z, axis=-1, keepdims=True))
    return z / np.maximum(norms, z.dtype.type(norm_eps))


def contextualize(z_tr, v=None, z_tl=None, bias=None, valid=None, *, eps, norm_eps,
                  causal, normalize, activation, acc=np.float64):
    """Restatement of ``_reference`` (``avey_kernels/ops.py:61-91``).

    Shapes: z_tr, z_tl [B, C, D]; v [C, C] indexed [query, key] and shared over
    the batch (``ops.py:4-6``); bias [D]; valid bool [B, C]. Returns the
    unrounded result in ``acc`` precision (the reference's final cast to the
    input dtype, ``ops.py:91``, is left to the caller).
    """
    z = np.array(z_tr, dtype=acc, copy=True)
    bsz, c, d = z.shape
    if valid is not None:
        valid = np.asarray(valid, dtype=bool)
        # ops.py:64-67 -- select zeros into padded rows before any arithmetic,
        # so NaN in padding cannot propagate.
        z = np.where(valid[:, :, None], z, acc(0))
    zn = normalize_rows(z, norm_eps)  # ops.py:68
    # ops.py:69 -- cosine similarity, S[b, i, j] = zn_i . zn_j.
    s = np.matmul(zn, np.swapaxes(zn, 1, 2))
    if v is not None:
        # ops.py:70-71 -- learned mixing weights, [query, key].
        s = s * np.asarray(v, dtype=acc)[None]
    if causal:
        # ops.py:72-75 -- keys after the query are dropped; the diagonal stays.
        allowed = np.tril(np.ones((c, c), dtype=bool))
        s = np.where(allowed[None], s, acc(0))
    if valid is not None:
        # ops.py:76-77 -- padded keys contribute nothing.
        s = np.where(valid[:, None, :], s, acc(0))
    # ops.py:78 -- mixing with the unnormalised rows.
    num = np.matmul(s, z)
    if normalize:
        # ops.py:79-80 -- signed row sum plus eps; no clamp, abs or softmax.
        num = num / (np.sum(s, axis=-1, keepdims=True) + acc(eps))
    if bias is not None:
        num = num + np.asarray(bias, dtype=acc)  # ops.py:81-82
    out = activate(num, activation)  # ops.py:83
    if z_tl is not None:
        gate = np.asarray(z_tl, dtype=acc)
        if valid is not None:
            gate = np.where(valid[:, :, None], gate, acc(0))  # ops.py:86-87
        out = out * gate  # ops.py:88
    if valid is not None:
        out = np.where(valid[:, :, None], out, acc(0))  # ops.py:89-90
    return out.astype(acc, copy=False)


def avey(z_tr, v, *, z_tl=None, bias=None, valid=None, causal=True, norm_eps=1e-12,
         activation='identity', acc=np.float64):
    """Avey defaults, ``avey_kernels/ops.py:117-133``: eps=1e-6 (unused, normalize off)."""
    return contextualize(z_tr, v, z_tl, bias, valid, eps=1e-6, norm_eps=norm_eps,
                         causal=causal, normalize=False, activation=activation, acc=acc)


def avey_b(z_tr, *, z_tl=None, bias=None, valid=None, eps=1e-6, norm_eps=1e-12,
           activation='identity', acc=np.float64):
    """Avey-B defaults, ``avey_kernels/ops.py:136-147``: no V, bidirectional, normalised."""
    return contextualize(z_tr, None, z_tl, bias, valid, eps=eps, norm_eps=norm_eps,
                         causal=False, normalize=True, activation=activation, acc=acc)


def key_tile_count(query_tile, c, bm, bn, causal, skip=True):
    """Key tiles a query tile visits, ``avey_kernels/_triton.py:38-50``.

    With causal skipping the tile holding the diagonal is kept and every
    tile strictly after the last query of the block is dropped.
    """
    if c <= bn:
        return 1
    if causal and skip:
        query_end = min((query_tile + 1) * bm, c)
        return -(-query_end // bn)
    return -(-c // bn)


def row_condition(z_tr, valid=None, *, v=None, causal=False, eps=1e-6, norm_eps=1e-12):
    """Per-row conditioning of the Avey-B denominator, sum_j |P_ij| / |sum_j P_ij + eps|.

    P is the masked, weighted similarity of ops.py:69-77 (S, times V when given,
    causal and key masks), summed over keys j. Reports how much a row amplifies
    rounding (no reference counterpart; derived from ops.py:79-80).
    """
    z = np.array(z_tr, dtype=np.float64, copy=True)
    if valid is not None:
        valid = np.asarray(valid, dtype=bool)
        z = np.where(valid[:, :, None], z, 0.0)
    zn = z / np.maximum(np.sqrt(np.sum(z * z, -1, keepdims=True)), norm_eps)
    s = np.matmul(zn, np.swapaxes(zn, 1, 2))
    if v is not None:
        s = s * np.asarray(v, dtype=np.float64)
    if causal:
        s = np.tril(s)
    if valid is not None:
        s = np.where(valid[:, None, :], s, 0.0)
    return np.sum(np.abs(s), -1) / np.abs(np.sum(s, -1) + eps)


def activate_grad(x, activation):
    """d act(x) / dx for the activations of ``avey_kernels/ops.py:49-58``.

    The reference has no written backward: its gradients are PyTorch autograd
    over ``_reference`` (``ops.py:96-106``), so these are the derivatives
    autograd takes. relu: 1 where x > 0 (threshold_backward); relu2: 2 max(x, 0);
    silu: s (1 + x (1 - s)) with s = sigmoid(x); gelu (tanh form):
    0.5 (1 + t) + 0.5 x (1 - t^2) k (1 + 3 * 0.044715 x^2), t = tanh(k (x + 0.044715 x^3)).
    """
    one = x.dtype.type(1)
    if activation == 'identity':
        return np.ones_like(x)
    if activation == 'relu':
        return (x > 0).astype(x.dtype)
    if activation == 'relu2':
        return 2 * np.maximum(x, 0)
    if activation == 'silu':
        s = _sigmoid(x)
        return s * (one + x * (one - s))
    if activation == 'gelu':
        t = np.tanh(_GELU_K * (x + 0.044715 * x * x * x))
        return 0.5 * (one + t) + 0.5 * x * (one - t * t) * _GELU_K * (one + 3 * 0.044715 * x * x)
    raise ValueError(f'unknown activation {activation!r}')


def contextualize_backward(dout, z_tr, v=None, z_tl=None, bias=None, valid=None, *, eps, norm_eps,
                           causal, normalize, activation, acc=np.float64, _plant=None):
    """Gradients of ``contextualize`` (the ``_reference`` math, ``ops.py:61-91``).

    Returns ``(dz_tr, dv, dz_tl, dbias)``, unrounded in ``acc``; entries for
    absent inputs are None. Written as the closed-form chain rule (no autograd),
    per batch item with P = S * V * M, y = num / den (normalize) or num,
    u = y + bias, r the valid-row mask:

    * dz_tl = dout * act(u) * r;  du = dout * gate * act'(u) * r;  dbias = sum du
    * normalize: dnum = du / den, dden_i = -sum_d du_id y_id / den_i; else dnum = du, dden = 0
    * dP_ij = dnum_i . z_j + dden_i;  dS = dP * V * M;  dv = sum_b dP * S * M
    * dz = r * (P^T dnum + J(dzhat)),  dzhat = dS zhat + dS^T zhat,
      J(x) = (x - zhat (zhat . x)) / ||z|| where ||z|| >= norm_eps, else x / norm_eps
      (F.normalize divides by clamp_min(||z||, norm_eps); the clamp passes no
      gradient to the norm below it).

    ``_plant`` injects a named mistake ('no_radial', 'no_transpose',
    'dden_sign') so the tests can show their checks catch it.
    """
    z = np.array(z_tr, dtype=acc, copy=True)
    g = np.array(dout, dtype=acc, copy=True)
    bsz, c, d = z.shape
    r = np.ones((bsz, c), dtype=bool) if valid is None else np.asarray(valid, dtype=bool)
    z = np.where(r[:, :, None], z, acc(0))
    g = np.where(r[:, :, None], g, acc(0))
    norms = np.sqrt(np.sum(z * z, axis=-1, keepdims=True))
    denom = np.maximum(norms, acc(norm_eps))
    zn = z / denom
    s = np.matmul(zn, np.swapaxes(zn, 1, 2))
    mask = np.broadcast_to(r[:, None, :], s.shape).copy()
    if causal:
        mask &= np.tril(np.ones((c, c), dtype=bool))[None]
    w = mask.astype(acc)
    if v is not None:
        w = w * np.asarray(v, dtype=acc)[None]
    p = s * w
    num = np.matmul(p, z)
    den = np.sum(p, axis=-1, keepdims=True) + acc(eps) if normalize else None
    y = num / den if normalize else num
    u = y + (np.asarray(bias, dtype=acc) if bias is not None else acc(0))
    a = activate(u, activation)
    if z_tl is not None:
        gate = np.where(r[:, :, None], np.asarray(z_tl, dtype=acc), acc(0))
        dz_tl = g * a
        du = g * gate * activate_grad(u, activation)
    else:
        dz_tl = None
        du = g * activate_grad(u, activation)
    dbias = du.sum(axis=(0, 1)) if bias is not None else None
    if normalize:
        dnum = du / den
        dden = -np.sum(du * y, axis=-1, keepdims=True) / den
        if _plant == 'dden_sign':
            dden = -dden
    else:
        dnum = du
        dden = np.zeros((bsz, c, 1), dtype=acc)
    dp = np.matmul(dnum, np.swapaxes(z, 1, 2)) + dden
    ds = dp * w
    dv = np.sum(dp * s * mask, axis=0) if v is not None else None
    dzn = np.matmul(ds, zn) + (0 if _plant == 'no_transpose' else np.matmul(np.swapaxes(ds, 1, 2), zn))
    radial = 0 if _plant == 'no_radial' else np.sum(zn * dzn, axis=-1, keepdims=True)
    dz_norm = np.where(norms >= acc(norm_eps), (dzn - zn * radial) / denom, dzn / acc(norm_eps))
    dz = np.matmul(np.swapaxes(p, 1, 2), dnum) + dz_norm
    dz = np.where(r[:, :, None], dz, acc(0))
    return dz, dv, dz_tl, dbias
