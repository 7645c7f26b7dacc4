"""Torch CPU restatement of the reference's eager contextualizer (CPU baseline).

TEST INFRASTRUCTURE ONLY, like ``avey_oracle.py``: only ``tests/`` and the
``cpu_baseline`` leg of ``bench.py`` use it. It is what the reference runs on a
ROCm machine today (``avey_kernels/ops.py:98`` never selects its Triton kernel
there), restated step for step from ``ops.py:61-91`` in PyTorch eager: fp32
accumulation for 16/32-bit inputs (fp64 kept), padded rows selected to zero
first, dense C x C similarity, V, causal and key masks, signed row sum, bias,
activation (``ops.py:49-58``), gate, row mask, one cast back.

Pinned by ``tests/test_oracle.py::test_torch_restatement_matches_numpy_oracle``
(every flag combination and activation against the numpy oracle).
"""

import torch
import torch.nn.functional as F


def activate(x, activation):
    """``avey_kernels/ops.py:49-58``."""
    if activation == 'relu':
        return F.relu(x)
    if activation == 'relu2':
        return F.relu(x).square()
    if activation == 'silu':
        return F.silu(x)
    if activation == 'gelu':
        return F.gelu(x, approximate='tanh')
    if activation == 'identity':
        return x
    raise ValueError(f'unknown activation {activation!r}')


def contextualize(z_tr, v=None, z_tl=None, bias=None, valid=None, *, eps, norm_eps, causal, normalize,
                  activation):
    """``_reference`` of ``avey_kernels/ops.py:61-91`` on torch tensors."""
    acc = torch.float64 if z_tr.dtype == torch.float64 else torch.float32
    z = z_tr.to(acc)
    if valid is not None:
        z = torch.where(valid[:, :, None], z, z.new_zeros(()))           # ops.py:64-67
    zn = F.normalize(z, p=2.0, dim=-1, eps=norm_eps)                      # ops.py:68
    s = zn @ zn.transpose(1, 2)                                           # ops.py:69
    if v is not None:
        s = s * v.to(acc)                                                 # ops.py:70-71
    if causal:
        c = z.shape[1]
        keep = torch.ones(c, c, dtype=torch.bool, device=z.device).tril()
        s = torch.where(keep, s, s.new_zeros(()))                         # ops.py:72-75
    if valid is not None:
        s = torch.where(valid[:, None, :], s, s.new_zeros(()))            # ops.py:76-77
    out = s @ z                                                           # ops.py:78
    if normalize:
        out = out / (s.sum(dim=-1, keepdim=True) + eps)                   # ops.py:79-80
    if bias is not None:
        out = out + bias.to(acc)                                          # ops.py:81-82
    out = activate(out, activation)                                      # ops.py:83
    if z_tl is not None:
        gate = z_tl.to(acc)
        if valid is not None:
            gate = torch.where(valid[:, :, None], gate, gate.new_zeros(()))
        out = out * gate                                                  # ops.py:84-88
    if valid is not None:
        out = torch.where(valid[:, :, None], out, out.new_zeros(()))      # ops.py:89-90
    return out.to(z_tr.dtype)                                             # ops.py:91
