"""Pin the oracle's backward (CPU only).

``orc.contextualize_backward`` is the closed-form chain rule of the forward
restatement. It is checked against what fixes it independently:
* central finite differences of ``orc.contextualize`` in fp64 (directional
  derivatives along random directions, for every input that has a gradient),
  including rows whose norm is below ``norm_eps`` (the clamp branch);
* PyTorch autograd over the package's eager path in fp64 (a separate
  restatement of ``avey_kernels/ops.py:61-91`` that autograd differentiates),
  with NaN in padded rows, which must reach no gradient;
* planted mistakes in the oracle (radial term dropped, transposed similarity
  term dropped, sign of the denominator term flipped) fail the finite
  differences.
"""

import itertools

import numpy as np
import pytest
import torch

from avey_kernel_amd import ops
from oracle import avey_oracle as orc

COMBOS = [  # (causal, normalize, use_v)
    (True, False, True), (False, False, True), (False, True, False), (True, True, False), (False, True, True),
]


def _inputs(seed, b=2, c=6, d=5, *, gate=True, bias=True, valid=False, small_row=False):
    rng = np.random.default_rng(seed)
    z = rng.standard_normal((b, c, d)) + 0.6  # keeps Avey-B row sums away from zero
    if small_row:
        z[0, 2] *= 0.05  # norm below norm_eps = 0.5 below: the clamp branch
    v = rng.uniform(-1, 1, (c, c))
    g = rng.standard_normal((b, c, d)) if gate else None
    bb = rng.standard_normal(d) * 0.3 if bias else None
    val = None
    if valid:
        val = np.ones((b, c), dtype=bool)
        val[0, -2:] = False
        val[1, 1] = False
    dout = rng.standard_normal((b, c, d))
    return z, v, g, bb, val, dout


def _fd_check(z, v, g, bb, val, dout, *, causal, normalize, activation, norm_eps, plant=None, seed=0):
    kw = dict(eps=1e-6, norm_eps=norm_eps, causal=causal, normalize=normalize, activation=activation)
    grads = orc.contextualize_backward(dout, z, v, g, bb, val, _plant=plant, **kw)
    args = [z, v, g, bb]
    rng = np.random.default_rng(seed + 100)
    h = 1e-6
    errs = []
    for k, x in enumerate(args):
        if x is None:
            continue
        direction = rng.standard_normal(x.shape)
        if val is not None and k in (0, 2):
            direction = np.where(val[:, :, None], direction, 0.0)

        def loss(t):
            a = list(args)
            a[k] = x + t * direction
            return float(np.sum(dout * orc.contextualize(*a, val, **kw)))

        fd = (loss(h) - loss(-h)) / (2 * h)
        an = float(np.sum(grads[k] * direction))
        errs.append(abs(fd - an) / max(1.0, abs(fd)))
    return max(errs)


@pytest.mark.parametrize('causal,normalize,use_v', COMBOS)
@pytest.mark.parametrize('activation', ['identity', 'relu', 'relu2', 'silu', 'gelu'])
def test_backward_matches_finite_differences(causal, normalize, use_v, activation):
    z, v, g, bb, val, dout = _inputs(1, valid=True)
    err = _fd_check(z, v if use_v else None, g, bb, val, dout, causal=causal, normalize=normalize,
                    activation=activation, norm_eps=1e-12)
    assert err < 1e-6


@pytest.mark.parametrize('causal,normalize,use_v', COMBOS)
def test_backward_clamped_norm_rows(causal, normalize, use_v):
    z, v, g, bb, _, dout = _inputs(2, small_row=True)
    norms = np.linalg.norm(z, axis=-1)
    assert (norms < 0.5).sum() == 1 and (norms > 0.6).sum() == norms.size - 1
    err = _fd_check(z, v if use_v else None, g, bb, None, dout, causal=causal, normalize=normalize,
                    activation='silu', norm_eps=0.5)
    assert err < 1e-6


def test_backward_without_gate_or_bias():
    z, v, _, _, val, dout = _inputs(3, gate=False, bias=False, valid=True)
    assert _fd_check(z, v, None, None, val, dout, causal=True, normalize=False, activation='gelu',
                     norm_eps=1e-12) < 1e-6


@pytest.mark.parametrize('plant', ['no_radial', 'no_transpose', 'dden_sign'])
def test_planted_backward_mistakes_fail_finite_differences(plant):
    z, v, g, bb, val, dout = _inputs(4, valid=True)
    normalize = plant == 'dden_sign'
    err = _fd_check(z, None if normalize else v, g, bb, val, dout, causal=not normalize, normalize=normalize,
                    activation='silu', norm_eps=1e-12, plant=plant)
    assert err > 1e-3


@pytest.mark.parametrize('causal,normalize,use_v', COMBOS)
@pytest.mark.parametrize('activation', ['identity', 'gelu'])
def test_backward_matches_torch_autograd_with_nan_padding(causal, normalize, use_v, activation):
    z, v, g, bb, val, dout = _inputs(5, b=3, c=9, d=7, valid=True)
    z = z.copy()
    g = g.copy()
    z[~val] = np.nan
    g[~val] = np.nan
    tz, tv, tg, tb = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (z, v, g, bb))
    out = ops._eager(tz, tv if use_v else None, tg, tb, torch.tensor(val), 1e-6, 1e-12, causal, normalize,
                     activation)
    out.backward(torch.tensor(dout))
    dz, dv, dg, db = orc.contextualize_backward(dout, z, v if use_v else None, g, bb, val, eps=1e-6,
                                                norm_eps=1e-12, causal=causal, normalize=normalize,
                                                activation=activation)
    for ours, theirs in ((dz, tz.grad), (dg, tg.grad), (db, tb.grad)) + (((dv, tv.grad),) if use_v else ()):
        assert np.isfinite(ours).all() and torch.isfinite(theirs).all()
        np.testing.assert_allclose(ours, theirs.numpy(), rtol=1e-9, atol=1e-9)
    assert (dz[~val] == 0).all() and (dg[~val] == 0).all()
