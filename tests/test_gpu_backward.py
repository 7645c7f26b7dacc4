"""Parity of the fused HIP backward (avey_bwd) against the CPU oracle (needs a gfx950 GPU).

The reference's gradients are autograd over its eager path (avey_kernels/ops.py:96-106);
the oracle's closed-form backward (pinned in tests/test_oracle_backward.py) restates
them in fp64. Every call here goes through the C ABI: the registered op
``avey_kernels::contextualize_backward`` or autograd through ``avey`` / ``avey_b``.

Tolerance per gradient tensor, against the fp64 oracle on the same (dtype-rounded)
inputs: |ours - oracle| <= tol * (|oracle| + max|oracle|), elementwise, with tol
1e-5 for fp32, 5e-3 for fp16 and 2e-2 for bf16 (the forward's bounds; the
backward computes in fp32, so the 16-bit error is the final rounding). Avey-B
configurations at full size, whose signed row sums cancel on some rows, are
compared normwise: ||ours - oracle||_F <= tol * ||oracle||_F. The max-abs error is
in every failure message. Gradients past the 16-bit range must overflow to the
same infinities as the oracle's value cast to the input type.
"""

import numpy as np
import pytest
import torch

from avey_kernel_amd import avey, avey_b
from avey_kernel_amd import workloads as wl
from conftest import gpu_available
from oracle import avey_oracle as orc

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason='needs a gfx950 GPU')]

TOL = {torch.float32: 1e-5, torch.float16: 5e-3, torch.bfloat16: 2e-2}
DEV = 'cuda'
NAMES = ('dz_tr', 'dv', 'dz_tl', 'dbias')


def _np(t):
    return None if t is None else t.detach().double().cpu().numpy()


def _case(b, c, d, dtype, *, seed, normalize, gate=True, bias=True, use_v=True, valid=False, nan_pad=True):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(b, c, d, generator=g) + (0.5 if normalize else 0.0)  # keeps Avey-B row sums off zero
    # With normalize, V in [0.5, 1.5] / sqrt(C) keeps the weighted row sums off zero too;
    # a row sum near zero amplifies every rounding error by 1 / den^2 in the gradient.
    v = None
    if use_v:
        u = torch.rand(c, c, generator=g)
        v = ((0.5 + u) if normalize else (u * 2 - 1)) / c ** 0.5
    gt = torch.randn(b, c, d, generator=g) if gate else None
    bs = torch.randn(d, generator=g) * 0.2 if bias else None
    dout = torch.randn(b, c, d, generator=g)
    vl = None
    if valid:
        lens = torch.randint(max(1, c // 2), c + 1, (b,), generator=g)
        vl = torch.arange(c)[None] < lens[:, None]
        if nan_pad:
            z[~vl] = float('nan')
            if gt is not None:
                gt[~vl] = float('nan')
    to = lambda t: None if t is None else t.to(dtype).to(DEV)  # noqa: E731
    return dict(z=to(z), v=to(v), gate=to(gt), bias=to(bs), valid=None if vl is None else vl.to(DEV),
                dout=to(dout))


def _oracle_grads(c, *, eps, causal, normalize, act):
    return orc.contextualize_backward(
        _np(c['dout']), _np(c['z']), _np(c['v']), _np(c['gate']), _np(c['bias']),
        None if c['valid'] is None else c['valid'].cpu().numpy(), eps=eps, norm_eps=1e-12, causal=causal,
        normalize=normalize, activation=act)


def _hip_grads(c, *, eps, causal, normalize, act):
    out = torch.ops.avey_kernels.contextualize_backward(
        c['dout'], c['z'], c['v'], c['gate'], c['bias'], c['valid'], float(eps), 1e-12, causal, normalize, act,
        True, True, True)
    return [None if t.numel() == 0 else t for t in out]


def _check(ours, want, dtype, label, normwise=False):
    for name, o, w in zip(NAMES, ours, want):
        if w is None:
            assert o is None, f'{label} {name} computed without its input'
            continue
        o = _np(o)
        tol = TOL[dtype]
        # Gradients beyond the dtype's range round to +-inf in the reference's cast
        # back to the input type; they must overflow the same way here.
        w_cast = torch.from_numpy(np.asarray(w, dtype=np.float64)).to(dtype).double().numpy()
        over = ~np.isfinite(w_cast)
        assert np.array_equal(o[over], w_cast[over]), f'{label} {name} overflow positions differ'
        assert np.isfinite(o[~over]).all(), f'{label} {name} not finite'
        o, w = np.where(over, 0.0, o), np.where(over, 0.0, w)
        err = np.abs(o - w)
        scale = float(np.abs(w).max())
        if normwise:
            rel = float(np.linalg.norm(o - w) / max(np.linalg.norm(w), 1e-30))
            assert rel <= tol, f'{label} {name} normwise {rel:.3e} max_abs={err.max():.3e} scale={scale:.3e}'
            continue
        bad = err > tol * (np.abs(w) + scale)
        assert not bad.any(), f'{label} {name}: {int(bad.sum())} beyond tol; max_abs={err.max():.3e} scale={scale:.3e}'


COMBOS = [  # (causal, normalize, use_v): Avey, bidirectional Avey, Avey-B, causal Avey-B, Avey-B with V
    (True, False, True), (False, False, True), (False, True, False), (True, True, False), (False, True, True),
]
# bf16 rows of a multiple of 8 features take the bf16 MFMA path (D = 64, 40, 768,
# 1024 here); the others, and fp32 / fp16, the fp32 MFMA path. C = 130 puts key
# tiles at rows that are not multiples of 64 in causal mode.
SHAPES = [(2, 37, 20), (1, 70, 64), (3, 130, 19), (2, 130, 40), (2, 16, 768), (1, 65, 1024)]


@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16, torch.float16], ids=['f32', 'bf16', 'f16'])
@pytest.mark.parametrize('shape', SHAPES, ids=['x'.join(map(str, s)) for s in SHAPES])
@pytest.mark.parametrize('causal,normalize,use_v', COMBOS)
def test_backward_matches_oracle(dtype, shape, causal, normalize, use_v):
    label = f'{dtype} {shape} causal={causal} normalize={normalize} v={use_v}'
    print(label, flush=True)
    c = _case(*shape, dtype, seed=sum(shape) + 7 * causal + 3 * normalize, normalize=normalize, use_v=use_v,
              valid=shape[1] > 20)
    kw = dict(eps=1e-6, causal=causal, normalize=normalize, act='identity')
    _check(_hip_grads(c, **kw), _oracle_grads(c, **kw), dtype, label)


@pytest.mark.parametrize('act', ['identity', 'relu', 'relu2', 'silu', 'gelu'])
@pytest.mark.parametrize('normalize', [False, True])
def test_backward_activations(act, normalize):
    c = _case(2, 45, 36, torch.float32, seed=11, normalize=normalize, use_v=not normalize, valid=True)
    kw = dict(eps=1e-6, causal=not normalize, normalize=normalize, act=act)
    _check(_hip_grads(c, **kw), _oracle_grads(c, **kw), torch.float32, f'{act} normalize={normalize}')


@pytest.mark.parametrize('gate,bias,valid', [(False, False, False), (True, False, True), (False, True, True)])
def test_backward_optional_inputs(gate, bias, valid):
    c = _case(2, 33, 24, torch.bfloat16, seed=5, normalize=False, gate=gate, bias=bias, valid=valid)
    kw = dict(eps=1e-6, causal=True, normalize=False, act='silu')
    _check(_hip_grads(c, **kw), _oracle_grads(c, **kw), torch.bfloat16, f'gate={gate} bias={bias} valid={valid}')


def test_backward_padding_gets_zero_gradient_and_no_nan():
    c = _case(3, 50, 40, torch.float32, seed=3, normalize=True, use_v=False, valid=True)
    dz, _, dg, _ = _hip_grads(c, eps=1e-6, causal=False, normalize=True, act='gelu')
    pad = ~c['valid']
    assert pad.any()
    assert torch.isfinite(dz).all() and torch.isfinite(dg).all()
    assert (dz[pad] == 0).all() and (dg[pad] == 0).all()


def test_backward_zero_rows_take_the_clamped_norm():
    # A valid all-zero row: F.normalize clamps its norm, so its gradient is dzhat / norm_eps.
    c = _case(1, 24, 16, torch.float32, seed=9, normalize=False)
    c['z'][0, 5] = 0
    kw = dict(eps=1e-6, causal=True, normalize=False, act='identity')
    _check(_hip_grads(c, **kw), _oracle_grads(c, **kw), torch.float32, 'zero row')


@pytest.mark.parametrize('name', ['C2', 'C3', 'C4', 'C5'])
def test_backward_benchmark_configs(name):
    """Full-size configurations against the fp64 oracle (identity activation, the
    benchmark's gate and bias, and a random incoming gradient)."""
    print(name, flush=True)
    cfg = wl.CONFIGS[name]
    inp = wl.make_inputs(cfg, device=DEV)
    g = torch.Generator().manual_seed(100 + cfg.seed)
    dout = torch.randn(inp['z_tr'].shape, generator=g).to(inp['z_tr'].dtype).to(DEV)
    c = dict(z=inp['z_tr'], v=inp.get('v') if cfg.op == 'avey' else None, gate=inp.get('z_tl'),
             bias=inp.get('bias'), valid=inp.get('valid'), dout=dout)
    normalize = cfg.op == 'avey_b'
    kw = dict(eps=1e-6, causal=cfg.causal, normalize=normalize, act='identity')
    ours = _hip_grads(c, **kw)
    torch.cuda.synchronize()
    _check(ours, _oracle_grads(c, **kw), cfg.dtype, name, normwise=normalize)


@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
def test_autograd_through_public_ops_uses_fused_backward(dtype):
    c = _case(2, 40, 48, dtype, seed=21, normalize=False, valid=True, nan_pad=False)
    z = c['z'].clone().requires_grad_()
    v = c['v'].clone().requires_grad_()
    gate = c['gate'].clone().requires_grad_()
    bias = c['bias'].clone().requires_grad_()
    out = avey(z, v, z_tl=gate, bias=bias, valid=c['valid'], activation='silu', backend='hip')
    out.backward(c['dout'])
    ours = [z.grad, v.grad, gate.grad, bias.grad]
    kw = dict(eps=1e-6, causal=True, normalize=False, act='silu')
    _check(ours, _oracle_grads(c, **kw), dtype, 'avey autograd')
    cb = _case(2, 40, 48, dtype, seed=22, normalize=True, use_v=False, valid=True, nan_pad=False)
    zb = cb['z'].clone().requires_grad_()
    out = avey_b(zb, valid=cb['valid'], backend='hip')
    out.backward(cb['dout'])
    want = orc.contextualize_backward(_np(cb['dout']), _np(cb['z']), valid=cb['valid'].cpu().numpy(), eps=1e-6,
                                      norm_eps=1e-12, causal=False, normalize=True, activation='identity')
    _check([zb.grad, None, None, None], want, dtype, 'avey_b autograd')


def test_autograd_only_requested_gradients():
    c = _case(1, 30, 32, torch.float32, seed=4, normalize=False)
    z = c['z'].clone().requires_grad_()
    out = avey(z, c['v'], z_tl=c['gate'], bias=c['bias'], backend='hip')
    out.backward(c['dout'])
    want = _oracle_grads(c, eps=1e-6, causal=True, normalize=False, act='identity')
    _check([z.grad, None, None, None], [want[0], None, None, None], torch.float32, 'z only')


def test_backward_is_deterministic_except_atomic_sums():
    # dz_tr and dz_tl come from fixed-order sums; dv and dbias from float atomics.
    c = _case(4, 130, 64, torch.bfloat16, seed=31, normalize=False, valid=True, nan_pad=False)
    kw = dict(eps=1e-6, causal=True, normalize=False, act='gelu')
    a = _hip_grads(c, **kw)
    b = _hip_grads(c, **kw)
    assert torch.equal(a[0], b[0]) and torch.equal(a[2], b[2])
    torch.testing.assert_close(a[1], b[1], rtol=1e-2, atol=1e-2)
    torch.testing.assert_close(a[3], b[3], rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float32])
def test_backward_hip_graph_replays_match_eager(dtype):
    """avey_bwd issues no memset (accumulators are cleared by a kernel), so it can be
    captured; every replay, with eager work between them, matches the eager call."""
    c = _case(2, 96, 64, dtype, seed=41, normalize=False, valid=True, nan_pad=False)
    kw = dict(eps=1e-6, causal=True, normalize=False, act='silu')
    eager = [t.clone() for t in _hip_grads(c, **kw)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _hip_grads(c, **kw)  # warm-up on the capture stream (allocator pools)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = _hip_grads(c, **kw)
    for rep in range(3):
        junk = torch.randn(1 << 20, device=DEV) * rep  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        del junk
        assert torch.equal(static[0], eager[0]) and torch.equal(static[2], eager[2]), f'replay {rep}'
        torch.testing.assert_close(static[1], eager[1], rtol=1e-2, atol=1e-2)
        torch.testing.assert_close(static[3], eager[3], rtol=1e-2, atol=1e-2)
