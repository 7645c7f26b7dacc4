"""Parity of the fused HIP backward (avey_bwd) against the CPU oracle (needs a gfx950 GPU).

The reference's gradients are autograd over its eager path (avey_kernels/ops.py:96-106),
which accumulates 16-bit inputs in fp32 (ops.py:62-63); the oracle's closed-form
backward (pinned in tests/test_oracle_backward.py) restates them in fp64. Every call
here goes through the C ABI: the registered op ``avey_kernels::contextualize_backward``
or autograd through ``avey`` / ``avey_b``. Inputs are unshifted: z, z_tl and the
incoming gradient N(0, 1), V uniform in [-1, 1] / sqrt(C).

Bar, for every element w of every gradient (fp64 oracle, same dtype-rounded
inputs): |ours - w| <= tol * (1 + |w|), tol 1e-5 for fp32, 5e-3 for fp16 and 2e-2
for bf16 inputs. Gradients past the 16-bit range must overflow to the same
infinities as the oracle's value cast to the input type.

Avey-B gradients divide by the signed row sums den_i = sum_j P_ij, and unshifted
inputs make some sums cancel: the largest row condition sum|P| / |den| reaches
1e4-3e5 here. avey_bwd computes those calls in fp64, which keeps them inside the
flat bound; fp32 arithmetic does not, the reference's own gradients (autograd
over ops.py:61-91, fp32) included. Every Avey-B case prints the largest row
condition and the flat-bound ratio of the reference's fp32 autograd (the eager
restatement oracle/avey_torch_ref.py on the CPU) next to ours, so the
conditioning is reported, not shaped out of the inputs.
"""

import numpy as np
import pytest
import torch

from avey_kernel_amd import avey, avey_b
from avey_kernel_amd import workloads as wl
from conftest import gpu_available
from oracle import avey_oracle as orc
from oracle import avey_torch_ref as tref

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason='needs a gfx950 GPU')]

TOL = {torch.float32: 1e-5, torch.float16: 5e-3, torch.bfloat16: 2e-2}
DEV = 'cuda'
NAMES = ('dz_tr', 'dv', 'dz_tl', 'dbias')


def _np(t):
    return None if t is None else t.detach().double().cpu().numpy()


def _case(b, c, d, dtype, *, seed, gate=True, bias=True, use_v=True, valid=False, nan_pad=True):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(b, c, d, generator=g)
    v = (torch.rand(c, c, generator=g) * 2 - 1) / c ** 0.5 if use_v else None
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


def _ref32_grads(c, *, eps, causal, normalize, act):
    """The reference's own gradients: autograd over its eager path (ops.py:61-91,
    fp32 accumulation) on the CPU, with leaves in the input dtype."""
    leaves = {k: None if c[k] is None else c[k].detach().cpu().clone().requires_grad_()
              for k in ('z', 'v', 'gate', 'bias')}
    valid = None if c['valid'] is None else c['valid'].cpu()
    out = tref.contextualize(leaves['z'], leaves['v'], leaves['gate'], leaves['bias'], valid, eps=eps,
                             norm_eps=1e-12, causal=causal, normalize=normalize, activation=act)
    out.backward(c['dout'].cpu())
    return [None if leaves[k] is None else leaves[k].grad for k in ('z', 'v', 'gate', 'bias')]


def _hip_grads(c, *, eps, causal, normalize, act):
    out = torch.ops.avey_kernels.contextualize_backward(
        c['dout'], c['z'], c['v'], c['gate'], c['bias'], c['valid'], float(eps), 1e-12, causal, normalize, act,
        True, True, True)
    return [None if t.numel() == 0 else t for t in out]


def _check(ours, want, dtype, label, ref=None):
    """Elementwise bar of the module docstring; `ref` (the reference's fp32 gradients,
    Avey-B only) is reported next to ours, not used in the bound."""
    tol = TOL[dtype]
    for k, (name, o, w) in enumerate(zip(NAMES, ours, want)):
        if w is None:
            assert o is None, f'{label} {name} computed without its input'
            continue
        o = _np(o)
        # Gradients beyond the dtype's range round to +-inf in the reference's cast
        # back to the input type; they must overflow the same way here.
        w_cast = torch.from_numpy(np.asarray(w, dtype=np.float64)).to(dtype).double().numpy()
        over = ~np.isfinite(w_cast)
        assert np.array_equal(o[over], w_cast[over]), f'{label} {name} overflow positions differ'
        assert np.isfinite(o[~over]).all(), f'{label} {name} not finite'
        o, w = np.where(over, 0.0, o), np.where(over, 0.0, w)
        err = np.abs(o - w)
        flat = tol * (1.0 + np.abs(w))
        note = f'flat ratio {float((err / flat).max()):.3g}'
        if ref is not None:
            r = np.where(over, 0.0, _np(ref[k]))
            note += f' (reference fp32 autograd: {float((np.abs(r - w) / flat).max()):.3g})'
        bad = err > flat
        print(f'  {label} {name}: {note}', flush=True)
        assert not bad.any(), (f'{label} {name}: {int(bad.sum())} beyond the bound; {note}; '
                               f'max_abs={err.max():.3e} max|w|={float(np.abs(w).max()):.3e}')


def _grads_and_check(c, dtype, label, **kw):
    """HIP gradients against the oracle; Avey-B also reports conditioning and the
    reference's fp32 autograd."""
    ours = _hip_grads(c, **kw)
    torch.cuda.synchronize()
    ref = None
    if kw['normalize']:
        valid = None if c['valid'] is None else c['valid'].cpu().numpy()
        z = np.nan_to_num(_np(c['z']))
        cond = orc.row_condition(z, valid, v=_np(c['v']), causal=kw['causal'], eps=kw['eps'])
        print(f'  {label}: largest row condition {float(cond.max()):.2e}', flush=True)
        ref = _ref32_grads(c, **kw)
    _check(ours, _oracle_grads(c, **kw), dtype, label, ref)


COMBOS = [  # (causal, normalize, use_v): Avey, bidirectional Avey, Avey-B, causal Avey-B, Avey-B with V
    (True, False, True), (False, False, True), (False, True, False), (True, True, False), (False, True, True),
]
# Avey-B calls take the fp64 MFMA path; Avey calls in bf16 with rows of a multiple
# of 8 features the bf16 MFMA path (D = 64, 40, 768, 1024 here), the others the fp32
# MFMA path. C = 130 puts key tiles at rows that are not multiples of 64 in causal mode.
SHAPES = [(2, 37, 20), (1, 70, 64), (3, 130, 19), (2, 130, 40), (2, 16, 768), (1, 65, 1024)]


@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16, torch.float16], ids=['f32', 'bf16', 'f16'])
@pytest.mark.parametrize('shape', SHAPES, ids=['x'.join(map(str, s)) for s in SHAPES])
@pytest.mark.parametrize('causal,normalize,use_v', COMBOS)
def test_backward_matches_oracle(dtype, shape, causal, normalize, use_v):
    label = f'{dtype} {shape} causal={causal} normalize={normalize} v={use_v}'
    print(label, flush=True)
    c = _case(*shape, dtype, seed=sum(shape) + 7 * causal + 3 * normalize, use_v=use_v, valid=shape[1] > 20)
    _grads_and_check(c, dtype, label, eps=1e-6, causal=causal, normalize=normalize, act='identity')


@pytest.mark.parametrize('act', ['identity', 'relu', 'relu2', 'silu', 'gelu'])
@pytest.mark.parametrize('normalize', [False, True])
def test_backward_activations(act, normalize):
    c = _case(2, 45, 36, torch.float32, seed=11, use_v=not normalize, valid=True)
    _grads_and_check(c, torch.float32, f'{act} normalize={normalize}', eps=1e-6, causal=not normalize,
                     normalize=normalize, act=act)


@pytest.mark.parametrize('gate,bias,valid', [(False, False, False), (True, False, True), (False, True, True)])
def test_backward_optional_inputs(gate, bias, valid):
    c = _case(2, 33, 24, torch.bfloat16, seed=5, gate=gate, bias=bias, valid=valid)
    kw = dict(eps=1e-6, causal=True, normalize=False, act='silu')
    _check(_hip_grads(c, **kw), _oracle_grads(c, **kw), torch.bfloat16, f'gate={gate} bias={bias} valid={valid}')


def test_backward_padding_gets_zero_gradient_and_no_nan():
    c = _case(3, 50, 40, torch.float32, seed=3, use_v=False, valid=True)
    dz, _, dg, _ = _hip_grads(c, eps=1e-6, causal=False, normalize=True, act='gelu')
    pad = ~c['valid']
    assert pad.any()
    assert torch.isfinite(dz).all() and torch.isfinite(dg).all()
    assert (dz[pad] == 0).all() and (dg[pad] == 0).all()


def test_backward_zero_rows_take_the_clamped_norm():
    # A valid all-zero row: F.normalize clamps its norm, so its gradient is dzhat / norm_eps.
    c = _case(1, 24, 16, torch.float32, seed=9)
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
    _grads_and_check(c, cfg.dtype, name, eps=1e-6, causal=cfg.causal, normalize=normalize, act='identity')


@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
def test_autograd_through_public_ops_uses_fused_backward(dtype):
    c = _case(2, 40, 48, dtype, seed=21, valid=True, nan_pad=False)
    z = c['z'].clone().requires_grad_()
    v = c['v'].clone().requires_grad_()
    gate = c['gate'].clone().requires_grad_()
    bias = c['bias'].clone().requires_grad_()
    out = avey(z, v, z_tl=gate, bias=bias, valid=c['valid'], activation='silu', backend='hip')
    out.backward(c['dout'])
    ours = [z.grad, v.grad, gate.grad, bias.grad]
    kw = dict(eps=1e-6, causal=True, normalize=False, act='silu')
    _check(ours, _oracle_grads(c, **kw), dtype, 'avey autograd')
    cb = _case(2, 40, 48, dtype, seed=22, use_v=False, gate=False, bias=False, valid=True, nan_pad=False)
    zb = cb['z'].clone().requires_grad_()
    out = avey_b(zb, valid=cb['valid'], backend='hip')
    out.backward(cb['dout'])
    kw = dict(eps=1e-6, causal=False, normalize=True, act='identity')
    _check([zb.grad, None, None, None], _oracle_grads(cb, **kw), dtype, 'avey_b autograd', _ref32_grads(cb, **kw))


def test_autograd_only_requested_gradients():
    c = _case(1, 30, 32, torch.float32, seed=4)
    z = c['z'].clone().requires_grad_()
    out = avey(z, c['v'], z_tl=c['gate'], bias=c['bias'], backend='hip')
    out.backward(c['dout'])
    want = _oracle_grads(c, eps=1e-6, causal=True, normalize=False, act='identity')
    _check([z.grad, None, None, None], [want[0], None, None, None], torch.float32, 'z only')


def test_backward_is_deterministic_except_atomic_sums():
    # dz_tr and dz_tl come from fixed-order sums; dv and dbias from float atomics.
    c = _case(4, 130, 64, torch.bfloat16, seed=31, valid=True, nan_pad=False)
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
    c = _case(2, 96, 64, dtype, seed=41, valid=True, nan_pad=False)
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
