"""Parity of the enriched forward (avey_fwd_enriched) against the fp64 oracle of the
enricher GEMM followed by the contextualizer (needs a gfx950 GPU).

avey_fwd_enriched forms z_tl = gate_act(x W_g^T + b_g) inside the 16-row fused
kernel, one [16, features] tile per row block, instead of reading a stored z_tl.
The oracle composes the same two steps in fp64 on the same dtype-rounded inputs:
``orc.enricher_gate`` (pinned in tests/test_oracle.py) and ``orc.contextualize``.

Bar: |ours - w| <= tol * (1 + |w|) for every element, tol 2e-2 for bf16 and 5e-3
for fp16 (the forward's bounds). The kernel keeps the gate in fp32 (the unfused path
rounds it to the input type before the op reads it), so the two paths agree to
that rounding, which the last test bounds.
"""

import numpy as np
import pytest
import torch

from avey_kernel_amd import avey, avey_b_enriched, avey_enriched
from conftest import gpu_available
from oracle import avey_oracle as orc

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason='needs a gfx950 GPU')]

TOL = {torch.float16: 5e-3, torch.bfloat16: 2e-2}
DEV = 'cuda'


def _np(t):
    return None if t is None else t.detach().double().cpu().numpy()


def _case(b, c, d, dm, dtype, *, seed, use_v=True, bias=True, b_gate=True, valid=False):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(b, c, d, generator=g)
    x = torch.randn(b, c, dm, generator=g)
    w = torch.randn(d, dm, generator=g) / dm ** 0.5
    bg = torch.randn(d, generator=g) * 0.5 if b_gate else None
    v = (torch.rand(c, c, generator=g) * 2 - 1) / c ** 0.5 if use_v else None
    bs = torch.randn(d, generator=g) * 0.2 if bias else None
    vl = None
    if valid:
        lens = torch.randint(max(1, c // 2), c + 1, (b,), generator=g)
        vl = torch.arange(c)[None] < lens[:, None]
        z[~vl] = float('nan')
        x[~vl] = float('nan')  # padded rows of the enricher input reach nothing either
    to = lambda t: None if t is None else t.to(dtype).to(DEV)  # noqa: E731
    return dict(z=to(z), x=to(x), w=to(w), bg=to(bg), v=to(v), bias=to(bs),
                valid=None if vl is None else vl.to(DEV))


def _run(c, *, causal, normalize, act, gate_act, eps=1e-6):
    kw = dict(b_gate=c['bg'], gate_activation=gate_act, bias=c['bias'], valid=c['valid'], activation=act,
              backend='hip')
    if normalize:
        return avey_b_enriched(c['x'], c['w'], c['z'], eps=eps, **kw)
    return avey_enriched(c['x'], c['w'], c['z'], c['v'], causal=causal, **kw)


def _oracle(c, *, causal, normalize, act, gate_act, eps=1e-6):
    valid = None if c['valid'] is None else c['valid'].cpu().numpy()
    x = _np(c['x'])
    if valid is not None:
        x = np.where(valid[..., None], x, 0.0)  # the gate of a padded row is masked anyway
    gate = orc.enricher_gate(x, _np(c['w']), _np(c['bg']), gate_act)
    return orc.contextualize(_np(c['z']), None if normalize else _np(c['v']), gate, _np(c['bias']), valid,
                             eps=eps, norm_eps=1e-12, causal=causal, normalize=normalize, activation=act)


def _check(ours, want, dtype, label):
    o = _np(ours)
    assert np.isfinite(o).all(), f'{label}: non-finite output'
    err = np.abs(o - want)
    flat = TOL[dtype] * (1.0 + np.abs(want))
    ratio = float((err / flat).max())
    print(f'  {label}: flat ratio {ratio:.3g}', flush=True)
    assert ratio <= 1.0, f'{label}: {int((err > flat).sum())} elements beyond the bound, max_abs {err.max():.3e}'


# (batch, context, features, model width): features cover every compiled slice width
# (32, 64, 96, 128, 192 and 256 per wave, full and partial), model widths a multiple of
# 32 and not (a partial last step), contexts with a partial row block and key tile.
SHAPES = [(2, 37, 40, 8), (1, 130, 128, 40), (2, 70, 264, 136), (1, 64, 512, 96), (2, 33, 768, 384),
          (1, 45, 1024, 200), (3, 1, 96, 64)]
FLAGS = [(True, False, True), (False, False, True), (False, True, False)]  # (causal, normalize, use_v)


@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16], ids=['bf16', 'f16'])
@pytest.mark.parametrize('shape', SHAPES, ids=['x'.join(map(str, s)) for s in SHAPES])
@pytest.mark.parametrize('causal,normalize,use_v', FLAGS, ids=['avey', 'avey_bidir', 'avey_b'])
def test_enriched_matches_gemm_then_contextualizer(dtype, shape, causal, normalize, use_v):
    label = f'{dtype} {shape} causal={causal} normalize={normalize}'
    print(label, flush=True)
    c = _case(*shape, dtype, seed=sum(shape) + 5 * causal + 3 * normalize, use_v=use_v, valid=shape[1] > 20)
    kw = dict(causal=causal, normalize=normalize, act='silu', gate_act='relu')
    _check(_run(c, **kw), _oracle(c, **kw), dtype, label)


@pytest.mark.parametrize('gate_act', ['identity', 'relu', 'relu2', 'silu', 'gelu'])
@pytest.mark.parametrize('act', ['identity', 'gelu'])
def test_enriched_gate_and_output_activations(gate_act, act):
    c = _case(2, 50, 192, 64, torch.bfloat16, seed=7, b_gate=gate_act != 'relu', valid=True)
    kw = dict(causal=True, normalize=False, act=act, gate_act=gate_act)
    _check(_run(c, **kw), _oracle(c, **kw), torch.bfloat16, f'gate {gate_act} act {act}')


def test_enriched_at_the_headline_shape():
    # C2's contextualizer (B 16, N 256, D 768, causal Avey) behind a d = 384 enricher.
    print('C2-shaped enriched call', flush=True)
    c = _case(16, 256, 768, 384, torch.bfloat16, seed=2, bias=False)
    kw = dict(causal=True, normalize=False, act='identity', gate_act='relu')
    _check(_run(c, **kw), _oracle(c, **kw), torch.bfloat16, 'C2 shape')


def test_enriched_reads_a_strided_z_tr_in_place():
    # z_tr as the second half of an enricher output [B, C, 2D]: the same result as a copy.
    c = _case(2, 70, 256, 64, torch.bfloat16, seed=9)
    full = torch.cat([torch.randn_like(c['z']), c['z']], dim=-1)
    view = full[..., 256:]
    assert not view.is_contiguous()
    a = avey_enriched(c['x'], c['w'], view, c['v'], b_gate=c['bg'], backend='hip')
    b = avey_enriched(c['x'], c['w'], view.contiguous(), c['v'], b_gate=c['bg'], backend='hip')
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_enriched_agrees_with_the_unfused_composition():
    # The unfused path: the gate GEMM in fp32, rounded to bf16, stored, then the op.
    c = _case(2, 96, 384, 128, torch.bfloat16, seed=13, valid=True)
    fused = _run(c, causal=True, normalize=False, act='identity', gate_act='relu2')
    x = torch.where(c['valid'][..., None], c['x'], torch.zeros((), dtype=c['x'].dtype, device=DEV))
    gate = torch.relu(torch.nn.functional.linear(x.float(), c['w'].float(), c['bg'].float())).square()
    unfused = avey(c['z'], c['v'], z_tl=gate.to(torch.bfloat16), bias=c['bias'], valid=c['valid'], backend='hip')
    torch.cuda.synchronize()
    # Both within the bf16 bound of the oracle; between them, the gate's rounding.
    want = _oracle(c, causal=True, normalize=False, act='identity', gate_act='relu2')
    _check(fused, want, torch.bfloat16, 'fused')
    _check(unfused, want, torch.bfloat16, 'unfused')
    diff = (fused.float() - unfused.float()).abs()
    assert float((diff / (2e-2 * (1 + unfused.float().abs()))).max()) <= 1.0


def test_enriched_without_the_fused_kernel_runs_the_composition():
    # backend='torch' (and gradients) take the eager composition, with the same result
    # to the bf16 bound.
    c = _case(1, 40, 64, 32, torch.bfloat16, seed=17)
    kw = dict(b_gate=c['bg'], gate_activation='silu', bias=c['bias'])
    fused = avey_enriched(c['x'], c['w'], c['z'], c['v'], backend='hip', **kw)
    eager = avey_enriched(c['x'], c['w'], c['z'], c['v'], backend='torch', **kw)
    want = _oracle(c, causal=True, normalize=False, act='identity', gate_act='silu')
    _check(fused, want, torch.bfloat16, 'fused')
    _check(eager, want, torch.bfloat16, 'eager composition')
    zg = c['z'].clone().requires_grad_()
    out = avey_enriched(c['x'], c['w'], zg, c['v'], **kw)
    out.float().sum().backward()
    assert zg.grad is not None and torch.isfinite(zg.grad).all()


def test_enriched_hip_graph_replays_match_eager():
    # avey_fwd_enriched allocates nothing and issues no memset, so it can be captured;
    # every replay, with eager work between them, gives the eager call's bits.
    c = _case(2, 96, 384, 128, torch.bfloat16, seed=19, valid=True)
    run = lambda: _run(c, causal=True, normalize=False, act='gelu', gate_act='relu')  # noqa: E731
    eager = run().clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()  # warm-up on the capture stream (allocator pools)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = run()
    for rep in range(3):
        junk = torch.randn(1 << 20, device=DEV) * rep  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        del junk
        assert torch.equal(static, eager), f'replay {rep}'


def test_enriched_auto_takes_the_composition_where_the_plan_uses_taller_blocks():
    # B 64, C 256, D 512 Avey-B: the plan runs 64-row workgroups there (256 of them), so
    # backend='auto' composes (gate GEMM, then the op); the result meets the same bound
    # either way.
    from avey_kernel_amd import _hip
    c = _case(64, 256, 512, 128, torch.bfloat16, seed=23, use_v=False)
    assert _hip.plan((64, 256, 512), torch.bfloat16, causal=False, normalize=True, has_bias=True)['block_m'] == 64
    kw = dict(causal=False, normalize=True, act='identity', gate_act='relu')
    want = _oracle(c, **kw)
    auto = avey_b_enriched(c['x'], c['w'], c['z'], b_gate=c['bg'], bias=c['bias'], gate_activation='relu')
    _check(auto, want, torch.bfloat16, 'auto (composition)')
    _check(_run(c, **kw), want, torch.bfloat16, 'hip (enriched kernel)')
