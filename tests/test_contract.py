"""Public API contract of avey_kernel_amd (CPU only).

Mirrors the reference's input-contract, autograd and NaN-padding tests
(tests/test_contextualizer.py:41-85, tests/test_autotune.py:25-30) and its
fake-tensor / Dynamo tracing of the custom op (tests/test_symbolic_tile.py:35-72),
and checks the eager path against the oracle.
"""

import numpy as np
import pytest
import torch

from avey_kernel_amd import avey, avey_b
from avey_kernel_amd import _hip  # noqa: F401  (registers avey_kernels::contextualize)
from conftest import load_kats
from oracle import avey_oracle as orc

KATS = load_kats()


def test_input_contract_raises_value_error():
    z = torch.ones(1, 3, 2)
    with pytest.raises(ValueError):
        avey(z, torch.ones(2, 2))
    with pytest.raises(ValueError):
        avey(z, None)
    with pytest.raises(ValueError):
        avey_b(z, eps=0.)
    with pytest.raises(ValueError):
        avey_b(z, eps=float('inf'))
    with pytest.raises(ValueError):
        avey_b(z, norm_eps=-1.)
    with pytest.raises(ValueError):
        avey_b(z, activation='softmax')
    with pytest.raises(ValueError):
        avey_b(z, backend='unknown')
    with pytest.raises(ValueError):
        avey_b(z, valid=torch.ones(1, 3))
    for tile in (16, 256, 32.0, True):
        with pytest.raises(ValueError):
            avey_b(z, output_tile=tile)
    with pytest.raises(ValueError):
        avey_b(z, autotune=1)
    with pytest.raises(ValueError):
        avey_b(torch.ones(1, 0, 2))
    with pytest.raises(ValueError):
        avey_b(torch.ones(3, 2))
    with pytest.raises(ValueError):
        avey_b(torch.ones(1, 3, 2, dtype=torch.int32))
    with pytest.raises(ValueError):
        avey_b(z, z_tl=torch.ones(1, 3, 2, dtype=torch.float64))
    with pytest.raises(ValueError):
        avey_b(z, bias=torch.ones(3))


@pytest.mark.parametrize('backend', ['hip', 'triton'])
def test_fused_backend_on_cpu_raises_value_error(backend):
    # The reference raises ValueError when its fused backend cannot run (ops.py:101-103).
    with pytest.raises(ValueError):
        avey_b(torch.ones(1, 3, 2), backend=backend)


@pytest.mark.parametrize('case', KATS['cases'], ids=[c['name'] for c in KATS['cases']])
def test_eager_path_known_answers(case):
    dt = torch.float64 if case['dtype'] == 'float64' else torch.float32
    z = torch.tensor(case['z_tr'], dtype=dt)
    kw = {k: v for k, v in case['kwargs'].items()}
    for key in ('z_tl', 'bias'):
        if key in case:
            kw[key] = torch.tensor(case[key], dtype=dt)
    if 'valid' in case:
        kw['valid'] = torch.tensor(case['valid'])
    out = avey(z, torch.tensor(case['v'], dtype=dt), **kw) if case['op'] == 'avey' else avey_b(z, **kw)
    assert out.dtype == dt
    if 'expected_row0' in case:
        torch.testing.assert_close(out[0, 0], torch.tensor(case['expected_row0'], dtype=dt))
    else:
        torch.testing.assert_close(out, torch.tensor(case['expected'], dtype=dt),
                                   rtol=case['rtol'], atol=case['atol'])


@pytest.mark.parametrize('dtype', [torch.float32, torch.float64, torch.bfloat16, torch.float16])
def test_eager_path_matches_oracle(dtype):
    g = torch.Generator().manual_seed(11)
    z = torch.randn(2, 35, 37, generator=g)
    gate = torch.randn(2, 35, 37, generator=g)
    v = torch.randn(35, 35, generator=g)
    bias = torch.randn(37, generator=g)
    valid = torch.ones(2, 35, dtype=torch.bool)
    valid[0, -1] = False
    valid[1, :5] = False
    z[~valid] = float('nan')
    z, gate, v, bias = (t.to(dtype) for t in (z, gate, v, bias))
    tol = {torch.float32: 1e-5, torch.float64: 1e-12, torch.bfloat16: 2e-2, torch.float16: 2e-3}[dtype]
    for causal, normalize, act in ((True, False, 'silu'), (False, True, 'gelu'), (False, False, 'relu2')):
        if normalize:
            out = avey_b(z, z_tl=gate, bias=bias, valid=valid, eps=0.25, activation=act, backend='torch')
        else:
            out = avey(z, v, z_tl=gate, bias=bias, valid=valid, causal=causal, activation=act, backend='torch')
        want = orc.contextualize(z.double().numpy(), None if normalize else v.double().numpy(),
                                 gate.double().numpy(), bias.double().numpy(), valid.numpy(),
                                 eps=0.25 if normalize else 1e-6, norm_eps=1e-12, causal=causal,
                                 normalize=normalize, activation=act)
        assert out.dtype == dtype
        np.testing.assert_allclose(out.double().numpy(), want, rtol=tol, atol=tol)


def test_gradients_through_eager_path():
    z = torch.rand(1, 3, 2, dtype=torch.float64, requires_grad=True)
    v = torch.rand(3, 3, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda x, w: avey(x, w, backend='torch'), (z, v))
    assert torch.autograd.gradcheck(lambda x: avey_b(x, backend='torch'), (z,))


def test_auto_backend_keeps_autograd():
    z = torch.ones(1, 3, 2, requires_grad=True)
    avey_b(z).sum().backward()
    assert z.grad is not None
    x = torch.rand(1, 5, 7, requires_grad=True)
    res = avey_b(x, autotune=True)
    torch.testing.assert_close(res, avey_b(x, backend='torch'))
    res.sum().backward()
    assert torch.isfinite(x.grad).all()


@pytest.mark.parametrize('normalized', [False, True])
def test_nan_padding_cannot_contaminate_gradients(normalized):
    z = torch.tensor([[[1., 2.], [3., 4.], [float('nan'), float('nan')]]], requires_grad=True)
    gate = torch.tensor([[[1., 1.], [1., 1.], [float('nan'), float('nan')]]], requires_grad=True)
    valid = torch.tensor([[True, True, False]])
    out = (avey_b(z, z_tl=gate, valid=valid) if normalized
           else avey(z, torch.ones(3, 3), z_tl=gate, valid=valid))
    out.sum().backward()
    assert torch.isfinite(z.grad).all() and torch.isfinite(gate.grad).all()
    torch.testing.assert_close(z.grad[:, -1], torch.zeros(1, 2))
    torch.testing.assert_close(gate.grad[:, -1], torch.zeros(1, 2))


def test_custom_op_fake_tracing_and_fullgraph_compile():
    # The fused op is opaque to Dynamo and has a fake implementation, so it
    # traces without a GPU (reference: tests/test_symbolic_tile.py:35-72).
    from torch._subclasses.fake_tensor import FakeTensorMode

    def fn(z):
        return torch.ops.avey_kernels.contextualize(z, None, None, None, None, 1e-6, 1e-12, False, True,
                                                    'identity')

    compiled = torch.compile(fn, backend='eager', fullgraph=True, dynamic=True)
    with FakeTensorMode():
        for shape in ((1, 5, 7), (2, 35, 37)):
            z = torch.empty(*shape, dtype=torch.bfloat16)
            out = compiled(z)
            assert out.shape == z.shape and out.dtype == z.dtype


def test_make_fx_records_exactly_one_fused_call():
    from torch.fx.experimental.proxy_tensor import make_fx

    def fn(z, gate):
        return torch.ops.avey_kernels.contextualize(z, None, gate, None, None, 1e-6, 1e-12, True, False, 'silu')

    graph = make_fx(fn, tracing_mode='fake')(torch.empty(2, 35, 37), torch.empty(2, 35, 37))
    calls = [n for n in graph.graph.nodes if 'contextualize' in str(n.target)]
    assert len(calls) == 1


def test_enriched_op_traces_as_one_opaque_call():
    # avey_kernels::contextualize_enriched (the enricher gate fused) has a fake too.
    from torch.fx.experimental.proxy_tensor import make_fx

    def fn(x, w, z):
        return torch.ops.avey_kernels.contextualize_enriched(x, w, None, z, None, None, None, 1e-6, 1e-12, True,
                                                             False, 'identity', 'relu')

    args = (torch.empty(2, 35, 24, dtype=torch.bfloat16), torch.empty(40, 24, dtype=torch.bfloat16),
            torch.empty(2, 35, 40, dtype=torch.bfloat16))
    graph = make_fx(fn, tracing_mode='fake')(*args)
    calls = [n for n in graph.graph.nodes if 'contextualize_enriched' in str(n.target)]
    assert len(calls) == 1
    out = [n for n in graph.graph.nodes if n.op == 'output'][0].args[0]
    assert tuple(out.meta['val'].shape) == (2, 35, 40)


def test_enriched_on_the_cpu_runs_the_composition():
    # Off the GPU (and with gradients) avey_enriched is the enricher's gate half
    # followed by the op, which the oracle restates in fp64.
    import numpy as np
    from avey_kernel_amd import avey_b_enriched, avey_enriched
    from oracle import avey_oracle as orc
    g = torch.Generator().manual_seed(3)
    x, w, bg = torch.randn(2, 9, 16, generator=g), torch.randn(12, 16, generator=g), torch.randn(12, generator=g)
    z, v = torch.randn(2, 9, 12, generator=g), torch.randn(9, 9, generator=g)
    for normalize in (False, True):
        gate = orc.enricher_gate(x.double().numpy(), w.double().numpy(), bg.double().numpy(), 'silu')
        want = orc.contextualize(z.double().numpy(), None if normalize else v.double().numpy(), gate,
                                 eps=1e-6, norm_eps=1e-12, causal=not normalize, normalize=normalize,
                                 activation='identity')
        got = (avey_b_enriched(x, w, z, b_gate=bg, gate_activation='silu') if normalize
               else avey_enriched(x, w, z, v, b_gate=bg, gate_activation='silu'))
        np.testing.assert_allclose(got.double().numpy(), want, rtol=1e-4, atol=1e-4)
    with pytest.raises(ValueError):
        avey_enriched(x, w, z, v, gate_activation='tanh')
    with pytest.raises(ValueError):
        avey_enriched(x, w[:, :8], z, v)
    with pytest.raises(ValueError):
        avey_enriched(x, w, z, v, backend='triton')


# The drop-in package: a reference caller's imports (`from avey_kernels import avey,
# avey_b`, avey_kernels/__init__.py:3-5; `avey_kernels.ops.avey`, ops.py:117-147)
# resolve to this build and give the reference's known answers.
@pytest.mark.parametrize('case', KATS['cases'], ids=[c['name'] for c in KATS['cases']])
def test_drop_in_package_known_answers(case):
    import avey_kernels
    import avey_kernels.ops as ak_ops
    assert avey_kernels.avey is ak_ops.avey and avey_kernels.avey_b is ak_ops.avey_b
    assert avey_kernels.__all__ == ['avey', 'avey_b']
    dt = torch.float64 if case['dtype'] == 'float64' else torch.float32
    z = torch.tensor(case['z_tr'], dtype=dt)
    kw = dict(case['kwargs'])
    for key in ('z_tl', 'bias'):
        if key in case:
            kw[key] = torch.tensor(case[key], dtype=dt)
    if 'valid' in case:
        kw['valid'] = torch.tensor(case['valid'])
    if case['op'] == 'avey':
        out = ak_ops.avey(z, torch.tensor(case['v'], dtype=dt), **kw)
    else:
        out = ak_ops.avey_b(z, **kw)
    want = case.get('expected')
    if want is None:
        torch.testing.assert_close(out[0, 0], torch.tensor(case['expected_row0'], dtype=dt))
    else:
        torch.testing.assert_close(out, torch.tensor(want, dtype=dt), rtol=case['rtol'], atol=case['atol'])
    # The eager path under the reference's own name.
    args = (z, torch.tensor(case['v'], dtype=dt) if case['op'] == 'avey' else None, kw.get('z_tl'), kw.get('bias'),
            kw.get('valid'))
    normalize = case['op'] == 'avey_b'
    ref = ak_ops._reference(*args, kw.get('eps', 1e-6) if normalize else 1e-6, 1e-12,
                            kw.get('causal', not normalize) and not normalize, normalize,
                            kw.get('activation', 'identity'))
    torch.testing.assert_close(ref, out)


def test_triton_backend_raises_like_the_reference_on_rocm():
    # ops.py:98-103: the reference's Triton path needs a CUDA (non-ROCm) build, so on
    # ROCm backend='triton' raises ValueError, with and without gradients
    # (tests/test_triton.py:217-224).
    import avey_kernels
    z = torch.rand(2, 5, 4)
    for requires_grad in (False, True):
        zz = z.clone().requires_grad_(requires_grad)
        with pytest.raises(ValueError, match='Triton requires'):
            avey_kernels.avey_b(zz, backend='triton')
        with pytest.raises(ValueError, match='Triton requires'):
            avey_kernels.avey(zz, torch.rand(5, 5), backend='triton')


def test_unknown_backend_message_is_the_references():
    with pytest.raises(ValueError, match=r'^backend must be auto, torch, or triton$'):
        avey_b(torch.ones(1, 3, 2), backend='cuda')


def test_layouts_read_in_place_or_copied():
    # The C ABI reads a row stride of 0 as "contiguous", so broadcast rows (stride 0)
    # and overlapping rows (0 < stride < D) must reach it as contiguous copies;
    # views with contiguous features and rows >= D apart go in place.
    base = torch.randn(2, 1, 64)
    expanded = base.expand(2, 8, 64)
    assert expanded.stride(1) == 0 and not _hip.readable_in_place(expanded)
    flat = torch.randn(2, 200)
    overlapping = flat.unfold(1, 64, 16)  # [2, 9, 64], rows 16 apart
    assert overlapping.stride() == (200, 16, 1) and not _hip.readable_in_place(overlapping)
    halves = torch.randn(3, 5, 128)[..., 64:]
    assert _hip.readable_in_place(halves) and _hip.row_strides(halves) == (128, 640)
    batch_bcast = torch.randn(1, 5, 64).expand(4, 5, 64)
    assert _hip.readable_in_place(batch_bcast) and _hip.row_strides(batch_bcast) == (64, 0)
    one_row = torch.randn(4, 3, 64)[:, 1:2]  # context 1: its row stride is meaningless
    assert _hip.row_strides(one_row) == (64, 192)
    for bad in (expanded, overlapping):
        with pytest.raises(ValueError):
            _hip.row_strides(bad)
    from avey_kernel_amd import ops
    for t in (expanded, overlapping, torch.randn(2, 64, 8).transpose(1, 2)):
        r = ops._rows(t)
        assert r.is_contiguous() and torch.equal(r, t)
    assert ops._rows(halves) is halves
