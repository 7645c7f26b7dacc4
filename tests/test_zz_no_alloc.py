"""avey_fwd_noalloc, the allocation-free forward, against avey_fwd (needs a gfx950 GPU).

It runs the same kernels as avey_fwd with the scratch taken from the library's
static device array, so its results must equal avey_fwd's bit for bit. Two calls
in a row, the second on a smaller input (the array keeps the first call's
contents), for the generic fp32 / fp64 kernel (which uses the scratch: per-row
inverse norms) and the fused bf16 kernel (which needs none).
"""

import ctypes

import pytest
import torch

from avey_kernel_amd import _hip
from conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason='needs a gfx950 GPU')]
DEV = 'cuda'


def _inputs(batch, context, features, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(batch, context, features, generator=g).to(DEV, dtype)
    gate = torch.randn(batch, context, features, generator=g).to(DEV, dtype)
    v = ((torch.rand(context, context, generator=g) * 2 - 1) / context ** 0.5).to(DEV, dtype)
    bias = (torch.randn(features, generator=g) * 0.1).to(DEV, dtype)
    lengths = torch.randint(context // 2, context + 1, (batch,), generator=g)
    valid = (torch.arange(context)[None, :] < lengths[:, None]).to(DEV)
    return z, gate, v, bias, valid


def _noalloc(z, v, gate, bias, valid, eps, causal, normalize, act):
    out = torch.empty_like(z)
    args = _hip.make_args(z, v, gate, bias, None if valid is None else valid.view(torch.uint8), out, eps, 1e-12,
                          causal, normalize, act)
    stream = torch.cuda.current_stream().cuda_stream
    st = _hip.load().avey_fwd_noalloc(ctypes.byref(args), ctypes.c_void_p(stream))
    assert st == 0, _hip.status_string(st)
    return out


@pytest.mark.parametrize('dtype,shapes', [
    (torch.float32, [(3, 97, 72), (2, 40, 33)]),
    (torch.float64, [(2, 65, 40), (1, 17, 9)]),
    (torch.bfloat16, [(4, 96, 256), (2, 35, 128)]),
], ids=['fp32', 'fp64', 'bf16'])
def test_noalloc_matches_avey_fwd_on_two_calls(dtype, shapes):
    for seed, (batch, context, features) in enumerate(shapes):
        print(f'[noalloc] {dtype} shape {(batch, context, features)}', flush=True)
        z, gate, v, bias, valid = _inputs(batch, context, features, dtype, seed)
        plan = _hip.plan((batch, context, features), dtype, causal=True, normalize=False)
        assert (plan['workspace_bytes'] > 0) == (dtype != torch.bfloat16)
        for normalize, causal, act, vv, vd, eps in ((False, True, 'silu', v, None, 1e-6),
                                                    (True, False, 'gelu', None, valid, 0.25)):
            want = torch.ops.avey_kernels.contextualize(z, vv, gate, bias, vd, eps, 1e-12, causal, normalize, act)
            got = _noalloc(z, vv, gate, bias, vd, eps, causal, normalize, act)
            torch.cuda.synchronize()
            assert torch.equal(got, want), (dtype, batch, context, features, normalize)
