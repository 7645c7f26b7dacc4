"""The C ABI of libavey_hip.so, exercised without a GPU.

Checks that the library loads, exports exactly what include/avey_hip.h
declares, rejects bad arguments with the documented status codes before
touching a device, and that the host-only planning functions follow the
reference's causal tile rule (tests/test_causal_skip.py:52-60).
"""

import ctypes
import os
import re

import pytest
import torch

from avey_kernel_amd import _hip
from conftest import REPO, load_kats

HEADER = os.path.join(REPO, 'include', 'avey_hip.h')


def _lib():
    if not os.path.exists(_hip.library_path()):
        from avey_kernel_amd import _build
        _build.build(verbose=False)
    return _hip.load()


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return set(re.findall(r'\b(avey_[a-z_0-9]+)\s*\(', text))


def test_library_exports_every_declared_symbol():
    lib = _lib()
    declared = _declared_functions()
    assert declared == set(_hip.EXPORTS), declared ^ set(_hip.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.avey_abi_version() == _hip.ABI_VERSION == 5


def _args(**over):
    base = dict(z_tr=1 << 40, v=None, z_tl=None, bias=None, valid=None, out=(1 << 40) + (1 << 36),
                batch=2, context=35, features=37, dtype=2, causal=1, normalize=0, activation=0, eps=1e-6,
                norm_eps=1e-12, z_tr_row_stride=0, z_tr_batch_stride=0, z_tl_row_stride=0, z_tl_batch_stride=0)
    base.update(over)
    return _hip.AveyFwdArgs(*[base[f] for f, _ in _hip.AveyFwdArgs._fields_])


@pytest.mark.parametrize('over,code', [
    (dict(z_tr=None), -1), (dict(out=None), -1),
    (dict(batch=0), -2), (dict(context=0), -2), (dict(features=-3), -2),
    (dict(dtype=9), -3), (dict(activation=5), -4), (dict(activation=-1), -4),
    (dict(eps=0.0), -5), (dict(norm_eps=float('nan')), -5), (dict(eps=float('inf')), -5),
    (dict(causal=2), -8), (dict(normalize=-1), -8),
    (dict(out=(1 << 40) + 64), -9),
    # Strided z_tr / z_tl: a row stride below `features` or a negative batch stride.
    (dict(z_tr_row_stride=36), -10), (dict(z_tr_row_stride=74, z_tr_batch_stride=-1), -10),
    (dict(z_tl=(1 << 41), z_tl_row_stride=1), -10),
    # out inside z_tr's strided span (rows 74 elements apart: 2 * 35 * 74 * 2 bytes)
    # though past what a contiguous z_tr would cover (2 * 35 * 37 * 2 bytes).
    (dict(z_tr_row_stride=74, z_tr_batch_stride=35 * 74, out=(1 << 40) + 2 * 35 * 37 * 2 + 64), -9),
])
def test_argument_errors_return_status_before_any_device_work(over, code):
    lib = _lib()
    args = _args(**over)
    assert lib.avey_fwd(ctypes.byref(args), None, 0, None) == code
    assert lib.avey_fwd_noalloc(ctypes.byref(args), None) == code
    assert lib.avey_fwd_plan(ctypes.byref(args), ctypes.byref(_hip.AveyFwdPlan())) == code
    assert lib.avey_fwd_workspace_bytes(ctypes.byref(args)) == -1
    assert lib.avey_status_string(code).decode() not in ('', 'unknown status')


def _bwd_args(dout=(1 << 42), dz_tr=(1 << 43), dv=None, dz_tl=None, dbias=None, **over):
    return _hip.AveyBwdArgs(_args(**over), dout, dz_tr, dv, dz_tl, dbias)


@pytest.mark.parametrize('over,code', [
    (dict(dout=None), -1), (dict(dz_tr=None), -1), (dict(batch=0), -2), (dict(activation=7), -4),
    (dict(dtype=3), -11), (dict(features=1025), -11), (dict(batch=65536), -11),
    (dict(z_tr_row_stride=40, z_tr_batch_stride=35 * 40), -11),
    (dict(dz_tr=(1 << 40) + 64), -9),              # dz_tr inside z_tr
    (dict(dz_tr=(1 << 42) + 2), -9),               # dz_tr inside dout
    (dict(z_tl=1 << 41, dz_tl=(1 << 43) + 8), -9),  # dz_tl overlaps dz_tr
])
def test_backward_argument_errors(over, code):
    lib = _lib()
    args = _bwd_args(**over)
    assert lib.avey_bwd(ctypes.byref(args), None, 0, None) == code
    assert lib.avey_bwd_workspace_bytes(ctypes.byref(args)) == code
    assert lib.avey_status_string(code).decode() not in ('', 'unknown status')


def test_backward_workspace_layout():
    lib = _lib()
    up = lambda n: -(-n // 64) * 64  # noqa: E731
    b, c, d = 2, 35, 37
    plain = lib.avey_bwd_workspace_bytes(ctypes.byref(_bwd_args()))
    assert plain == 4 * (2 * up(b * c) + 2 * up(b * c * d))
    # dv and dbias accumulators only when both the input and its gradient are given.
    assert lib.avey_bwd_workspace_bytes(ctypes.byref(_bwd_args(dv=1 << 44))) == plain
    full = _bwd_args(v=1 << 41, dv=1 << 44, bias=(1 << 41) + (1 << 30), dbias=1 << 45)
    assert lib.avey_bwd_workspace_bytes(ctypes.byref(full)) == plain + 4 * (up(c * c) + up(d))
    # bf16 rows of a multiple of 8 features (16-byte aligned z_tr): the bf16 path keeps
    # z^T and dnum^T ([D][C rounded up to 128] bf16) and dnum in bf16 instead of fp32.
    d8, cp = 40, 128
    fast = lib.avey_bwd_workspace_bytes(ctypes.byref(_bwd_args(features=d8)))
    assert fast == 4 * (2 * up(b * c) + up(b * c * d8) + 2 * up(b * d8 * cp // 2) + up(b * c * d8 // 2))
    assert lib.avey_bwd_workspace_bytes(ctypes.byref(_bwd_args(features=d8, dtype=1))) == \
        4 * (2 * up(b * c) + 2 * up(b * c * d8))
    # Avey-B (normalize) computes in fp64 whatever the type: 8-byte parts, no bf16 copies.
    for dt, dd in ((2, d8), (0, d)):
        assert lib.avey_bwd_workspace_bytes(ctypes.byref(_bwd_args(features=dd, dtype=dt, normalize=1))) == \
            8 * (2 * up(b * c) + 2 * up(b * c * dd))
    # The launch refuses a short or misaligned workspace before touching a device.
    assert lib.avey_bwd(ctypes.byref(full), None, 0, None) == -6
    assert lib.avey_bwd(ctypes.byref(full), (1 << 46) + 4, 1 << 30, None) == -6


def test_null_args_pointer():
    lib = _lib()
    assert lib.avey_fwd(None, None, 0, None) == -1
    assert lib.avey_fwd_enriched(None, None) == -1


def _enriched_args(x=1 << 44, w_gate=1 << 45, b_gate=None, model_dim=384, gate_activation=1, **over):
    base = dict(features=768, context=256, batch=4)
    base.update(over)
    return _hip.AveyEnrichedArgs(_args(**base), x, w_gate, b_gate, model_dim, gate_activation)


@pytest.mark.parametrize('over,code', [
    (dict(batch=0), -2), (dict(activation=6), -4),            # checks of the op itself come first
    (dict(z_tl=1 << 41), -13),                                 # the gate is formed, not passed
    (dict(x=None), -13), (dict(w_gate=None), -13),
    (dict(x=(1 << 44) + 8), -13), (dict(b_gate=(1 << 46) + 2), -13),   # alignment
    (dict(model_dim=0), -13), (dict(model_dim=388), -13), (dict(model_dim=65544), -13),
    (dict(gate_activation=5), -13),
    (dict(dtype=0), -13), (dict(features=1032), -13),          # fp32, wider than the fused kernel
    (dict(features=770), -13),                                 # rows of a multiple of 8 only
    (dict(x=(1 << 40) + (1 << 36) + 64), -9),                  # out inside x
])
def test_enriched_argument_errors(over, code):
    lib = _lib()
    args = _enriched_args(**over)
    assert lib.avey_fwd_enriched(ctypes.byref(args), None) == code
    assert lib.avey_status_string(code).decode() not in ('', 'unknown status')


def test_key_tile_count_follows_reference_table():
    lib = _lib()
    for case in load_kats()['causal_tile_counts']['cases']:
        c, bm, bn = case['c'], case['bm'], case['bn']
        n = len(case['expected'])
        assert [lib.avey_key_tile_count(q, c, bm, bn, 1, 1) for q in range(n)] == case['expected']
        full = [-(-c // bn)] * n
        assert [lib.avey_key_tile_count(q, c, bm, bn, 1, 0) for q in range(n)] == full
        assert [lib.avey_key_tile_count(q, c, bm, bn, 0, 1) for q in range(n)] == full
    assert lib.avey_key_tile_count(5, 64, 16, 16, 1, 1) == -1  # tile past the context


def test_static_tile_table():
    _lib()
    # Headline config: bf16, causal, D=768 -> fused MFMA kernel, 4 x 192-feature wave slices.
    p = _hip.plan((16, 256, 768), torch.bfloat16, causal=True, normalize=False, has_v=True, has_gate=True,
                  has_bias=True)
    assert p['kernel'] == 'fused_mfma' and p['block_d'] == 192 and p['block_n'] == 32
    assert p['grid'] >= 256 and p['workspace_bytes'] == 0
    # The grid keeps every CU of the 256 busy where the shape allows it.
    for shape in ((32, 512, 768), (4, 2048, 1024), (256, 128, 512)):
        q = _hip.plan(shape, torch.bfloat16, causal=False, normalize=True)
        assert q['kernel'] == 'fused_mfma' and q['grid'] >= 256
    # Row blocks and threads per workgroup: 8 waves where a variant splits roles (16
    # rows) or query blocks (32 / 64 rows whose state fits 256 registers), 4 where it
    # needs 512 registers per lane.
    for shape, causal, bm, threads in (((16, 256, 768), True, 16, 512), ((32, 512, 768), False, 64, 256),
                                       ((4, 2048, 1024), True, 16, 512), ((256, 128, 512), False, 64, 512),
                                       ((64, 128, 256), False, 32, 512)):
        q = _hip.plan(shape, torch.bfloat16, causal=causal, normalize=True)
        assert (q['block_m'], q['threads']) == (bm, threads), shape
    # Causal skipping visits about half the key tiles of the full traversal.
    full = _hip.plan((4, 2048, 1024), torch.bfloat16, causal=False, normalize=False)
    half = _hip.plan((4, 2048, 1024), torch.bfloat16, causal=True, normalize=False)
    assert half["block_m"] == full["block_m"]
    assert abs(half['key_tile_steps'] / full['key_tile_steps'] - 0.5) < 0.02
    # fp32 / fp64 and very wide features take the generic kernel, which needs a workspace.
    for dt in (torch.float32, torch.float64):
        g = _hip.plan((2, 64, 64), dt, causal=True, normalize=False)
        assert g['kernel'] == 'generic_valu' and g['workspace_bytes'] == 2 * 64 * (8 if dt == torch.float64 else 4)
    assert _hip.plan((1, 8, 4096), torch.bfloat16, causal=False, normalize=True)['kernel'] == 'generic_valu'


def test_strided_views_choose_the_kernel_by_stride_alignment():
    _lib()
    shape = (16, 256, 768)
    # The two halves of a [B, C, 2D] enricher output: rows 2D apart, items C * 2D apart.
    halves = (2 * 768, 256 * 2 * 768)
    p = _hip.plan(shape, torch.bfloat16, causal=True, normalize=False, has_gate=True, z_tr_strides=halves,
                  z_tl_strides=halves)
    q = _hip.plan(shape, torch.bfloat16, causal=True, normalize=False, has_gate=True)
    assert p == q and p['kernel'] == 'fused_mfma'
    # Strides that are not whole 16-byte chunks take the generic kernel (any stride).
    for zs, gs in (((772, 256 * 772), (0, 0)), ((0, 0), (776, 256 * 776 + 4))):
        r = _hip.plan(shape, torch.bfloat16, causal=True, normalize=False, has_gate=True, z_tr_strides=zs,
                      z_tl_strides=gs)
        assert r['kernel'] == 'generic_valu', (zs, gs)
    # A batch item spanning 2^30 elements or more also leaves the fused kernel.
    wide = _hip.plan((1, 32768, 512), torch.bfloat16, causal=False, normalize=True, z_tr_strides=(32776, 0))
    assert wide['kernel'] == 'generic_valu'


def test_row_strides_of_torch_views():
    x = torch.empty(2, 5, 16)
    assert _hip.row_strides(x) == (0, 0) and _hip.row_strides(None) == (0, 0)
    assert _hip.row_strides(x[..., 8:]) == (16, 80)
    with pytest.raises(ValueError):
        _hip.row_strides(x.transpose(1, 2))


def test_noalloc_rejects_calls_beyond_its_scratch_before_any_device_work():
    # The generic fp32 kernel needs 4 bytes of scratch per (batch, context) row: 2 x
    # 600000 rows need 4.8 MB, past the 4 MiB static array of avey_fwd_noalloc.
    lib = _lib()
    assert _hip.NOALLOC_SCRATCH_BYTES == 4 << 20
    big = _args(dtype=0, context=600000)
    assert lib.avey_fwd_workspace_bytes(ctypes.byref(big)) == 2 * 600000 * 4
    assert lib.avey_fwd_noalloc(ctypes.byref(big), None) == -12
    assert 'AVEY_NOALLOC_SCRATCH_BYTES' in lib.avey_status_string(-12).decode()
    # At the limit the size check passes (the call then goes on to the device check).
    fits = _args(dtype=0, batch=1, context=(4 << 20) // 4)
    assert lib.avey_fwd_workspace_bytes(ctypes.byref(fits)) == 4 << 20
    assert lib.avey_fwd_noalloc(ctypes.byref(fits), None) != -12
