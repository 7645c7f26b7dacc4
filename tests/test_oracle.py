"""Pin the CPU oracle before trusting it (CPU only).

Checks, each chosen so that a plausible slip in the oracle fails one of them:
* the reference's own hand-computed answers (tests/golden/kats.json);
* closed forms of every activation;
* agreement with the independent C restatement (oracle/avey_oracle.c, a
  per-query streaming loop) over every flag combination, tails and NaN padding;
* invariants: causal rows ignore the future, permutation equivariance of the
  bidirectional op, scale behaviour, Avey-B numerator = unweighted Avey;
* the causal tile-count rule against the reference's table and brute force;
* planted mistakes in the oracle (transposed V, strict causal mask, bias before
  the division) are caught by the known answers.
"""

import itertools
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import c_contextualize, load_kats
from oracle import avey_oracle as orc

KATS = load_kats()


def _run_kat(case, contextualize=orc.contextualize, acc=np.float64):
    dt = np.float64 if case['dtype'] == 'float64' else np.float32
    z = np.asarray(case['z_tr'], dtype=dt)
    v = np.asarray(case['v'], dtype=dt) if 'v' in case else None
    gate = np.asarray(case['z_tl'], dtype=dt) if 'z_tl' in case else None
    bias = np.asarray(case['bias'], dtype=dt) if 'bias' in case else None
    valid = np.asarray(case['valid'], dtype=bool) if 'valid' in case else None
    kw = dict(case['kwargs'])
    if case['op'] == 'avey':
        args = dict(eps=1e-6, causal=kw.get('causal', True), normalize=False)
    else:
        args = dict(eps=kw.get('eps', 1e-6), causal=False, normalize=True)
    return contextualize(z, v, gate, bias, valid, norm_eps=1e-12, activation=kw.get('activation', 'identity'),
                         acc=acc, **args)


def _check_kat(case, out):
    if 'expected_row0' in case:
        np.testing.assert_allclose(out[0, 0], case['expected_row0'], rtol=case['rtol'], atol=case['atol'])
    else:
        np.testing.assert_allclose(out, case['expected'], rtol=case['rtol'], atol=case['atol'])


@pytest.mark.parametrize('case', KATS['cases'], ids=[c['name'] for c in KATS['cases']])
@pytest.mark.parametrize('acc', [np.float64, np.float32])
def test_numpy_oracle_known_answers(case, acc):
    _check_kat(case, _run_kat(case, acc=acc))


@pytest.mark.parametrize('case', KATS['cases'], ids=[c['name'] for c in KATS['cases']])
def test_c_oracle_known_answers(case):
    def c_ctx(z, v, gate, bias, valid, acc=None, **kw):
        return c_contextualize(z, v, gate, bias, valid, **kw)
    _check_kat(case, _run_kat(case, contextualize=c_ctx))


def test_normalization_known_answer():
    kat = KATS['normalization']
    z = np.asarray(kat['z_tr'], dtype=np.float64)
    np.testing.assert_allclose(orc.normalize_rows(z, 1e-12), kat['expected'], rtol=0, atol=1e-15)
    # A zero row stays zero (the clamp, not a division by zero).
    assert np.all(orc.normalize_rows(np.zeros((1, 2, 3)), 1e-12) == 0)


def test_activation_closed_forms():
    x = np.array([-3.0, -1.0, 0.0, 1.0, 2.5])
    np.testing.assert_array_equal(orc.activate(x, 'identity'), x)
    np.testing.assert_array_equal(orc.activate(x, 'relu'), [0, 0, 0, 1, 2.5])
    np.testing.assert_array_equal(orc.activate(x, 'relu2'), [0, 0, 0, 1, 6.25])
    # silu(1) = 1 / (1 + e^-1); silu(-1) = -1 / (1 + e)
    np.testing.assert_allclose(orc.activate(np.array([1.0, -1.0, 0.0]), 'silu'),
                               [1 / (1 + math.exp(-1)), -1 / (1 + math.e), 0.0], rtol=1e-15)
    # tanh-GELU at +-1: 0.5 * x * (1 + tanh(sqrt(2/pi) * 1.044715 * x))
    t = math.tanh(math.sqrt(2 / math.pi) * 1.044715)
    np.testing.assert_allclose(orc.activate(np.array([1.0, -1.0]), 'gelu'), [0.5 * (1 + t), -0.5 * (1 - t)],
                               rtol=1e-15)
    # Large arguments: no overflow, correct limits.
    big = np.array([-800.0, 800.0])
    np.testing.assert_allclose(orc.activate(big, 'silu'), [0.0, 800.0], atol=1e-300)


@pytest.mark.parametrize('act', orc.ACTIVATIONS)
def test_activation_matches_torch_functional(act):
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1000, generator=g, dtype=torch.float64) * 4
    ref = {'identity': x, 'relu': F.relu(x), 'relu2': F.relu(x) ** 2, 'silu': F.silu(x),
           'gelu': F.gelu(x, approximate='tanh')}[act]
    np.testing.assert_allclose(orc.activate(x.numpy(), act), ref.numpy(), rtol=1e-13, atol=1e-15)


def _random_case(rng, b, c, d, nan_pad=True):
    z = rng.standard_normal((b, c, d))
    gate = rng.standard_normal((b, c, d))
    v = rng.standard_normal((c, c))
    bias = rng.standard_normal(d)
    valid = np.ones((b, c), dtype=bool)
    if c > 1:
        valid[0, -1] = False
    if b > 1:
        valid[1, : c // 2] = False
    if nan_pad:
        z[~valid] = np.nan
        gate[~valid] = np.nan
    return z, gate, v, bias, valid


@pytest.mark.parametrize('shape', [(1, 1, 1), (2, 5, 7), (2, 35, 37), (1, 67, 65)])
@pytest.mark.parametrize('causal,normalize,use_v', [(True, False, True), (False, False, True),
                                                    (False, True, False), (True, True, True)])
@pytest.mark.parametrize('act', orc.ACTIVATIONS)
def test_numpy_and_c_restatements_agree(shape, causal, normalize, use_v, act):
    rng = np.random.default_rng(hash((shape, causal, normalize, use_v, act)) % (2 ** 32))
    z, gate, v, bias, valid = _random_case(rng, *shape)
    kw = dict(eps=0.25, norm_eps=1e-12, causal=causal, normalize=normalize, activation=act)
    for vv, gg, bb, val in ((v if use_v else None, gate, bias, valid), (v if use_v else None, None, None, None)):
        zz = z if val is not None else np.nan_to_num(z)
        a = orc.contextualize(zz, vv, gg, bb, val, acc=np.float64, **kw)
        c = c_contextualize(zz, vv, gg, bb, val, **kw)
        assert np.all(np.isfinite(a))
        np.testing.assert_allclose(a, c, rtol=1e-10, atol=1e-12)


def test_nan_padding_never_reaches_valid_outputs():
    rng = np.random.default_rng(1)
    z, gate, v, bias, valid = _random_case(rng, 2, 9, 6)
    for causal, normalize in ((True, False), (False, True)):
        out = orc.contextualize(z, v, gate, bias, valid, eps=1e-6, norm_eps=1e-12, causal=causal,
                                normalize=normalize, activation='gelu')
        assert np.all(np.isfinite(out))
        assert np.all(out[~valid] == 0)


def test_causal_rows_ignore_future_rows():
    rng = np.random.default_rng(2)
    z = rng.standard_normal((1, 12, 5))
    v = rng.standard_normal((12, 12))
    base = orc.avey(z, v)
    z2 = z.copy()
    z2[0, 7:] = rng.standard_normal((5, 5))
    moved = orc.avey(z2, v)
    np.testing.assert_array_equal(base[0, :7], moved[0, :7])
    assert not np.allclose(base[0, 7:], moved[0, 7:])


def test_bidirectional_permutation_equivariance():
    rng = np.random.default_rng(3)
    z = rng.standard_normal((2, 10, 6))
    perm = rng.permutation(10)
    out = orc.avey_b(z, eps=0.5)
    out_p = orc.avey_b(z[:, perm], eps=0.5)
    np.testing.assert_allclose(out_p, out[:, perm], rtol=1e-12, atol=1e-12)


def test_avey_b_numerator_is_unweighted_bidirectional_avey():
    # avey_b(x) * (sum_j S_ij + eps) == avey(x, ones, causal=False): ties the
    # division path to the V path.
    rng = np.random.default_rng(4)
    z = rng.standard_normal((2, 8, 5))
    eps = 0.3
    zn = orc.normalize_rows(z, 1e-12)
    den = np.matmul(zn, np.swapaxes(zn, 1, 2)).sum(-1, keepdims=True) + eps
    np.testing.assert_allclose(orc.avey_b(z, eps=eps) * den, orc.avey(z, np.ones((8, 8)), causal=False),
                               rtol=1e-11, atol=1e-12)


def test_scaling_rows_scales_avey_output():
    # S is scale free, so avey(c * x) = c * avey(x) for c > 0 (identity activation).
    rng = np.random.default_rng(6)
    z = rng.standard_normal((1, 9, 4))
    v = rng.standard_normal((9, 9))
    np.testing.assert_allclose(orc.avey(3.5 * z, v), 3.5 * orc.avey(z, v), rtol=1e-12)


def test_fp32_oracle_within_1e5_of_fp64():
    rng = np.random.default_rng(7)
    z = rng.random((2, 35, 37)).astype(np.float32)
    v = rng.standard_normal((35, 35)).astype(np.float32)
    for fn in (lambda a: orc.avey(z, v, acc=a), lambda a: orc.avey_b(z, acc=a)):
        np.testing.assert_allclose(fn(np.float32), fn(np.float64), rtol=1e-5, atol=1e-5)


def test_key_tile_count_reference_table():
    table = KATS['causal_tile_counts']
    for case in table['cases']:
        c, bm, bn = case['c'], case['bm'], case['bn']
        n_tiles = len(case['expected'])
        for causal, skip in ((True, True), (True, False), (False, True)):
            got = [orc.key_tile_count(q, c, bm, bn, causal, skip) for q in range(n_tiles)]
            want = case['expected'] if (causal and skip) else [-(-c // bn)] * n_tiles
            assert got == want, (case, causal, skip)


@pytest.mark.parametrize('c,bm,bn', list(itertools.product((1, 5, 31, 32, 33, 64, 100, 256), (16, 32, 64),
                                                          (16, 32, 64))))
def test_key_tile_count_brute_force(c, bm, bn):
    # Causal skip keeps exactly the tiles holding an allowed pair (key <= query),
    # except that a context fitting in one key tile always uses that tile.
    for q in range(-(-c // bm)):
        queries = range(q * bm, min((q + 1) * bm, c))
        tiles = {k // bn for i in queries for k in range(i + 1)}
        want = 1 if c <= bn else max(tiles) + 1
        assert orc.key_tile_count(q, c, bm, bn, True) == want


def _variant_transposed_v(z, v, gate, bias, valid, **kw):
    return orc.contextualize(z, None if v is None else np.swapaxes(v, 0, 1), gate, bias, valid, **kw)


def _variant_strict_causal(z, v, gate, bias, valid, *, causal, **kw):
    out = orc.contextualize(z, v, gate, bias, valid, causal=False, **kw)
    if not causal:
        return out
    # Recompute with the diagonal dropped (j < i instead of j <= i).
    zz = np.asarray(z, dtype=np.float64)
    zn = orc.normalize_rows(zz, 1e-12)
    s = np.matmul(zn, np.swapaxes(zn, 1, 2)) * (1 if v is None else v)
    s = np.where(np.tril(np.ones(s.shape[-2:], bool), -1)[None], s, 0)
    return np.matmul(s, zz)


def _variant_bias_before_division(z, v, gate, bias, valid, *, normalize, eps, **kw):
    if not normalize or bias is None:
        return orc.contextualize(z, v, gate, bias, valid, normalize=normalize, eps=eps, **kw)
    zz = np.asarray(z, dtype=np.float64)
    zn = orc.normalize_rows(zz, 1e-12)
    s = np.matmul(zn, np.swapaxes(zn, 1, 2))
    num = np.matmul(s, zz) + bias
    y = orc.activate(num / (s.sum(-1, keepdims=True) + eps), kw['activation'])
    return y * (1 if gate is None else gate)


@pytest.mark.parametrize('variant', [_variant_transposed_v, _variant_strict_causal, _variant_bias_before_division])
def test_planted_mistakes_are_caught_by_known_answers(variant):
    caught = False
    for case in KATS['cases']:
        out = _run_kat(case, contextualize=variant)
        try:
            _check_kat(case, out)
        except AssertionError:
            caught = True
    assert caught, f'{variant.__name__} passes every known answer'


# row_condition: sum_j |S_ij| / |sum_j S_ij + eps| (the Avey-B denominator of
# ops.py:79-80). Closed forms on rows whose cosine similarities are +-1 or 0, so
# that a dropped eps (division by zero), eps added outside the absolute value, an
# absolute value inside the signed sum, or padded keys left in, each fail one case.
@pytest.mark.parametrize('z,valid,eps,want', [
    # S = [[1, -1], [-1, 1]]: both signed sums cancel to 0, so |0 + 0.5| sets it.
    ([[1., 0.], [-2., 0.]], None, 0.5, [4.0, 4.0]),
    # S = [[1,1,-1],[1,1,-1],[-1,-1,1]]: sums 1, 1, -1; |-1 + 0.25| = 0.75 for the last row.
    ([[1., 0.], [3., 0.], [-1., 0.]], None, 0.25, [3 / 1.25, 3 / 1.25, 3 / 0.75]),
    # Orthogonal rows: S = I.
    ([[3., 4.], [4., -3.]], None, 1e-6, [1 / (1 + 1e-6)] * 2),
    # A padded key (row 2) is dropped from both sums; the padded row itself has S = 0.
    ([[1., 0.], [-2., 0.], [7., 1.]], [True, True, False], 0.5, [4.0, 4.0, 0.0]),
])
def test_row_condition_closed_forms(z, valid, eps, want):
    z = np.asarray([z])
    valid = None if valid is None else np.asarray([valid])
    np.testing.assert_allclose(orc.row_condition(z, valid, eps=eps)[0], want, rtol=1e-12)


@pytest.mark.parametrize('use_v,causal', [(False, False), (True, False), (False, True), (True, True)])
def test_row_condition_matches_a_loop_over_keys(use_v, causal):
    rng = np.random.default_rng(11)
    z = rng.standard_normal((2, 9, 5))
    valid = rng.random((2, 9)) > 0.3
    v = rng.uniform(-1, 1, (9, 9)) if use_v else None
    got = orc.row_condition(z, valid, v=v, causal=causal, eps=0.1)
    for b in range(2):
        for i in range(9):
            zi = z[b, i] if valid[b, i] else np.zeros(5)
            s = [0.0 if not (valid[b, i] and valid[b, j]) or (causal and j > i) else
                 float(zi @ z[b, j]) / (np.linalg.norm(zi) * np.linalg.norm(z[b, j])) * (v[i, j] if use_v else 1.0)
                 for j in range(9)]
            assert abs(got[b, i] - sum(map(abs, s)) / abs(sum(s) + 0.1)) < 1e-12 * (1 + got[b, i])


def test_row_condition_weights_and_mask_closed_form():
    # S = [[1, -1], [-1, 1]] with V = [[1, 0.5], [2, 1]]: P = [[1, -0.5], [-2, 1]],
    # sums 0.5 and -1, so at eps = 0.5 the conditions are 1.5 / 1 and 3 / 0.5;
    # causal drops P_01, leaving 1 / 1.5 for row 0.
    z = np.asarray([[[1., 0.], [-2., 0.]]])
    v = np.asarray([[1., 0.5], [2., 1.]])
    np.testing.assert_allclose(orc.row_condition(z, v=v, eps=0.5)[0], [1.5, 6.0], rtol=1e-12)
    np.testing.assert_allclose(orc.row_condition(z, v=v, causal=True, eps=0.5)[0], [2 / 3, 6.0], rtol=1e-12)


@pytest.mark.parametrize('causal,normalize,use_v,act', [
    (True, False, True, 'identity'), (False, False, True, 'silu'), (False, True, False, 'gelu'),
    (False, True, False, 'relu2'), (True, False, False, 'relu')])
def test_torch_restatement_matches_numpy_oracle(causal, normalize, use_v, act):
    # oracle/avey_torch_ref.py (the CPU baseline bench.py times) against the numpy
    # oracle, in fp64 (agreement to rounding) and in fp32 / bf16 storage.
    from oracle import avey_torch_ref as tref
    g = torch.Generator().manual_seed(3)
    z = torch.randn(3, 19, 12, generator=g, dtype=torch.float64)
    gate = torch.randn(3, 19, 12, generator=g, dtype=torch.float64)
    bias = torch.randn(12, generator=g, dtype=torch.float64)
    v = torch.randn(19, 19, generator=g, dtype=torch.float64) if use_v else None
    valid = torch.rand(3, 19, generator=g) > 0.25
    z[~valid] = float('nan')
    kw = dict(eps=0.5, norm_eps=1e-12, causal=causal, normalize=normalize, activation=act)
    want = orc.contextualize(z.numpy(), None if v is None else v.numpy(), gate.numpy(), bias.numpy(),
                             valid.numpy(), acc=np.float64, **kw)
    got = tref.contextualize(z, v, gate, bias, valid, **kw)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-12, atol=1e-12)
    for dt in (torch.float32, torch.bfloat16):
        zz, gg, bb = (t.to(dt) for t in (z, gate, bias))
        vv = None if v is None else v.to(dt)
        got = tref.contextualize(zz, vv, gg, bb, valid, **kw)
        assert got.dtype == dt
        want = orc.contextualize(zz.double().numpy(), None if vv is None else vv.double().numpy(),
                                 gg.double().numpy(), bb.double().numpy(), valid.numpy(), acc=np.float32, **kw)
        tol = 1e-5 if dt == torch.float32 else 1e-2
        np.testing.assert_allclose(got.double().numpy(), want, rtol=tol, atol=tol)


def test_enricher_gate_hand_case_and_torch_linear():
    # x = [1, 2], W = [[1, -1], [0.5, 0.25]], b = [0.5, -1]: x W^T + b = [-0.5, 0], relu -> [0, 0],
    # identity -> [-0.5, 0], relu2 of [-0.5, 3] (b = [0.5, 2]) -> [0, 9].
    x = np.array([[1.0, 2.0]])
    w = np.array([[1.0, -1.0], [0.5, 0.25]])
    np.testing.assert_array_equal(orc.enricher_gate(x, w, np.array([0.5, -1.0]), 'identity'), [[-0.5, 0.0]])
    np.testing.assert_array_equal(orc.enricher_gate(x, w, np.array([0.5, -1.0]), 'relu'), [[0.0, 0.0]])
    np.testing.assert_array_equal(orc.enricher_gate(x, w, np.array([0.5, 2.0]), 'relu2'), [[0.0, 9.0]])
    g = torch.Generator().manual_seed(5)
    xt = torch.randn(2, 7, 24, generator=g, dtype=torch.float64)
    wt = torch.randn(40, 24, generator=g, dtype=torch.float64)
    bt = torch.randn(40, generator=g, dtype=torch.float64)
    for act, fn in (('relu', torch.relu), ('silu', torch.nn.functional.silu),
                    ('gelu', lambda t: torch.nn.functional.gelu(t, approximate='tanh'))):
        want = fn(torch.nn.functional.linear(xt, wt, bt)).numpy()
        np.testing.assert_allclose(orc.enricher_gate(xt.numpy(), wt.numpy(), bt.numpy(), act), want,
                                   rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(orc.enricher_gate(xt.numpy(), wt.numpy(), None, 'identity'),
                               torch.nn.functional.linear(xt, wt).numpy(), rtol=1e-12, atol=1e-12)

