"""Every LDS read of copied rows in the fused kernels waits for its copy.

The fused sources are compiled to gfx950 assembly with the library's own flags
and checked by tests/dma_waits.py (its docstring states the rules): per wave for
the 32- and 64-row kernels, and across the two roles of the 16-row kernel, whose
similarity waves copy the rows its mixing waves read. The first tests pin the
checker itself on small hand-written instruction sequences, so that the check
over the real kernels cannot pass by classifying nothing.
"""

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

import dma_waits as dw
from avey_kernel_amd import _build

KEY = ['ds_read_b128 v[10:13], v2', 'v_mfma_f32_16x16x32_bf16 v[20:23], v[10:13], v[30:33], v[20:23]']
QUERY = ['ds_read_b128 v[10:13], v2', 'v_mfma_f32_16x16x32_bf16 v[20:23], v[30:33], v[10:13], v[20:23]']
MIX = ['ds_read_b64_tr_b16 v[10:11], v2']
GATE = ['ds_read_b64 v[10:11], v2']
COPY = 'buffer_load_dwordx4 v1, s[0:3], 0 offen lds'
TOUCH = 'buffer_load_dword v1, s[0:3], 0 offen lds'
LOAD = 'buffer_load_dwordx2 v[4:5], v1, s[0:3], 0 offen'


def _bad(lines, bm=16, nk=8):
    bad, _ = dw.check_kernel(lines + ['s_endpgm'], bm, nk)
    return bad


def test_ring_geometry():
    # (R, copies per key tile, copies for the query rows, per wave): C2's variant
    # keeps three slots, 768-feature rows in the 32-row variant only two; the 32-
    # and 64-row variants split the copies between the two waves of a slice.
    assert dw.ring(16, 6) == (3, 12, 6)
    assert dw.ring(16, 8) == (2, 16, 8)
    assert dw.ring(32, 6) == (2, 6, 6)
    assert dw.ring(32, 8) == (2, 16, 16)
    assert dw.ring(64, 4) == (3, 4, 8)
    assert dw.ring(64, 6) == (2, 12, 24)


def test_refill_read_without_wait_is_flagged():
    # Two slots: the copy issued in the previous iteration filled the slot read now.
    assert _bad(['s_barrier', COPY, 's_barrier'] + KEY)
    assert not _bad(['s_barrier', COPY, 's_barrier', 's_waitcnt vmcnt(0)'] + KEY)
    # Three slots: a copy one iteration old (two barriers) is the next tile's.
    assert not _bad(['s_barrier', COPY, 's_barrier', 's_barrier'] + KEY, bm=16, nk=2)
    assert _bad(['s_barrier', COPY] + ['s_barrier'] * 3 + KEY, bm=16, nk=2)


def test_vmcnt_retires_in_issue_order():
    # vmcnt(N) leaves the N newest loads in flight: with two loads after the copy,
    # vmcnt(2) retires it and vmcnt(3) does not.
    seq = ['s_barrier', COPY, LOAD, LOAD, 's_barrier']
    assert not _bad(seq + ['s_waitcnt vmcnt(2)'] + KEY)
    assert _bad(seq + ['s_waitcnt vmcnt(3)'] + KEY)


def test_every_path_counts():
    # The wait sits on one arm of a branch only: the other arm reaches the read
    # with the copy in flight.
    seq = ['s_barrier', COPY, 's_barrier', 's_cbranch_scc1 .LBB0_2', 's_waitcnt vmcnt(0)', '.LBB0_2:']
    assert _bad(seq + KEY)
    assert not _bad(seq + ['s_waitcnt vmcnt(0)'] + KEY)


def test_prologue_and_gate_rules():
    bm, nk = 16, 2
    _, kdma, nq = dw.ring(bm, nk)
    queries, tile0 = [COPY] * nq, [COPY] * kdma
    assert _bad(queries + tile0 + QUERY, bm, nk)  # query rows not waited for
    # Waiting for the query rows only (tile 0 may still land) is enough for them.
    assert not _bad(queries + tile0 + [f's_waitcnt vmcnt({kdma})'] + QUERY, bm, nk)
    assert _bad(queries + tile0 + [f's_waitcnt vmcnt({kdma})'] + KEY, bm, nk)
    assert _bad([COPY] + GATE)
    assert not _bad([TOUCH] + GATE)  # a touch's landing place is never read
    assert not _bad([COPY, 's_waitcnt vmcnt(0)'] + GATE)


def test_mixing_read_rule():
    # Tile t's mixing operands are read at the end of iteration t: its own refill
    # (one barrier back) may be in flight, the previous one may not.
    assert not _bad(['s_barrier', COPY, 's_barrier'] + MIX)
    assert _bad(['s_barrier', COPY, 's_barrier', 's_barrier'] + MIX)


def test_query_split_needs_the_wait_before_the_barrier():
    # Both waves of a slice read the rows each one copied: a wait after the barrier
    # orders the copy for this wave only, not for its partner.
    bm, nk = 32, 6
    assert _bad(['s_barrier', COPY, 's_barrier', 's_waitcnt vmcnt(0)'] + KEY, bm, nk)
    assert not _bad(['s_barrier', COPY, 's_waitcnt vmcnt(0)', 's_barrier'] + KEY, bm, nk)
    assert _bad(['s_barrier', COPY, 's_barrier', 's_barrier', 's_waitcnt vmcnt(0)'] + MIX, bm, nk)
    assert not _bad(['s_barrier', COPY, 's_barrier', 's_waitcnt vmcnt(0)', 's_barrier'] + MIX, bm, nk)
    # A wave's own query and gate rows need only its own wait.
    assert not _bad([COPY, 's_waitcnt vmcnt(0)'] + GATE, bm, nk)
    _, kdma, nq = dw.ring(bm, nk)
    assert not _bad([COPY] * (nq + kdma) + [f's_waitcnt vmcnt({kdma})'] + QUERY, bm, nk)


def _bad16(lines, nk=6):
    bad, _ = dw.check16(lines + ['s_endpgm'], nk)
    return bad


def test_ring16_geometry():
    # (R, copies per similarity wave per tile): three 48 KB slots at 768 features,
    # two 64 KB ones at 1024.
    assert dw.ring16(6) == (3, 12)
    assert dw.ring16(8) == (2, 16)
    assert dw.ring16(2) == (3, 4)


def test_role_split_cross_wave_rules():
    r, kd = dw.ring16(6)
    tile = [COPY] * kd
    pro = [COPY] * 6 + tile + tile  # query rows, tile 0, tile 1
    bar = ['s_waitcnt lgkmcnt(0)', 's_barrier']
    # First barrier: only tile 1 (the newest kd copies) may still be in flight.
    assert not _bad16(pro + [f's_waitcnt vmcnt({kd})'] + bar + [f's_waitcnt vmcnt(0)'] + bar)
    assert _bad16(pro + [f's_waitcnt vmcnt({kd + 1})'] + bar + ['s_waitcnt vmcnt(0)'] + bar)
    # Tile 1 may pass the second barrier but not the third.
    seq = pro + [f's_waitcnt vmcnt({kd})'] + bar + bar
    assert not _bad16(seq + tile + [f's_waitcnt vmcnt({kd})'] + bar + ['s_waitcnt vmcnt(0)'] + bar)
    assert _bad16(seq + tile + bar + ['s_waitcnt vmcnt(0)'] + bar)
    # A refill may be in flight at the barrier that ends its interval (three slots),
    # not at the next one.
    loop = [f's_waitcnt vmcnt(0)'] + bar
    assert not _bad16(loop + tile + [f's_waitcnt vmcnt({kd})'] + bar + ['s_waitcnt vmcnt(0)'] + bar)
    assert _bad16(loop + tile + bar + bar + ['s_waitcnt vmcnt(0)'] + bar)
    # Two slots: no refill may cross a barrier.
    r8, kd8 = dw.ring16(8)
    tile8 = [COPY] * kd8
    assert _bad16([f's_waitcnt vmcnt(0)'] + bar + tile8 + bar + ['s_waitcnt vmcnt(0)'] + bar, nk=8)
    assert not _bad16([f's_waitcnt vmcnt(0)'] + bar + tile8 + ['s_waitcnt vmcnt(0)'] + bar + bar, nk=8)
    # The last barrier (the mixing waves read the gate rows after it): nothing in flight.
    assert _bad16(loop + [COPY] + bar)
    assert not _bad16(loop + [COPY, 's_waitcnt vmcnt(0)'] + bar)
    # Touches land in a word no one reads: never counted.
    assert not _bad16(loop + [TOUCH] + bar)
    # Every path counts: a wait on one arm of a branch only.
    br = ['s_cbranch_scc1 .LBB0_9', 's_waitcnt vmcnt(0)', '.LBB0_9:']
    assert _bad16(loop + [COPY] + br + bar)
    assert not _bad16(loop + [COPY, 's_waitcnt vmcnt(0)'] + br + bar)


def test_copy_or_pad_blocks_count_one_operation_on_either_path():
    # The inline-asm block issues a copy or a 4-byte pad (numeric local labels): a wait
    # that keeps the newest kd operations then retires every older copy on every path.
    r, kd = dw.ring16(6)
    block = ['s_cmp_eq_u32 s14, 0', 's_cbranch_scc1 1f', COPY, 's_branch 2f', '1:', 's_mov_b32 m0, s7', TOUCH, '2:']
    bar = ['s_waitcnt lgkmcnt(0)', 's_barrier']
    old = ['s_waitcnt vmcnt(0)'] + bar + [COPY] * kd
    assert not _bad16(old + block * kd + [f's_waitcnt vmcnt({kd})'] + bar + ['s_waitcnt vmcnt(0)'] + bar)
    # One operation short: an older copy survives the wait.
    assert _bad16(old + block * (kd - 1) + [f's_waitcnt vmcnt({kd})'] + bar + bar + ['s_waitcnt vmcnt(0)'] + bar)


def _compile(src, out_dir):
    out = os.path.join(out_dir, os.path.splitext(src)[0] + '.s')
    cmd = [_build.hipcc(), *_build.HIP_FLAGS, *_build.EXTRA_FLAGS.get(src, []), '--cuda-device-only', '-S',
           os.path.join(_build.CSRC, src), '-o', out]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return out


@pytest.mark.skipif(shutil.which('hipcc') is None and not os.path.exists('/opt/rocm/bin/hipcc'),
                    reason='hipcc not available')
def test_fused_kernels_wait_for_their_copies(tmp_path):
    sources = [s for s in _build.SOURCES if s.startswith('avey_fused_bm')]
    with ThreadPoolExecutor(max_workers=min(6, os.cpu_count() or 1)) as pool:
        files = list(pool.map(lambda s: _compile(s, str(tmp_path)), sources))
    checked = checked16 = 0
    problems = []
    for path in files:
        text = open(path).read()
        for name, (bad, counts, (bm, nk)) in dw.check_asm(text).items():
            checked += 1
            # Non-vacuous: the key, query, mixing and gate reads were all found.
            for role in ('A', 'Q', 'T', 'G'):
                assert counts.get(role, 0) > 0, (name, counts)
            problems += [(name, b) for b in bad[:3]]
        # The 16-row role-split kernels: copies of one wave read by another.
        for name, (bad, counts, nk) in dw.check_asm16(text).items():
            checked16 += 1
            assert counts['barrier'] > 0 and counts['prologue'] > 0, (name, counts)
            problems += [(name, b) for b in bad[:3]]
    assert checked >= 6 * 10, checked
    assert checked16 >= 4 * 24, checked16
    assert not problems, problems[:6]
