"""Static check of the buffer-to-LDS copy waits in the fused kernel's gfx950 code.

The fused kernel stages key tiles, query rows and gate rows in LDS with
``buffer_load_dwordx4 ... lds`` (one instruction copies 64 lanes x 16 bytes). A
wave must execute ``s_waitcnt vmcnt(N)`` before it reads those rows, with N small
enough that the copy has retired. The compiler derives these waits from its own
tracking of which LDS object a copy writes, and that tracking has been seen to
drop a wait: a read of a ring slot whose refill was still in flight. Such a read
fails only when the copy is slow, so the parity tests catch it now and then at
best; this check finds it in the assembly.

Method: a dataflow over the control-flow graph of each kernel. For every copy
that may still be in flight at an LDS read it keeps the Pareto set, over paths,
of (vector-memory loads issued since, barriers passed since); a wait
``vmcnt(N)`` retires the copies with at least N loads after them (vector memory
returns in issue order). Reads are classified by the use of their result: key
operands (16-byte read feeding an MFMA A operand), query operands (B operand),
mixing operands (``ds_read_b64_tr_b16``) and the epilogue's gate words
(``ds_read_b64``). The rules, for a ring of R key slots:

* prologue copies (query rows, key tiles 0 .. R-2): before the first barrier no
  query-row copy may be in flight at a query read, and no query-row or tile-0
  copy at a key read; after it, no prologue copy at any key or mixing read;
* ring refills: a copy in flight at a key read has passed at most 2 (R - 2)
  barriers (an older one filled the slot being read); at a mixing read at most
  2 (R - 2) + 1 where the mixing operands are read at the end of the tile's own
  iteration (all but the 4-wave 64-row variants), else 2 (R - 1) (at the start
  of the next);
* gate reads: nothing in flight but the 4-byte cache-line touches, whose
  landing place is never read.

In the query-split variants (32 and 64 rows, see query_split) the two waves of a feature slice
each copy half of a key tile's rows and both read all of them, so a copy is
visible to the partner only once it retired before a barrier the partner then
passed. For those, a copy retired by a wait stays "pending" (counted as in
flight at key, mixing and prologue key reads) until the next barrier; the query
and gate rows a wave reads are its own copies, for which its own wait suffices.

Branch correlations are ignored (every path through the graph counts), so the
check can over-report but not miss a path.

The 16-row role-split kernel (fused16_kernel, check16) has its similarity waves
issue every copy and its mixing waves read their rows (transposed key operands,
gate rows). A copy is visible to another wave only once its issuing wave retired
it with a vmcnt wait and then passed a barrier the reader passes too; every
wave runs the same barrier sequence. In a ring of R key slots, tile t's copies
go out in the interval of tile t-R+1 and both roles read tile t after the
barrier that ends interval t-1, so at every barrier:

* the first: only the prologue's tile-1 copies (the newest per-tile count of
  the wave's vector-memory operations) may be in flight; the query rows and
  tile 0 are read after it;
* later: a prologue copy (tile 1) may be in flight only at the second (it is
  read after the third); a loop refill only at the first barrier after its
  issue with three slots, and at none with two;
* the last ones (those an s_endpgm follows with no barrier between): nothing,
  since the mixing waves read the gate rows after them.

The similarity waves' own reads follow from the same rules; the mixing waves
issue no copy, so their reads see only copies those rules already retired.
"""

import re
from collections import defaultdict

CAP_LOADS, CAP_BARRIERS = 64, 9
PENDING = 10 ** 6  # load count of a retired copy not yet ordered by a barrier (query split)
_KERNEL = re.compile(r'^(_ZN4avey16fused_fwd_kernelI\w+):', re.M)
_SHAPE = re.compile(r'fused_fwd_kernelI\w+?Li(\d+)ELi(\d+)ELb(\d)E')


def query_split(bm, nk):
    """Whether the (BM, NK) variant splits its query blocks over two waves per slice
    (the kernel's fused_query_split)."""
    return (bm == 32 and nk <= 6) or (bm == 64 and nk <= 4)


def ring(bm, nk):
    """(R, copies per key tile, copies for the query rows) one wave issues in a
    (BM, NK) variant, as the kernel's LDS geometry fixes them (query split: half)."""
    cpr = 4 * nk
    cprp = (cpr + 7) // 8 * 8
    tile = 4 * 32 * cprp * 16
    qb = bm // 16
    sx, px = 4 * 2 * qb * 64 * 16, (qb + 1) * 64 * 16
    ovf = tile if (bm > 32 and tile > sx + 2 * px) else sx + 2 * px  # two planes of P
    small = 4 * (4 * 32 + 32 + 4 * bm + bm + (qb + 1) * 2 * 4 * 16 + bm)
    r = 3 if 3 * tile + ovf + small <= 160 * 1024 else 2
    share = 2 if query_split(bm, nk) else 1
    return r, 32 * cprp // 64 // share, bm * cprp // 64 // share


def kernels(asm_text):
    """{symbol: [instruction or 'label:' strings]} for each fused kernel."""
    out = {}
    for m in _KERNEL.finditer(asm_text):
        name = m.group(1)
        body = asm_text[m.end():asm_text.index('.Lfunc_end', m.end())]
        lines = []
        for raw in body.split('\n'):
            t = ' '.join(raw.split(';')[0].split())
            if not t or (t.startswith('.') and not t.startswith('.LBB')):
                continue
            lines.append(t)
        out[name] = lines
    return out


def _local_labels(lines):
    """Give the numeric local labels of inline asm (`1:`, referenced as `1f` / `1b`)
    unique names and resolve the branches that use them."""
    out, defs = list(lines), {}
    for i, t in enumerate(lines):
        m = re.fullmatch(r'(\d+):', t)
        if m:
            out[i] = f'.Lnum{m.group(1)}_{i}:'
            defs.setdefault(m.group(1), []).append(i)
    for i, t in enumerate(out):
        parts = t.split()
        if len(parts) == 2 and parts[0].startswith(('s_branch', 's_cbranch')):
            m = re.fullmatch(r'(\d+)([fb])', parts[1])
            if m:
                cands = defs[m.group(1)]
                j = min(c for c in cands if c > i) if m.group(2) == 'f' else max(c for c in cands if c < i)
                out[i] = f'{parts[0]} .Lnum{m.group(1)}_{j}'
    return out


def _blocks(lines):
    lines = _local_labels(lines)
    blocks, cur, anon = [], ['entry', []], 0
    for t in lines:
        if t.endswith(':'):
            blocks.append(cur)
            cur = [t[:-1], []]
            continue
        cur[1].append(t)
        if t.split()[0].startswith(('s_branch', 's_cbranch', 's_endpgm', 's_setpc')):
            blocks.append(cur)
            anon += 1
            cur = [f'<fallthrough {anon}>', []]
    blocks.append(cur)
    index = {b[0]: k for k, b in enumerate(blocks)}
    succ = []
    for k, (_, ins) in enumerate(blocks):
        op = ins[-1].split() if ins else ['']
        nxt = [k + 1] if k + 1 < len(blocks) else []
        if op[0] == 's_branch':
            succ.append([index[op[1]]])
        elif op[0].startswith('s_cbranch'):
            succ.append([index[op[1]]] + nxt)
        elif op[0] in ('s_endpgm', 's_setpc_b64'):
            succ.append([])
        else:
            succ.append(nxt)
    return blocks, succ


def _is_vmem_load(t):
    # (Stores count in vmcnt as well; leaving them out only makes the check stricter.)
    return t.startswith(('buffer_load', 'global_load', 'flat_load', 'scratch_load'))


def _is_copy(t):
    return _is_vmem_load(t) and t.endswith(' lds')


def _is_touch(t):
    return t.startswith('buffer_load_dword ') and t.endswith(' lds')


def _front(pairs):
    out = []
    for q in pairs:
        out, _ = _add(out, q)
    return out


def _add(front, pair):
    loads, bars = pair
    if any(l2 <= loads and b2 >= bars for l2, b2 in front):
        return front, False
    return [p for p in front if not (loads <= p[0] and bars >= p[1])] + [pair], True


def _regs(tok):
    m = re.match(r'([va])\[(\d+):(\d+)\]$', tok)
    if m:
        return m.group(1), int(m.group(2)), int(m.group(3))
    m = re.match(r'([va])(\d+)$', tok)
    return (m.group(1), int(m.group(2)), int(m.group(2))) if m else None


def _role(flat, i):
    """'T' mixing, 'G' gate, 'A' key operand, 'Q' query operand, or None."""
    t = flat[i]
    if t.startswith('ds_read_b64_tr'):
        return 'T'
    if t.startswith('ds_read_b64 '):
        return 'G'
    if not t.startswith('ds_read_b128'):
        return None
    dst = _regs(t.split()[1].rstrip(','))
    if dst is None:
        return None
    for t2 in flat[i + 1:i + 600]:
        parts = [x.rstrip(',') for x in t2.split()]
        if parts[0].startswith('v_mfma') and len(parts) >= 4:
            for pos, tok in enumerate(parts[2:4]):
                r = _regs(tok)
                if r and r[0] == dst[0] and r[1] <= dst[1] and dst[2] <= r[2]:
                    return 'A' if pos == 0 else 'Q'
        if len(parts) > 1 and not parts[0].startswith(('ds_write', 'buffer_store', 'v_cmp', 's_')):
            r = _regs(parts[1])
            if r and r[0] == dst[0] and not (r[2] < dst[1] or r[1] > dst[2]):
                return None  # overwritten before any MFMA used it
    return None


def check_kernel(lines, bm, nk):
    """Violations [(read, rule)] and per-role read counts of one kernel."""
    r, kdma, nq = ring(bm, nk)
    qs = query_split(bm, nk)
    split = bm <= 32 or qs
    blocks, succ = _blocks(lines)
    order, gidx, flat, first_barrier = [], {}, [], None
    for k, (_, ins) in enumerate(blocks):
        for p, t in enumerate(ins):
            gidx[(k, p)] = len(flat)
            flat.append(t)
            if _is_copy(t) and not _is_touch(t):
                order.append((k, p))
            if t.startswith('s_barrier') and first_barrier is None:
                first_barrier = len(flat) - 1
    if first_barrier is None:
        first_barrier = len(flat)
    prologue = [s for s in order if gidx[s] < first_barrier]
    pro_q = set(prologue[:nq])
    pro_t0 = set(prologue[nq:nq + kdma])
    pro_all = set(prologue[:nq + (r - 1) * kdma])

    state_in = [None] * len(blocks)
    state_in[0] = {}
    work = [0]
    at_read = {}
    while work:
        k = work.pop(0)
        st = {s: list(f) for s, f in state_in[k].items()}
        for p, t in enumerate(blocks[k][1]):
            m = re.search(r'vmcnt\((\d+)\)', t) if t.startswith('s_waitcnt') else None
            if m:
                n = int(m.group(1))
                if qs:
                    st = {s: _front([q if q[0] < n else (PENDING, q[1]) for q in f]) for s, f in st.items()}
                else:
                    st = {s: [q for q in f if q[0] < n] for s, f in st.items()}
                st = {s: f for s, f in st.items() if f}
            elif t.startswith('s_barrier'):
                st = {s: [(q[0], min(q[1] + 1, CAP_BARRIERS)) for q in f if q[0] != PENDING] for s, f in st.items()}
                st = {s: f for s, f in st.items() if f}
            elif _is_vmem_load(t):
                st = {s: [(q[0] if q[0] == PENDING else min(q[0] + 1, CAP_LOADS), q[1]) for q in f]
                      for s, f in st.items()}
                if _is_copy(t) and not _is_touch(t):
                    st[(k, p)] = [(0, 0)]
            elif t.startswith('ds_read'):
                at_read[(k, p)] = st
        for s2 in succ[k]:
            if state_in[s2] is None:
                state_in[s2] = {s: list(f) for s, f in st.items()}
                work.append(s2)
                continue
            new, changed = {s: list(f) for s, f in state_in[s2].items()}, False
            for s, f in st.items():
                front = new.get(s, [])
                for q in f:
                    front, c = _add(front, q)
                    changed |= c
                new[s] = front
            if changed:
                state_in[s2] = new
                work.append(s2)

    lim_key = 2 * (r - 2)
    lim_mix = 2 * (r - 2) + 1 if split else 2 * (r - 1)
    counts, bad = defaultdict(int), []
    for (k, p), st in at_read.items():
        i = gidx[(k, p)]
        role = _role(flat, i)
        if role is None:
            continue
        counts[role] += 1
        for s, front in st.items():
            if role in ('G', 'Q'):  # the wave's own rows: pending copies have landed
                front = [q for q in front if q[0] != PENDING]
                if not front:
                    continue
            bars = max(q[1] for q in front)
            why = None
            if role == 'G':
                why = 'gate read with a copy in flight'
            elif i < first_barrier:
                if role == 'Q' and s in pro_q:
                    why = 'query read with a query-row copy in flight'
                elif role == 'A' and (s in pro_q or s in pro_t0):
                    why = 'tile-0 key read with a prologue copy in flight'
            elif role in ('A', 'T') and s in pro_all:
                why = 'prologue copy in flight after the first barrier'
            elif role == 'A' and bars > lim_key:
                why = f'key read with a copy {bars} barriers old in flight (at most {lim_key})'
            elif role == 'T' and bars > lim_mix:
                why = f'mixing read with a copy {bars} barriers old in flight (at most {lim_mix})'
            if why:
                bad.append((f'{blocks[k][0]}+{p}: {flat[i]}', f'{why}; copy at {blocks[s[0]][0]}+{s[1]}'))
    return bad, dict(counts)


def check_asm(asm_text):
    """{kernel: (violations, read counts, (BM, NK))} for every fused kernel in a file."""
    out = {}
    for name, lines in kernels(asm_text).items():
        m = _SHAPE.search(name)
        bm, nk = int(m.group(1)), int(m.group(2))
        bad, counts = check_kernel(lines, bm, nk)
        out[name] = (bad, counts, (bm, nk))
    return out


_KERNEL16 = re.compile(r'^(_ZN4avey14fused16_kernelI\w+):', re.M)
_SHAPE16 = re.compile(r'fused16_kernelI\w+?Li(\d+)ELb')


def ring16(nk):
    """(R, copies per similarity wave per key tile) of the 16-row role-split kernel
    with NK 32-feature steps per slice, as its LDS geometry fixes them (G16)."""
    cpr = 4 * nk
    cprp = (cpr + 7) // 8 * 8
    tile = 4 * 32 * cprp * 16
    small = 2 * (2 * 2 * 64 * 16) + 2 * 2 * 32 * 4 + 2 * 16 * 4 + 32 * 4 + 256
    r = 3 if 3 * tile + small <= 160 * 1024 else 2
    return r, 2 * (cprp // 4)


def kernels16(asm_text):
    out = {}
    for m in _KERNEL16.finditer(asm_text):
        name = m.group(1)
        body = asm_text[m.end():asm_text.index('.Lfunc_end', m.end())]
        lines = []
        for raw in body.split('\n'):
            t = ' '.join(raw.split(';')[0].split())
            if not t or (t.startswith('.') and not t.startswith('.LBB')):
                continue
            lines.append(t)
        out[name] = lines
    return out


def _dataflow(blocks, succ):
    """State (copy -> Pareto front of (loads since, barriers since)) before every
    instruction, keyed (block, position): plain per-wave counting, every path."""
    state_in = [None] * len(blocks)
    state_in[0] = {}
    work = [0]
    before = {}
    while work:
        k = work.pop(0)
        st = {c: list(f) for c, f in state_in[k].items()}
        for p, t in enumerate(blocks[k][1]):
            before[(k, p)] = st
            m = re.search(r'vmcnt\((\d+)\)', t) if t.startswith('s_waitcnt') else None
            if m:
                n = int(m.group(1))
                st = {c: [q for q in f if q[0] < n] for c, f in st.items()}
                st = {c: f for c, f in st.items() if f}
            elif t.startswith('s_barrier'):
                st = {c: [(q[0], min(q[1] + 1, CAP_BARRIERS)) for q in f] for c, f in st.items()}
            elif _is_vmem_load(t):
                st = {c: [(min(q[0] + 1, CAP_LOADS), q[1]) for q in f] for c, f in st.items()}
                if _is_copy(t) and not _is_touch(t):
                    st[(k, p)] = [(0, 0)]
        for s2 in succ[k]:
            if state_in[s2] is None:
                state_in[s2] = {c: list(f) for c, f in st.items()}
                work.append(s2)
                continue
            new, changed = {c: list(f) for c, f in state_in[s2].items()}, False
            for c, f in st.items():
                front = new.get(c, [])
                for q in f:
                    front, ch = _add(front, q)
                    changed |= ch
                new[c] = front
            if changed:
                state_in[s2] = new
                work.append(s2)
    return before


def check16(lines, nk):
    """Violations [(place, rule)] and per-kind counts of one 16-row role-split kernel."""
    r, kd = ring16(nk)
    blocks, succ = _blocks(lines)
    copies = [(k, p) for k, (_, ins) in enumerate(blocks) for p, t in enumerate(ins)
              if _is_copy(t) and not _is_touch(t)]
    # The prologue: what the entry reaches before any barrier (each role's code path
    # has its own), and the barriers that end it.
    prologue, first_barriers, seen, work = set(), set(), {0}, [0]
    while work:
        k = work.pop()
        for p, t in enumerate(blocks[k][1]):
            if t.startswith('s_barrier'):
                first_barriers.add((k, p))
                break
            if _is_copy(t) and not _is_touch(t):
                prologue.add((k, p))
        else:
            for s2 in succ[k]:
                if s2 not in seen:
                    seen.add(s2)
                    work.append(s2)
    before = _dataflow(blocks, succ)
    # Final barriers: an s_endpgm is reachable from them without another barrier.
    reach_end = set()
    changed = True
    while changed:
        changed = False
        for k, (_, ins) in enumerate(blocks):
            if k in reach_end:
                continue
            tail = ins
            for idx in range(len(ins) - 1, -1, -1):
                if ins[idx].startswith('s_barrier'):
                    tail = None
                    break
            ends = any(t.startswith('s_endpgm') for t in ins) or any(s2 in reach_end for s2 in succ[k])
            if tail is not None and ends:
                reach_end.add(k)
                changed = True
    bad, counts = [], defaultdict(int)
    for (k, p), st in before.items():
        t = blocks[k][1][p]
        if not t.startswith('s_barrier'):
            continue
        counts['barrier'] += 1
        rest = blocks[k][1][p + 1:]
        final = not any(x.startswith('s_barrier') for x in rest) and (
            any(x.startswith('s_endpgm') for x in rest) or any(s2 in reach_end for s2 in succ[k]))
        first = (k, p) in first_barriers
        for c, front in st.items():
            why = None
            if final:
                why = 'copy in flight at a last barrier'
            elif first:
                if any(q[0] >= kd for q in front) or r == 2:
                    why = 'query rows or tile 0 in flight at the first barrier'
            elif c in prologue:
                if max(q[1] for q in front) > (1 if r == 3 else 0):
                    why = 'prologue tile in flight past the barrier before its interval'
            elif r == 2 or max(q[1] for q in front) > 0:
                why = 'refill in flight at a barrier after the one that ends its interval'
            if why:
                bad.append((f'{blocks[k][0]}+{p}', f'{why}; copy at {blocks[c[0]][0]}+{c[1]}'))
    counts['copies'] = len(copies)
    counts['prologue'] = len(prologue)
    return bad, dict(counts)


def check_asm16(asm_text):
    """{kernel: (violations, counts, NK)} for every 16-row role-split kernel in a file."""
    out = {}
    for name, lines in kernels16(asm_text).items():
        nk = int(_SHAPE16.search(name).group(1))
        bad, counts = check16(lines, nk)
        out[name] = (bad, counts, nk)
    return out
