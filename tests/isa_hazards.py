"""Static check of compiled gfx950 code (test infrastructure).

The forward grouped GEMM issues its packed-weight loads into registers with
inline assembly, so the compiler neither tracks them for wait counts nor knows
that their destination registers are written some time after issue.  Vector
memory loads have no interlock on their destination registers: an instruction
that reads them before a covering ``s_waitcnt vmcnt`` gets stale data, and one
that writes them (a reallocated temporary, a spill reload) is overwritten when
the load lands.  ``violations`` walks every control-flow path from each such
load until a ``s_waitcnt vmcnt(N)`` with at least N vector-memory operations
issued after the load on that path, and reports any instruction on the way
that reads or writes the load's destination registers.
"""
from __future__ import annotations

import re


def _regs(tok: str) -> set[int]:
    m = re.match(r'v\[(\d+):(\d+)\]', tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r'v(\d+)$', tok)
    return {int(m.group(1))} if m else set()


def function_body(asm: str, symbol: str) -> list[str]:
    """Lines of one function of a compiler .s listing."""
    lines = asm.split('\n')
    start = next(i for i, l in enumerate(lines) if l.startswith(symbol + ':'))
    end = next(i for i in range(start, len(lines)) if lines[i].startswith('.Lfunc_end'))
    return lines[start:end]


def violations(lines: list[str]) -> tuple[int, list[str]]:
    """(number of inline-asm register loads checked, list of hazards)."""
    ins, labels, in_asm = [], {}, False
    for l in lines:
        if ';;#ASMSTART' in l:
            in_asm = True
            continue
        if ';;#ASMEND' in l:
            in_asm = False
            continue
        t = l.split(';')[0].strip()
        m = re.match(r'^(\.LBB\d+_\d+):', t)
        if m:
            labels[m.group(1)] = len(ins)
            continue
        if not t or t.startswith('.') or t.endswith(':'):
            continue
        ins.append((t, in_asm))

    def succ(i):
        t = ins[i][0]
        op = t.split()[0]
        if op == 's_branch':
            return [labels[t.split()[1]]]
        if op.startswith('s_cbranch'):
            return [labels[t.split()[1]], i + 1]
        if op in ('s_endpgm', 's_setpc_b64'):
            return []
        return [i + 1]

    def touched(t):
        op = t.split()[0]
        ops = [o.strip() for o in re.split(r'[ ,]+', t)[1:] if o.strip()]
        r = set()
        for o in ops:
            r |= _regs(o)
        return r

    found, n = [], 0
    for i, (t, a) in enumerate(ins):
        if not (a and t.startswith('global_load_dwordx4 v')):
            continue
        n += 1
        dst = _regs(t.split()[1].rstrip(','))
        stack, seen = [(i + 1, 0)], set()
        while stack:
            j, newer = stack.pop()
            if j >= len(ins) or (j, min(newer, 64)) in seen:
                continue
            seen.add((j, min(newer, 64)))
            u = ins[j][0]
            op = u.split()[0]
            m = re.search(r'vmcnt\((\d+)\)', u)
            if op == 's_waitcnt' and m and newer >= int(m.group(1)):
                continue
            if touched(u) & dst:
                found.append(f"{t} -> {u}")
                break
            nn = newer + (1 if op.startswith(('global_', 'buffer_', 'scratch_', 'flat_')) else 0)
            stack.extend((s, nn) for s in succ(j))
    return n, found
