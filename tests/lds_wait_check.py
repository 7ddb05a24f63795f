"""Static check of the attention kernel's LDS read waits in compiled gfx950
assembly (test infrastructure).

The MFMA decode kernel issues its LDS reads as inline asm and waits for them
with counted ``s_waitcnt lgkmcnt(N)`` statements of its own, so the compiler
does not know when a read's destination registers are written. If it copies
or otherwise touches such a register between the read and the wait that
retires it, that instruction sees stale data. This module walks a kernel's
instructions in order with an in-order model of the LDS counter: every LDS
operation is pending until a wait retires it (``lgkmcnt(N)`` retires all but
the newest N), and any other instruction that reads or writes a register a
pending read will write is reported (vector-memory loads can be tracked the
same way against vmcnt).

The walk is linear: branches are not followed, so code of a skipped arm is
scanned in place. That over-approximates the pending set on some paths and
is exact on the straight-line hot loop.
"""

from __future__ import annotations

import re


def _regs(tok: str) -> set:
    tok = tok.strip()
    m = re.match(r"([va])\[(\d+):(\d+)\]", tok)
    if m:
        return {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r"([va])(\d+)\b", tok)
    if m:
        return {(m.group(1), int(m.group(2)))}
    return set()


def _operands(line: str) -> list:
    parts = line.split(None, 1)
    return re.split(r",\s*", parts[1]) if len(parts) > 1 else []


def kernels(asm: str, prefix: str) -> dict:
    """{symbol: [instruction lines]} for every function whose symbol starts
    with ``prefix`` in an assembly listing."""
    out, cur = {}, None
    for line in asm.splitlines():
        m = re.match(r"^(\S+):", line)
        if m and m.group(1).startswith(prefix):
            cur = m.group(1)
            out[cur] = []
            continue
        if cur is None:
            continue
        if line.startswith(".Lfunc_end"):
            cur = None
            continue
        s = line.strip()
        if s and not s.startswith((";", ".")) and not re.match(r"^\.?L\w*:", s):
            out[cur].append(s)
    return out


def _retire(pend: list, k: int) -> list:
    return [] if k == 0 else (pend[len(pend) - k:] if k < len(pend) else pend)


def _dead_high_half_read(instrs: list, n: int, pending: set) -> bool:
    """True when instruction n is a v_mad_u64_u32 whose only pending register
    is the high half of its 64-bit addend and whose result's high half is
    overwritten (next in program text) before anything reads it: the low 32 bits of a*b + c depend
    only on the low 32 bits of c, so the stale high half cannot reach a use.
    (The compiler forms such 64-bit addends from a 32-bit value and whatever
    the next register holds when it only keeps the low half of the sum.)"""
    ins = instrs[n]
    if ins.split()[0] != "v_mad_u64_u32":
        return False
    ops = _operands(ins)
    if len(ops) < 5:
        return False
    dst, addend = _regs(ops[0]), sorted(_regs(ops[4]))
    if len(addend) != 2 or (_regs(ops[4]) & pending) != {addend[1]}:
        return False
    if (_regs(ops[2]) | _regs(ops[3])) & pending:
        return False
    hi = max(dst)
    # like the rest of this module, the walk is linear: the next instruction
    # in program text that names the high half must overwrite it
    for later in instrs[n + 1:]:
        op = later.split()[0]
        if op.startswith(("s_setpc", "s_endpgm")):
            return False
        lops = _operands(later)
        reads = set()
        for o in (lops[1:] if lops else []):
            reads |= _regs(o)
        if hi in reads:
            return False
        if lops and hi in _regs(lops[0]) and not op.startswith(("ds_", "global_", "buffer_")):
            return True  # overwritten by a VALU result before any read
    return False


def pending_uses(instrs: list, counters=("lgkm",)) -> list:
    """Instructions that touch a register an unretired LDS read (counter
    "lgkm") or vector-memory load ("vm") will write. Vector-memory operations
    are modelled like LDS operations with their own in-order counter (stores
    and HBM->LDS copies count without a destination). A v_mad_u64_u32 that
    reads only the unused high half of a pending 64-bit addend
    (_dead_high_half_read) is not reported."""
    pend = {"lgkm": [], "vm": []}  # counter -> [(destination registers, index)]
    bad = []
    for n, ins in enumerate(instrs):
        op = ins.split()[0]
        if op == "s_waitcnt":
            for cnt in ("lgkm", "vm"):
                m = re.search(cnt + r"cnt\((\d+)\)", ins)
                if m:
                    pend[cnt] = _retire(pend[cnt], int(m.group(1)))
            continue
        ops = _operands(ins)
        is_load = op.startswith(("global_load", "buffer_load")) and "_lds_" not in op
        vmem = op.startswith(("global_", "buffer_", "scratch_"))
        reads_dest = op.startswith("ds_read") or is_load
        used = set()
        for o in ops[1:] if reads_dest else ops:
            used |= _regs(o)
        for cnt in counters:
            for dest, at in pend[cnt]:
                if dest & used and not _dead_high_half_read(instrs, n, dest & used):
                    bad.append((n, ins, at, instrs[at]))
        if op.startswith("ds_"):
            pend["lgkm"].append((_regs(ops[0]) if op.startswith("ds_read") else set(), n))
        elif vmem:
            pend["vm"].append((_regs(ops[0]) if is_load else set(), n))
    return bad
