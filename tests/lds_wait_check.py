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

pending_uses walks linearly: branches are not followed, so code of a
skipped arm is scanned in place, which over-approximates the pending set on
some paths and is exact on the straight-line hot loop. pending_uses_cfg walks
the control-flow graph instead (labels kept by kernels_with_labels), so a
branch arm is checked with the state of the paths that reach it, loops
included.
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


def kernels_with_labels(asm: str, prefix: str) -> dict:
    """As kernels(), but branch-target labels stay in the lists as "Lname:"
    entries (for pending_uses_cfg)."""
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
        lm = re.match(r"^(\.?L\w*):", s)
        if lm:
            out[cur].append(lm.group(1) + ":")
        elif s and not s.startswith((";", ".")):
            out[cur].append(s)
    return out


def _blocks(lines: list):
    """Basic blocks of a labelled instruction list: [(start, end)] over the
    instruction indices (labels removed), the label -> block map, and each
    block's successors."""
    instrs, labels_at = [], {}
    for ln in lines:
        if ln.endswith(":") and " " not in ln:
            labels_at.setdefault(len(instrs), []).append(ln[:-1])
        else:
            instrs.append(ln)
    starts = {0} | set(labels_at)
    for i, ins in enumerate(instrs):
        op = ins.split()[0]
        if op.startswith(("s_branch", "s_cbranch", "s_setpc", "s_endpgm")):
            starts.add(i + 1)
    starts = sorted(s for s in starts if s < len(instrs))
    blocks = [(s, (starts[k + 1] if k + 1 < len(starts) else len(instrs))) for k, s in enumerate(starts)]
    block_of = {s: k for k, (s, _) in enumerate(blocks)}
    label_block = {name: block_of[i] for i, names in labels_at.items() if i in block_of for name in names}
    succ = []
    for k, (s, e) in enumerate(blocks):
        last = instrs[e - 1].split()
        op = last[0]
        nxt = [k + 1] if k + 1 < len(blocks) else []
        if op == "s_branch":
            succ.append([label_block[last[1]]])
        elif op in ("s_cbranch_execz", "s_cbranch_execnz") and e - 2 >= s and instrs[e - 2].startswith("s_and_saveexec"):
            # the branch of a divergent if: its all-lanes-inactive outcome is not followed
            succ.append(nxt if op == "s_cbranch_execz" else [label_block[last[1]]])
        elif op.startswith("s_cbranch"):
            succ.append([label_block[last[1]]] + nxt)
        elif op.startswith(("s_setpc", "s_endpgm")):
            succ.append([])
        else:
            succ.append(nxt)
    return instrs, blocks, succ


def pending_uses_cfg(lines: list, counters=("lgkm",), max_states=256) -> list:
    """pending_uses along the control-flow graph of a labelled instruction
    list (kernels_with_labels): every branch edge is followed with the
    in-order counter state of the path that reaches it (each distinct state
    once per block; states are compared by their pending destination
    registers), so the arm a branch skips is not scanned in place. The
    all-lanes-inactive outcome of a divergent if (an exec branch right after
    s_and_saveexec: the taken edge of s_cbranch_execz, the fall-through of
    s_cbranch_execnz) is not followed: the kernels issue every memory
    operation that a static count includes with some lane active (a
    lane-subset copy or store always has lanes), which is the invariant those
    counts rest on. Other exec branches (loops over lanes) keep both edges."""
    instrs, blocks, succ = _blocks(lines)
    bad, seen = {}, {}
    work = [(0, ((), ()))]
    while work:
        k, state = work.pop()
        key = (tuple(d for d, _ in state[0]), tuple(d for d, _ in state[1]))
        if key in seen.setdefault(k, set()):
            continue
        if len(seen[k]) >= max_states:
            raise RuntimeError("too many counter states at one block")
        seen[k].add(key)
        pend = {"lgkm": [(set(d), i) for d, i in state[0]], "vm": [(set(d), i) for d, i in state[1]]}
        s, e = blocks[k]
        for n in range(s, e):
            ins = instrs[n]
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
                        bad[(n, at)] = (n, ins, at, instrs[at])
            if op.startswith("ds_"):
                pend["lgkm"].append((_regs(ops[0]) if op.startswith("ds_read") else set(), n))
            elif vmem:
                pend["vm"].append((_regs(ops[0]) if is_load else set(), n))
        # more pending operations than any counter can hold (lgkmcnt 15, vmcnt
        # 63) only arise in a loop without waits: keep the newest, so the walk
        # ends
        for cnt in ("lgkm", "vm"):
            pend[cnt] = pend[cnt][-64:]
        out = (tuple((frozenset(d), i) for d, i in pend["lgkm"]), tuple((frozenset(d), i) for d, i in pend["vm"]))
        for nk in succ[k]:
            work.append((nk, out))
    return [bad[key] for key in sorted(bad)]
