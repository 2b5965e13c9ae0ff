"""Static check of the copy-ring kernels' register spills (gfx950 assembly).

The FP8 decode kernels count their outstanding HBM -> LDS copies
(global_load_lds) with hand-written `s_waitcnt vmcnt(N)`. A scratch access
(register spill or reload) issued while such copies are in flight adds to
the same counter. A reload is a load: loads return in issue order, so it can
only make a later `vmcnt(N)` wait for more copies than it needs. A spill
store is not ordered with the loads: it may complete ahead of older copies,
and a hand-written wait would then no longer prove that a stage has landed.
A spill store is harmless where no copy can be outstanding: before the first
copy, or after a `s_waitcnt vmcnt(0)` on every path.

`ring_violations(asm, kernel)` runs that check as a forward dataflow over the
kernel's basic blocks: the state is "a copy may be outstanding", set by
global_load_lds, cleared by `s_waitcnt vmcnt(0)`, joined (or) at block
entries; any scratch_store reached in that state is reported (with
loads=True, reloads too).
"""
from __future__ import annotations

import re

_LABEL = re.compile(r"^(\.LBB\w+|\w+):")
_BB_COMMENT = re.compile(r"^; %bb\.\d+:")


def kernel_body(asm: str, symbol: str) -> list[str]:
    """The instruction lines of `symbol` (from its label to s_endpgm)."""
    lines = asm.splitlines()
    out, inside = [], False
    for ln in lines:
        if not inside:
            if ln.startswith(symbol + ":"):
                inside = True
            continue
        out.append(ln)
        if ln.strip().startswith("s_endpgm"):
            break
    return out


def _blocks(body: list[str]):
    """Basic blocks: (label or None, [instructions]) in layout order."""
    blocks, cur_label, cur = [], None, []
    for raw in body:
        ln = raw.split(";")[0].strip() if not raw.lstrip().startswith(";") else ""
        m = _LABEL.match(raw.strip())
        if m and not raw.startswith("\t"):
            blocks.append((cur_label, cur))
            cur_label, cur = m.group(1), []
            continue
        if _BB_COMMENT.match(raw.strip()):
            blocks.append((cur_label, cur))
            cur_label, cur = None, []
            continue
        if not ln or ln.startswith(".") or ln.startswith(";;"):
            continue
        cur.append(ln)
        op = ln.split()[0]
        if op.startswith("s_branch") or op.startswith("s_cbranch") or op == "s_endpgm" \
                or op.startswith("s_setpc"):
            blocks.append((cur_label, cur))
            cur_label, cur = None, []
    blocks.append((cur_label, cur))
    return [b for b in blocks if b[0] is not None or b[1]]


def ring_violations(asm: str, symbol: str, loads: bool = False) -> list[str]:
    blocks = _blocks(kernel_body(asm, symbol))
    index = {lab: i for i, (lab, _) in enumerate(blocks) if lab}
    succ = []
    for i, (_, ins) in enumerate(blocks):
        s = []
        last = ins[-1] if ins else ""
        op = last.split()[0] if last else ""
        if op.startswith("s_branch"):
            s.append(index[last.split()[1]])
        elif op.startswith("s_cbranch"):
            s.append(index[last.split()[1]])
            if i + 1 < len(blocks):
                s.append(i + 1)
        elif op != "s_endpgm" and i + 1 < len(blocks):
            s.append(i + 1)
        succ.append(s)

    def transfer(state, ins, report=None):
        for ln in ins:
            op = ln.split()[0]
            if op.startswith("global_load_lds"):
                state = True
            elif op == "s_waitcnt" and re.search(r"vmcnt\(0\)", ln):
                state = False
            elif (op.startswith("scratch_store") or (loads and op.startswith("scratch_load"))) \
                    and state and report is not None:
                report.append(ln)
        return state

    entry = [False] * len(blocks)
    seen = [False] * len(blocks)
    seen[0] = True
    work = [0]
    while work:
        i = work.pop()
        out = transfer(entry[i], blocks[i][1])
        for j in succ[i]:
            if not seen[j] or (out and not entry[j]):
                seen[j] = True
                entry[j] = entry[j] or out
                work.append(j)
    bad: list[str] = []
    for i, (_, ins) in enumerate(blocks):
        if seen[i]:
            transfer(entry[i], ins, bad)
    return bad
