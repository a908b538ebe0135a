"""In-flight load check over a kernel's gfx950 assembly.

Some kernels issue buffer loads as inline assembly, which the compiler's wait-count pass does not
track: the kernel's own `s_waitcnt vmcnt(N)` must have covered a load before any instruction reads
or writes its destination registers. This walks a kernel's assembly along one execution path
(a fixed number of loop iterations, or none), keeps the loads in flight in issue order (vector
memory loads complete in order, so `vmcnt(N)` retires all but the newest N), and reports every
instruction that touches a register whose load has not been retired.

Path choice: the loop is found from the compiler's loop comments; a branch that jumps over a
block of direct-to-LDS loads goes into the alternative block of the same count that follows it
(the in-range and past-the-end variants of a step's loads), a branch over the loop header enters
or skips the loop as asked, and other forward branches fall through.
"""
from __future__ import annotations

import re


def _regs(tok: str) -> set[int]:
    m = re.match(r"^v\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"^v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def kernel_names(asm: str, prefix: str) -> list[str]:
    return re.findall(r"^(" + re.escape(prefix) + r"\w*):", asm, re.M)


def kernel_body(asm: str, name: str) -> list[str]:
    i = asm.index(name + ":")
    return asm[i:asm.index(".Lfunc_end", i)].split("\n")


def _plan(raw: list[str], enter_loop: bool):
    lab = {m.group(1): k for k, l in enumerate(raw) for m in [re.match(r"^(\.LBB\w+):", l)] if m}
    header = next((m.group(1) for l in raw for m in [re.match(r"^(\.LBB\w+):.*Inner Loop Header", l)] if m), None)
    latch = next((m.group(1) for l in raw for m in [re.match(r"^(\.LBB\w+):\s+;\s+in Loop", l)] if m), None)
    if header is None:
        raise ValueError("no loop")
    if latch is None or lab[latch] > lab[header]:
        latch = header
    exit_label = None
    k = lab[latch] + 1
    while k < len(raw):
        t = raw[k].split(";")[0].strip()
        m = re.match(r"^s_cbranch_\w+\s+(\.LBB\w+)", t)
        if m and m.group(1) != header:
            exit_label = m.group(1)
            break
        if k > lab[latch] + 1 and re.match(r"^\.LBB", raw[k]):
            break
        k += 1
    take = {}
    for k, l in enumerate(raw):
        t = l.split(";")[0].strip()
        m = re.match(r"^s_cbranch_(\w+)\s+(\.LBB\w+)", t)
        if not m or m.group(2) not in lab or m.group(2) == exit_label:
            continue
        tgt, end = m.group(2), lab[m.group(2)]
        if end <= k:
            q = k + 1
            while q < len(raw) and not raw[q].split(";")[0].strip().startswith("s_branch"):
                q += 1
            if any(" lds" in raw[r] for r in range(k + 1, q)):
                take[tgt] = False
            continue
        if k < lab[header] < end:
            take[tgt] = not enter_loop
        elif any(" lds" in raw[r] for r in range(k, end)):
            take[tgt] = m.group(1).startswith("scc")
        else:
            take[tgt] = False
    return lab, latch, exit_label, take


def simulate(raw: list[str], iterations: int, enter_loop: bool = True) -> dict:
    """Walks one path; returns {'hazards': [...], 'loads': n, 'max_in_flight': n, 'iterations': n}."""
    lab, latch, exit_label, take = _plan(raw, enter_loop)
    body = [l.split(";")[0].strip() for l in raw]
    q: list[set[int]] = []
    out = {"hazards": [], "loads": 0, "max_in_flight": 0, "iterations": 0}
    k = steps = it = 0
    while k < len(body) and steps < 50000:
        steps += 1
        line = body[k]
        if not line or line.startswith("."):
            k += 1
            continue
        parts = line.replace(",", " ").split()
        op, ops = parts[0], parts[1:]
        if op == "s_endpgm":
            break
        if op.startswith("s_waitcnt") and "vmcnt" in line:
            n = int(re.search(r"vmcnt\((\d+)\)", line).group(1))
            del q[:max(0, len(q) - n)]
        pending = set().union(*q) if q else set()
        touched = set().union(*[_regs(t) for t in ops]) if ops else set()
        if op.startswith("buffer_load") or op.startswith("global_load"):
            dest = set() if line.endswith(" lds") else _regs(ops[0])
            if touched & pending:
                out["hazards"].append((k, line))
            q.append(dest)
            out["loads"] += 1
            out["max_in_flight"] = max(out["max_in_flight"], len(q))
        elif touched & pending:
            out["hazards"].append((k, line))
        if op == "s_branch":
            it += ops[0] == latch
            k = lab[ops[0]]
            continue
        if op.startswith("s_cbranch"):
            tgt = ops[0]
            if tgt in take:
                if take[tgt]:
                    it += tgt == latch
                    k = lab[tgt]
                else:
                    k += 1
            elif tgt == latch:
                it += 1
                k = lab[tgt] if it < iterations else k + 1
            elif tgt == exit_label:
                k = lab[tgt] if it >= iterations else k + 1
            else:
                k += 1
            continue
        k += 1
    out["iterations"] = it
    return out
