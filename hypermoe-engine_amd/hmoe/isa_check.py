"""Static check of compiled gfx950 code: no register of an untracked load is
touched before a wait that completes the load.

The grouped INT8 GEMM (csrc/hm_gemm_mfma.hip) loads its B fragments with
inline-asm buffer loads the compiler does not track, so the compiler inserts
no wait for them and the kernel's own `s_waitcnt vmcnt(N)` statements decide
when the registers are complete.  If register allocation ever copied,
spilled or read such a register before that wait, the kernel would compute
with stale data and no test could be relied on to notice.  This module reads
the assembly the compiler produced for the object and proves the contrary.

For every `buffer_load_dwordx4 v[...]` that writes VGPRs (not the LDS
variants, which write no registers), it follows every control-flow path from
the load, counting the vector memory instructions issued after it, until an
`s_waitcnt` whose vmcnt(N) has N <= that count: loads return in issue order,
so the load is then complete.  Any instruction on such a path that names one
of the load's destination registers (reads, writes, spills, copies, MFMA
operands) is a violation, and so is a path that reaches the end of the
kernel.  Loads the compiler itself tracks pass trivially (the compiler waits
before every use, and its counts never exceed the true count of younger
instructions), so the check covers every kernel of the file.
"""
from __future__ import annotations

import re
import sys
from pathlib import Path

_VMEM = re.compile(r"^(buffer_|global_|scratch_|flat_)")
_VMCNT = re.compile(r"vmcnt\((\d+)\)")
_KERNEL = re.compile(r"^([A-Za-z_][\w.$]*):")
_MAX_COUNT = 64  # vmcnt saturates at 63 on gfx9


def _vregs(op: str) -> set[int]:
    m = re.match(r"v\[(\d+):(\d+)\]$", op)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", op)
    return {int(m.group(1))} if m else set()


def _functions(text: str) -> list[tuple[str, list[list[str]], dict[str, int]]]:
    """Splits an assembly listing into functions: (name, instructions as
    operand lists, label -> instruction index)."""
    out = []
    name, ins, labels = None, [], {}
    for raw in text.split("\n"):
        line = raw.split(";")[0].strip()
        if not line:
            continue
        m = _KERNEL.match(line)
        if m and line.endswith(":") and not line.startswith("."):
            if name is not None:
                out.append((name, ins, labels))
            name, ins, labels = m.group(1), [], {}
            continue
        if line.endswith(":"):
            if name is not None:
                labels[line[:-1]] = len(ins)
            continue
        if line.startswith(".") or name is None:
            continue
        ins.append(line.replace(",", " ").split())
        if ins[-1][0] == "s_endpgm":
            out.append((name, ins, labels))
            name, ins, labels = None, [], {}
    if name is not None and ins:
        out.append((name, ins, labels))
    return out


def _decode(ins: list[list[str]], labels: dict[str, int]):
    """Per instruction: (register bitmask, is vector memory, vmcnt of a wait
    or None, successors, terminal reason or None)."""
    out = []
    for i, u in enumerate(ins):
        op = u[0]
        mask = 0
        for o in u[1:]:
            for r in _vregs(o):
                mask |= 1 << r
        m = _VMCNT.search(" ".join(u)) if op == "s_waitcnt" else None
        term = None
        if op == "s_endpgm":
            succ, term = [], "reaches s_endpgm"
        elif op.startswith("s_setpc") or op.startswith("s_swappc"):
            succ, term = [], "indirect branch"
        elif op == "s_branch":
            succ = [labels[u[1]]]
        elif op.startswith("s_cbranch"):
            succ = [i + 1, labels[u[1]]]
        else:
            succ = [i + 1]
        out.append((mask, bool(_VMEM.match(op)), int(m.group(1)) if m else None, succ, term))
    return out


def _check_function(ins: list[list[str]], labels: dict[str, int]) -> list[tuple[int, int, str]]:
    bad = []
    dec = None
    for p, t in enumerate(ins):
        if t[0] != "buffer_load_dwordx4" or "lds" in t or not t[1].startswith("v"):
            continue
        if dec is None:
            dec = _decode(ins, labels)
        dest = 0
        for r in _vregs(t[1]):
            dest |= 1 << r
        stack, seen = [(p + 1, 0)], set()
        while stack:
            i, c = stack.pop()
            if i >= len(ins):
                bad.append((p, i, "falls off the end of the function"))
                continue
            if (i, c) in seen:
                continue
            seen.add((i, c))
            mask, vmem, wait, succ, term = dec[i]
            if wait is not None and c >= wait:
                continue
            if mask & dest:
                bad.append((p, i, " ".join(ins[i])))
            if term:
                bad.append((p, i, term))
                continue
            c2 = min(c + 1, _MAX_COUNT) if vmem else c
            for n in succ:
                stack.append((n, c2))
    return bad


def check_text(text: str) -> list[str]:
    """Violations in an assembly listing, one line each (empty: clean)."""
    problems = []
    for name, ins, labels in _functions(text):
        for p, i, what in _check_function(ins, labels):
            problems.append(f"{name}: load #{p} ({' '.join(ins[p])}) -> instruction #{i}: {what}")
    return problems


def check_file(path: str | Path) -> list[str]:
    return check_text(Path(path).read_text())


if __name__ == "__main__":
    found = []
    for arg in sys.argv[1:]:
        found += check_file(arg)
    for line in found[:50]:
        print(line)
    print("clean" if not found else f"{len(found)} violation(s)")
    sys.exit(1 if found else 0)
