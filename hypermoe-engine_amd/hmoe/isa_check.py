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

Two further rules guard the hand-written blocks (between the compiler's
;;#ASMSTART and ;;#ASMEND markers):

- M0.  The LDS-DMA statements set M0 themselves and name it as clobbered,
  but the compiler treats M0 as a reserved register and ignores that
  clobber, so a value of its own kept in M0 across such a statement would
  be lost.  No instruction outside the blocks may therefore name M0 or use
  it implicitly (relative-index moves, messages, GWS and ordered-count LDS
  operations, the LDS forms of the memory loads).
- Vector memory inside the blocks.  Only the forms this check understands
  may appear there: the 16-byte VGPR buffer load (the untracked load above)
  and the LDS-DMA loads (buffer/global ... lds, which write no registers).
  Any other vector memory instruction (another width, an AGPR destination,
  a flat or global register load, a store) is refused, since its registers
  would escape the first rule.
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


def _functions(text: str, asm_flags: list | None = None
               ) -> list[tuple[str, list[list[str]], dict[str, int]]]:
    """Splits an assembly listing into functions: (name, instructions as
    operand lists, label -> instruction index).  With asm_flags, appends per
    function a list saying which instructions lie in a hand-written block."""
    out = []
    name, ins, labels = None, [], {}
    flags: list[bool] = []
    in_asm = False
    for raw in text.split("\n"):
        stripped = raw.strip()
        if stripped.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if stripped.startswith(";;#ASMEND"):
            in_asm = False
            continue
        line = raw.split(";")[0].strip()
        if not line:
            continue
        m = _KERNEL.match(line)
        if m and line.endswith(":") and not line.startswith("."):
            if name is not None:
                out.append((name, ins, labels))
                if asm_flags is not None:
                    asm_flags.append(flags)
            name, ins, labels, flags = m.group(1), [], {}, []
            continue
        if line.endswith(":"):
            if name is not None:
                labels[line[:-1]] = len(ins)
            continue
        if line.startswith(".") or name is None:
            continue
        ins.append(line.replace(",", " ").split())
        flags.append(in_asm)
        if ins[-1][0] == "s_endpgm":
            out.append((name, ins, labels))
            if asm_flags is not None:
                asm_flags.append(flags)
            name, ins, labels, flags = None, [], {}, []
    if name is not None and ins:
        out.append((name, ins, labels))
        if asm_flags is not None:
            asm_flags.append(flags)
    return out


# instructions that read or write M0 without naming it
_IMPLICIT_M0 = re.compile(r"^(s_movrel|v_movrel|s_sendmsg|ds_gws_|ds_append|ds_consume|"
                          r"ds_ordered_count|s_set_gpr_idx|v_interp_|s_ttracedata)")


def _uses_m0(u: list[str]) -> bool:
    if _IMPLICIT_M0.match(u[0]):
        return True
    if _VMEM.match(u[0]) and ("lds" in u[1:] or "_lds_" in u[0]):
        return True  # LDS-DMA loads address the LDS through M0
    return any(o == "m0" for o in u[1:])


def _asm_vmem_ok(u: list[str]) -> bool:
    """The vector memory forms allowed inside the hand-written blocks."""
    op, ops = u[0], u[1:]
    if op in ("global_load_lds_dwordx4", "global_load_lds_dword"):
        return True
    if op == "buffer_load_dwordx4" and "lds" in ops:
        return True
    return op == "buffer_load_dwordx4" and "offen" in ops and bool(ops) and ops[0].startswith("v")


def _check_blocks(ins: list[list[str]], flags: list[bool]) -> list[tuple[int, str]]:
    bad = []
    for i, (u, in_asm) in enumerate(zip(ins, flags)):
        if not in_asm and _uses_m0(u):
            bad.append((i, "M0 used outside a hand-written block"))
        if in_asm and _VMEM.match(u[0]) and not _asm_vmem_ok(u):
            bad.append((i, "unrecognised vector memory instruction in a hand-written block"))
    return bad


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
    flags: list[list[bool]] = []
    for (name, ins, labels), fl in zip(_functions(text, flags), flags):
        for p, i, what in _check_function(ins, labels):
            problems.append(f"{name}: load #{p} ({' '.join(ins[p])}) -> instruction #{i}: {what}")
        for i, what in _check_blocks(ins, fl):
            problems.append(f"{name}: instruction #{i} ({' '.join(ins[i])}): {what}")
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
