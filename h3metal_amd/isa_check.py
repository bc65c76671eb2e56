"""Checks the gfx950 assembly of kernels that issue MFMAs from inline assembly for the two hazards the compiler
cannot see there (its own builtin MFMAs it protects itself):

* an access by any other instruction to the destination (accumulator) registers of an inline-assembly MFMA
  within 18 wait states after it (a 16-pass XDL result is written that late; reading earlier sees the old
  value, writing earlier is overwritten by it), except an MFMA of the same opcode whose srcC is exactly that
  destination (back-to-back accumulation, which the matrix unit forwards without wait states);
* a VALU write of a register that an MFMA reads, within 2 wait states before that MFMA;
* a VALU write of a register that a DPP instruction reads through its DPP operand (src0), within 2 wait states
  before it (the cross-lane butterflies of the row kernels are DPP fmacs written as assembly).

The scan is straight-line over each function (a conservative approximation across branches: pending results
are carried into the next block in layout order). Used by build.py on the sources it lists in ISA_CHECKED; also runnable as
`python -m h3metal_amd.isa_check file.s`.
"""

from __future__ import annotations

import re
import sys

XDL_WAIT = 18
VALU_TO_MFMA = 2
VALU_TO_DPP = 2


def _regs(tok: str) -> set:
    m = re.match(r"([av])\[(\d+):(\d+)\]", tok)
    if m:
        return {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r"([av])(\d+)$", tok)
    return {(m.group(1), int(m.group(2)))} if m else set()


def scan(text: str, name: str = "<asm>") -> list[str]:
    problems = []
    pending: dict = {}  # register -> wait states still to go after an inline-assembly MFMA wrote it
    recent: dict = {}   # register -> wait states since a VALU wrote it
    asm_dst: dict = {}  # register -> (opcode, destination operand) of the inline-assembly MFMA that wrote it
    in_asm = False
    for ln, line in enumerate(text.split("\n"), 1):
        s = line.strip()
        if s == ";;#ASMSTART":
            in_asm = True
            continue
        if s == ";;#ASMEND":
            in_asm = False
            continue
        if s.endswith(":") and not s.startswith((".", ";")) and not s.startswith(".LBB"):
            pending.clear()
            recent.clear()
            asm_dst.clear()
            continue
        if not s or s.startswith((".", ";", "//")):
            continue
        op = s.split()[0]
        args = [a.strip() for a in s[len(op):].split(",")] if len(s) > len(op) else []
        ws = int(s.split()[1], 0) + 1 if op == "s_nop" else 1
        if op.startswith("v_mfma"):
            dst = _regs(args[0])
            for r in set().union(*[_regs(a) for a in args[1:]]):
                if r in recent and recent[r] - 1 < VALU_TO_MFMA and r not in dst:
                    problems.append(f"{name}:{ln}: VALU write of {r} {recent[r] - 1} wait states before: {s}")
            # an MFMA of the same opcode that accumulates onto exactly the registers an inline-assembly MFMA wrote
            # (srcC = that vdst) needs no wait states (the matrix unit forwards the result); every other access
            # of pending registers is a hazard
            src_c = args[3] if len(args) > 3 else ""
            c_regs = _regs(src_c)
            chained = bool(c_regs) and all(r in pending and asm_dst.get(r) == (op, src_c) for r in c_regs)
            used = set().union(*[_regs(a) for a in args[1:3]]) | (set() if chained else c_regs)
            hit = sorted(r for r in used if pending.get(r, 0) > 0)
            if hit:
                problems.append(f"{name}:{ln}: {op} reads {hit[0]} {XDL_WAIT - pending[hit[0]]} wait states "
                                f"after its MFMA: {s}")
            if chained and args[0] == src_c:
                for r in c_regs:
                    pending.pop(r, None)
                    asm_dst.pop(r, None)
            if in_asm:
                for r in dst:
                    pending[r] = XDL_WAIT + 1  # reads k + 1 after k wait states: clear once k >= XDL_WAIT
                    asm_dst[r] = (op, args[0])
        elif not op.startswith("s_"):
            if op.endswith("_dpp") and len(args) > 1:
                for r in _regs(args[1]):
                    if r in recent and recent[r] - 1 < VALU_TO_DPP:
                        problems.append(f"{name}:{ln}: VALU write of {r} {recent[r] - 1} wait states before the DPP "
                                        f"read: {s}")
            used = set().union(*[_regs(a) for a in args]) if args else set()
            hit = sorted(r for r in used if pending.get(r, 0) > 0)
            if hit:
                problems.append(f"{name}:{ln}: {op} accesses {hit[0]} {XDL_WAIT - pending[hit[0]]} wait states "
                                f"after its MFMA: {s}")
            if op.startswith("v_") and args:
                for r in _regs(args[0]):
                    recent[r] = 0
        for r in list(pending):
            pending[r] -= ws
            if pending[r] <= 0:
                del pending[r]
        for r in list(recent):
            recent[r] += ws
            if recent[r] > max(VALU_TO_MFMA, VALU_TO_DPP) + 1:
                del recent[r]
    return problems


if __name__ == "__main__":
    bad = []
    for p in sys.argv[1:]:
        with open(p) as f:
            bad += scan(f.read(), p)
    print("\n".join(bad[:50]))
    print(f"{len(bad)} hazards")
    sys.exit(1 if bad else 0)
