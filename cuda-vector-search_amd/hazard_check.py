"""Build-time check of MFMA result hazards in the gfx950 scan kernels.

    python cuda-vector-search_amd/hazard_check.py cvs_scan.s

A VALU instruction that reads VGPRs an MFMA writes must issue at least
passes + 4 wait states after it on gfx950 (32x32x16 f16 and 32x32x32 i8: 8
passes of 4 cycles, 16x16x32 f16: 4 passes).  With the MFMA accumulators in
VGPRs (-amdgpu-mfma-vgpr-form) this compiler separates an 8-pass MFMA from its
first VALU reader by only passes + 3, and the reader then sees a partial sum
(the score matrix intermittently lacked the last k-step).  The scan pads its
epilogue for it; this check walks every path of the built device assembly from
every MFMA (fall-through and branch targets, 1 wait state per instruction,
n + 1 per s_nop n) and fails the build on any read that comes too early, so a
code change cannot reintroduce the hazard unnoticed.  It reads only assembly
built in this tree.
"""

from __future__ import annotations

import re
import sys
from pathlib import Path

PASSES = {"v_mfma_f32_16x16x32_f16": 4, "v_mfma_f32_32x32x16_f16": 8, "v_mfma_i32_32x32x32_i8": 8,
          "v_mfma_f32_16x16x32_bf16": 4, "v_mfma_f32_32x32x16_bf16": 8}
EXTRA_WAIT_STATES = 4  # gfx950 XDL write -> VALU read: passes + 4


def operand_regs(tok: str) -> set[int]:
    """Registers named by one operand: VGPR n as n, AGPR n as 1000 + n."""
    m = re.fullmatch(r"([va])\[(\d+):(\d+)\]", tok)
    if m:
        base = 1000 if m[1] == "a" else 0
        return {base + r for r in range(int(m[2]), int(m[3]) + 1)}
    m = re.fullmatch(r"([va])(\d+)", tok)
    return {(1000 if m[1] == "a" else 0) + int(m[2])} if m else set()


def kernels(asm: str):
    """{kernel symbol: (instructions, {label: index})} of the device assembly."""
    out, cur = {}, None
    for raw in asm.splitlines():
        line = raw.split(";")[0].strip()
        if not line:
            continue
        m = re.fullmatch(r"(_Z\w+):", line)
        if m:
            cur = m[1]
            out[cur] = ([], {})
            continue
        if cur is None:
            continue
        if line.startswith(".Lfunc_end"):
            cur = None
            continue
        m = re.fullmatch(r"(\.L\w+):", line)
        if m:
            out[cur][1][m[1]] = len(out[cur][0])
        elif not line.startswith("."):
            out[cur][0].append(line)
    return out


def split(insn: str):
    op = insn.split()[0]
    return op, [t.strip() for t in insn[len(op):].split(",") if t.strip()]


def early_reads(insns, labels):
    """(mfma index, reader index, wait states, needed) for every VALU read of an
    MFMA's destination registers that comes too early on some path."""
    found = []
    for i, ins in enumerate(insns):
        op, args = split(ins)
        if not op.startswith("v_mfma") or not args:
            continue
        need = PASSES.get(op, 16) + EXTRA_WAIT_STATES
        dst = operand_regs(args[0])
        stack, seen = [(i + 1, 0)], set()
        while stack:
            j, ws = stack.pop()
            while j < len(insns) and ws < need and (j, ws) not in seen:
                seen.add((j, ws))
                o, a = split(insns[j])
                if o.startswith("v_") and not o.startswith("v_mfma"):
                    if any(operand_regs(t) & dst for t in a[1:]):
                        found.append((i, j, ws, need))
                        break
                if o.startswith("v_mfma") and a and operand_regs(a[0]) & dst and a[-1] != a[0]:
                    break  # overwritten (not accumulated) by another MFMA
                ws += int(a[0], 0) + 1 if o == "s_nop" else 1
                if o.startswith("s_cbranch") and a[0] in labels:
                    stack.append((labels[a[0]], ws))
                elif o == "s_branch":
                    if a and a[0] in labels:
                        stack.append((labels[a[0]], ws))
                    break
                elif o == "s_endpgm" or o.startswith("s_setpc"):
                    break
                j += 1
    return found


def check(path) -> list[str]:
    problems = []
    for name, (insns, labels) in kernels(Path(path).read_text()).items():
        for i, j, ws, need in early_reads(insns, labels):
            problems.append(f"{name}: '{insns[j]}' reads the result of '{insns[i]}' after {ws} of {need} "
                            "wait states")
    return problems


def main(argv):
    bad = []
    for p in argv[1:]:
        bad += check(p)
    for line in bad[:20]:
        print(line)
    print(f"{len(bad)} early MFMA result reads")
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
