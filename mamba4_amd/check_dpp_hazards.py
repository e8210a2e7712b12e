"""Static check of the hand-written DPP instructions in compiled gfx950 code.

rows16.hpp emits DPP instructions (``v_fmac_f32_dpp``, ``v_mov_b32_dpp``)
through inline asm, which the compiler's hazard recognizer does not
inspect.  GFX9 requires two wait states between a VALU instruction that
writes a VGPR and a DPP instruction that reads it.  This script reads the
AMD assembly of our own build and fails if any DPP instruction inside an
inline-asm block reads, as its DPP source, a VGPR written by a VALU
instruction fewer than two wait states earlier (every instruction counts
one wait state, ``s_nop N`` counts N+1).  After a label or branch the
history is unknown, so such a DPP instruction within two wait states of one
is also reported.  DPP instructions the compiler emits itself are covered by
its own hazard recognizer and are not checked.
"""

import re
import sys

_REG = re.compile(r"v\[(\d+):(\d+)\]|v(\d+)")


def _regs(text):
    out = set()
    for m in _REG.finditer(text):
        if m.group(3) is not None:
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def check(asm_text):
    """Return a list of violation descriptions (empty when the code is safe)."""
    problems = []
    history = []  # (wait states since, set of VGPRs written) for recent VALU writes
    unknown = 0  # wait states left during which the history is unknown
    kernel = "?"
    in_asm = False
    for line_no, raw in enumerate(asm_text.splitlines(), 1):
        if ";;#ASMSTART" in raw:
            in_asm = True
        elif ";;#ASMEND" in raw:
            in_asm = False
        line = raw.split(";")[0].strip()
        if not line or line.startswith("."):
            if line.startswith(".type") or line.startswith(".globl"):
                kernel = line.split()[-1].split(",")[0]
            continue
        if line.endswith(":"):
            history, unknown = [], 2
            continue
        mnemonic, _, operands = line.partition(" ")
        if in_asm and mnemonic.endswith("_dpp"):
            ops = [o.strip() for o in operands.split(",")]
            src0 = _regs(ops[1])
            if unknown > 0:
                problems.append(f"{kernel}:{line_no}: DPP instruction right after a label/branch")
            for age, written in history:
                if age < 2 and written & src0:
                    problems.append(f"{kernel}:{line_no}: {line} reads v{sorted(written & src0)} "
                                    f"written {age} wait state(s) earlier")
        waits = int(operands) + 1 if mnemonic == "s_nop" else 1
        history = [(age + waits, w) for age, w in history if age + waits < 2]
        unknown = max(0, unknown - waits)
        if mnemonic.startswith("s_branch") or mnemonic.startswith("s_cbranch"):
            history, unknown = [], 2
        if mnemonic.startswith("v_") and not mnemonic.startswith("v_cmp"):
            ops = operands.split(",")
            # v_permlane16_swap / v_permlane32_swap write both of their operands.
            written = _regs(ops[0]) | (_regs(ops[1]) if "_swap" in mnemonic else set())
            if written:
                history.append((0, written))
    return problems


def main(paths):
    bad = []
    for path in paths:
        bad += [f"{path}: {p}" for p in check(open(path).read())]
    for p in bad:
        print(p, file=sys.stderr)
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
