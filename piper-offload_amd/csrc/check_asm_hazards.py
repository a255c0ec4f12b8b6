"""Check the compiled gfx950 kernels for inline asm that races an MFMA.

gfx950 requires software wait states between an MFMA and a later VALU
instruction that reads or overwrites the MFMA's destination registers, or
overwrites its accumulator input (srcC), while the MFMA is in flight.  The
compiler inserts them (``s_nop``) for the instructions it emits, but not for
inline asm, whose operands it treats as ordinary registers.  An asm
instruction that touches such a register too early sees or leaves stale
values, depending on timing.

This script scans the device assembly that ``make`` keeps next to the
objects (``-save-temps=obj``; blocks between ``;;#ASMSTART`` and
``;;#ASMEND`` are inline asm).  For every asm VALU instruction it checks,
within one function and in program order, every MFMA issued fewer than
``NEED`` wait states before it (``s_nop n`` counts n + 1):

* the asm reads or writes a register the MFMA writes (RAW / WAW), or
* the asm writes a register the MFMA reads as its accumulator (WAR).

An MFMA is retired from the window once a compiler-emitted instruction
accesses one of its registers (the compiler padded that access, so the MFMA
has completed), and a register defined again stops being tracked.  ``NEED``
is 19, above the largest requirement of the 16x16x16 and 16x16x32 MFMAs these
kernels use, so a clean result needs no per-instruction table.  Branches are
read in layout order; the asm helpers are straight-line code inside unrolled
loop bodies, so the windows that matter are not split by a back edge.

Exit status 1 and one line per finding when any asm instruction is inside an
MFMA's window.
"""

from __future__ import annotations

import re
import sys
from pathlib import Path

NEED = 19
REG = re.compile(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b")
FUNC = re.compile(r"^([A-Za-z_][\w.$]*):")
NO_VGPR_DEF = ("v_cmp", "v_cmpx", "v_readlane", "v_readfirstlane")


def _regs(text: str) -> set[int]:
    out: set[int] = set()
    for m in REG.finditer(text):
        if m.group(1):
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
        else:
            out.add(int(m.group(3)))
    return out


def scan(path: Path) -> list[str]:
    findings: list[str] = []
    func, window, ws, in_asm = "?", [], 0, False
    with open(path) as fh:
        for line in fh:
            line = line.rstrip("\n")
            st = line.strip()
            m = FUNC.match(line)
            if m:
                func, window, ws = m.group(1), [], 0
                continue
            if st == ";;#ASMSTART":
                in_asm = True
                continue
            if st == ";;#ASMEND":
                in_asm = False
                continue
            s = st.split(";")[0].strip()
            if not s or s.startswith(".") or s.endswith(":"):
                continue
            op = s.split()[0]
            ws += int(s.split()[1], 0) + 1 if op == "s_nop" else 1
            if not op.startswith("v_"):
                continue
            parts = s.split(None, 1)[1].split(",") if " " in s else [""]
            dst = set() if op.startswith(NO_VGPR_DEF) else _regs(parts[0])
            src = _regs(",".join(parts[1:]))
            if in_asm:
                for w in window:
                    gap = ws - w["ws"] - 1
                    if gap < NEED and ((src | dst) & w["dst"] or dst & w["srcc"]):
                        findings.append(f"{path.name}: {func}: '{s}' {gap} wait states after '{w['text']}'")
            else:
                window = [w for w in window if not ((src | dst) & w["dst"] or dst & w["srcc"])]
            for w in window:
                w["dst"] -= dst
            if op.startswith(("v_mfma", "v_smfmac")):
                srcc = _regs(parts[3]) if len(parts) > 3 else set()
                window.append({"ws": ws, "dst": set(dst), "srcc": srcc, "text": s})
                window = window[-32:]
    return findings


def main(argv: list[str]) -> int:
    paths = [Path(p) for p in argv]
    if not paths:
        print("usage: check_asm_hazards.py <device .s files>", file=sys.stderr)
        return 2
    findings = [f for p in paths for f in scan(p)]
    for f in findings:
        print(f)
    print(f"check_asm_hazards: {len(paths)} files, {len(findings)} asm instructions inside an MFMA window")
    return 1 if findings else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
