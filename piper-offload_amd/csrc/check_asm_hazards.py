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

It also checks every vector-memory store of 12 or 16 bytes, compiler-emitted
or not: no instruction may overwrite the store's data registers fewer than
``STORE_NEED`` wait states after it.  Measured on gfx950, a VALU write to a
data register of a 16-byte buffer store in the very next instruction corrupts
what the store writes (the last lanes of each row of 16), and the compiler
does not pad it.  (8-byte stores followed at once by such a write exist in
kernels whose outputs are checked bit for bit, and never differed.)  A store
that needs a guard gets one in the source: an ``s_nop 1`` in inline asm that
takes the data registers as inputs, placed after the store.

Exit status 1 and one line per finding when any asm instruction is inside an
MFMA's window or a store's data is overwritten too early.
"""

from __future__ import annotations

import re
import sys
from pathlib import Path

NEED = 19
STORE_NEED = 2
WIDE_STORE = re.compile(r"^(global|buffer|flat|scratch)_store_(dwordx[34]|b96|b128)\b")
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
    stores: list[dict] = []  # recent wide stores: data registers and issue position
    with open(path) as fh:
        for line in fh:
            line = line.rstrip("\n")
            st = line.strip()
            m = FUNC.match(line)
            if m:
                func, window, ws, stores = m.group(1), [], 0, []
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
            parts = s.split(None, 1)[1].split(",") if " " in s else [""]
            # register defined by this instruction (VALU result or load destination)
            if op.startswith(("v_", "global_load", "buffer_load", "flat_load", "scratch_load", "ds_read", "ds_load")):
                written = set() if op.startswith(NO_VGPR_DEF) or " lds" in s else _regs(parts[0])
                stores = [t for t in stores if ws - t["ws"] - 1 < STORE_NEED]
                for t in stores:
                    if written & t["data"]:
                        findings.append(f"{path.name}: {func}: '{s}' overwrites the data of '{t['text']}' "
                                        f"{ws - t['ws'] - 1} wait states after it")
            if WIDE_STORE.match(op):
                data = _regs(parts[0] if op.startswith("buffer") else (parts[1] if len(parts) > 1 else ""))
                stores.append({"ws": ws, "data": data, "text": s})
            if not op.startswith("v_"):
                continue
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
    print(f"check_asm_hazards: {len(paths)} files, {len(findings)} findings (asm inside an MFMA window, "
          "store data overwritten early)")
    return 1 if findings else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
