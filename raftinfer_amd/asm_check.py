"""Build-time check of the prefill kernel's inline-asm MFMAs.

`prefill_mfma_kernel` issues its PV MFMAs as inline asm (so that the O^T
accumulators stay in AGPRs).  The compiler cannot see an MFMA inside asm, so
it neither inserts the wait states the MFMA's result needs before another
instruction reads it nor avoids placing a register copy of the accumulator
right after it.  If it ever places such a copy, the copy reads the
accumulator before the MFMA has written it and the results are wrong
(a code change that let this happen computed wrong prefill outputs).  The
build therefore scans the kernel's gfx950 assembly and fails on any read of
an inline-asm MFMA's destination AGPRs within the MFMA's result latency.
"""
from __future__ import annotations

import re

# Wait states a v_mfma_f32_32x32x16_bf16 result (16 passes) needs before a
# VALU or v_accvgpr read of it; the kernel's own drain after each tile's PV
# batch gives 20 (s_nop 7, s_nop 7, s_nop 3).
RESULT_WAIT_STATES = 19

_AGPR_RANGE = re.compile(r"^a\[(\d+):(\d+)\]$")
_AGPR_ONE = re.compile(r"^a(\d+)$")
_NOP = re.compile(r"^s_nop\s+(\d+)")


def _agprs(operand: str):
    operand = operand.strip()
    m = _AGPR_RANGE.match(operand)
    if m:
        return int(m.group(1)), int(m.group(2))
    m = _AGPR_ONE.match(operand)
    if m:
        return int(m.group(1)), int(m.group(1))
    return None


def asm_mfma_hazards(assembly: str) -> list[str]:
    """Reads of an inline-asm MFMA's destination AGPRs issued fewer than
    RESULT_WAIT_STATES wait states after it (s_nop n counts n + 1, any other
    instruction 1).  Code is followed in listing order, labels included, so a
    fall-through is checked like straight-line code; a taken branch is not
    followed (the kernel drains its asm MFMAs before each loop back-edge).
    Reads by other MFMAs are not checked: the kernel's accumulators feed only
    the next MFMA of their own chain, which the hardware's dependency check
    covers."""
    hazards: list[str] = []
    pending: list[list[int]] = []  # [first AGPR, last AGPR, wait states left, line]
    in_asm = False
    for number, raw in enumerate(assembly.splitlines(), 1):
        text = raw.strip()
        if text.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if text.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if not text or text.startswith((";", ".")) or text.endswith(":"):
            continue
        opcode = text.split()[0]
        operands = [x for x in text[len(opcode):].split(",")]
        nop = _NOP.match(text)
        if opcode.startswith("v_mfma"):
            if in_asm:
                dest = _agprs(operands[0])
                if dest is not None:
                    pending.append([dest[0], dest[1], RESULT_WAIT_STATES, number])
                    continue
        elif nop is None:
            for operand in operands[1:]:
                src = _agprs(operand)
                if src is None:
                    continue
                for first, last, left, line in pending:
                    if left > 0 and not (src[1] < first or src[0] > last):
                        hazards.append(f"line {number}: '{text}' reads a[{first}:{last}], written by the "
                                       f"inline-asm MFMA at line {line}, after "
                                       f"{RESULT_WAIT_STATES - left} wait states")
        step = int(nop.group(1)) + 1 if nop else 1
        for entry in pending:
            entry[2] -= step
        pending = [entry for entry in pending if entry[2] > 0]
    return hazards
