"""Wait-state check of the kernels' inline asm in the gfx950 assembly of this build.

The compiler inserts the wait states a hardware hazard needs (``s_nop``) only
between instructions it generated itself; an inline-asm block is opaque to that
check, so the block has to carry its own.  Three hazards can reach one here:

* a VMEM instruction (``buffer_``/``global_``/``flat_``) may read an SGPR only 5
  wait states after a VALU instruction wrote it -- the compiler keeps buffer
  descriptors spilled in VGPR lanes and reloads them with ``v_readlane_b32`` right
  before a block;
* a VALU instruction may read the result of ``v_mfma_f32_16x16x32_f16`` only 8
  wait states after the MFMA issued;
* a VALU instruction may read the result of a transcendental VALU instruction
  (``v_exp``, ``v_log``, ``v_rcp``, ``v_rsq``, ``v_sqrt``, ``v_sin``, ``v_cos``) only 1
  wait state after it.

For every VMEM or VALU instruction inside an ``;;#ASMSTART`` / ``;;#ASMEND`` block,
``check`` walks back over every control-flow path (fall-through and each branch
to a label) counting wait states (1 per instruction, N + 1 per ``s_nop N``) and
reports a hazardous writer of one of its source registers found too close.

Usage: ``make asm ASMDIR=<dir>`` in this folder, then
``python asm_hazards.py <dir>/*.s`` (exit status 1 when a hazard is found).
"""
from __future__ import annotations

import re
import sys

VALU_SGPR_WAIT = 5   # VALU writes an SGPR -> VMEM reads it
MFMA_VALU_WAIT = 8   # v_mfma_f32_16x16x32_f16 writes a VGPR -> VALU reads it
TRANS_VALU_WAIT = 1  # a transcendental VALU op writes a VGPR -> VALU reads it
_TRANS = re.compile(r"^v_(exp|log|rcp|rsq|sqrt|sin|cos)_")
_HORIZON = max(VALU_SGPR_WAIT, MFMA_VALU_WAIT)


def _regs(text: str, kind: str) -> set:
    out = set()
    for m in re.finditer(kind + r"\[(\d+):(\d+)\]", text):
        out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    for m in re.finditer(r"\b" + kind + r"(\d+)\b", text):
        out.add(int(m.group(1)))
    return out


def _split(line: str) -> tuple:
    parts = line.split(None, 1)
    return parts[0], (parts[1] if len(parts) > 1 else "")


def check(asm_text: str) -> tuple:
    """Returns (number of inline-asm VMEM / VALU instructions checked, list of
    hazards as strings)."""
    lines = []
    for raw in asm_text.split("\n"):
        s = raw.strip()
        lines.append(s if s.startswith(";;#ASM") else raw.split(";")[0].strip())
    preds: dict = {}
    for k, line in enumerate(lines):
        m = re.match(r"^s_c?branch\w*\s+(\.LBB\w+)", line)
        if m:
            preds.setdefault(m.group(1), []).append(k)

    def walk(k, ws, need_s, need_v, seen, hits):
        kk = k - 1
        while kk >= 0 and ws < _HORIZON:
            t = lines[kk]
            if not t or t.startswith(";;#ASM") or (t.startswith(".") and not t.endswith(":")):
                kk -= 1
                continue
            if t.endswith(":"):  # a label: every branch to it is a predecessor too
                lab = t[:-1]
                if (lab, ws) in seen:
                    return
                seen.add((lab, ws))
                for b in preds.get(lab, []):
                    walk(b + 1, ws, need_s, need_v, seen, hits)
                p = kk - 1
                while p >= 0 and (not lines[p] or lines[p].startswith(";;#ASM")):
                    p -= 1
                if p >= 0 and (lines[p].startswith("s_branch") or lines[p].startswith("s_endpgm")):
                    return  # no fall-through into the label
                kk -= 1
                continue
            op, args = _split(t)
            dst = args.split(",")[0] if args else ""
            if need_s and op.startswith("v_") and ws < VALU_SGPR_WAIT and _regs(dst, "s") & need_s:
                hits.append(f"VALU writes an SGPR {ws} wait states before: {t}")
            if need_v and op.startswith("v_mfma") and ws < MFMA_VALU_WAIT and _regs(dst, "v") & need_v:
                hits.append(f"MFMA writes a VGPR {ws} wait states before: {t}")
            if need_v and _TRANS.match(op) and ws < TRANS_VALU_WAIT and _regs(dst, "v") & need_v:
                hits.append(f"a transcendental op writes a VGPR {ws} wait states before: {t}")
            ws += int(args.strip()) + 1 if op == "s_nop" else 1
            kk -= 1

    checked, hazards = 0, []
    in_asm = False
    for k, line in enumerate(lines):
        if line.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if line.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if not in_asm or not line or line.startswith(".") or line.endswith(":"):
            continue
        op, args = _split(line)
        is_vmem = op.startswith(("buffer_", "global_", "flat_"))
        is_valu = op.startswith("v_") and not op.startswith("v_mfma")
        if not (is_vmem or is_valu):
            continue
        checked += 1
        srcs = args.split(",", 1)[1] if (is_valu and "," in args) else args
        hits: list = []
        walk(k, 0, _regs(srcs, "s") if is_vmem else set(), _regs(srcs, "v") if is_valu else set(), set(), hits)
        hazards += [f"line {k + 1}: {line} <- {h}" for h in hits]
    return checked, hazards


def main(paths) -> int:
    bad = 0
    for path in paths:
        with open(path) as f:
            checked, hazards = check(f.read())
        print(f"{path}: {checked} inline-asm instructions checked, {len(hazards)} hazards")
        for h in hazards[:20]:
            print("  " + h)
        bad += len(hazards)
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
