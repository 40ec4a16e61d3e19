"""Register-safety check of the inline-asm LDS reads of the ordered chains
(CHAIN_READ8 / CHAIN_WAIT in needle_cs_amd/csrc/common.hpp).

Each CHAIN_READ8 issues eight ds_read_b128 whose destination registers are
written by the hardware later; the compiler believes them written at the asm
statement.  The code is correct only if no compiler-generated instruction
reads or writes those registers before the s_waitcnt that covers the batch.
This walks the gfx950 assembly of a kernel file along every branch from each
read batch and reports any such instruction:
  * the batch at offset 0 (read before the loop) is covered by the first
    s_waitcnt asm met on every path (the loop reads the next batch before
    waiting for this one, so lgkmcnt(8) then means this batch has landed);
  * the batches read inside the loop are covered by the second one.
"""
from __future__ import annotations

import re


def _regs(tok: str) -> set[int]:
    m = re.match(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def _insn_regs(line: str) -> set[int]:
    out: set[int] = set()
    for tok in re.split(r"[\s,]+", line.strip()):
        out |= _regs(tok)
    return out


def check(asm_text: str) -> tuple[int, list[str]]:
    """Returns (read batches found, violations as messages)."""
    lines = asm_text.split("\n")
    in_asm, flag = [], False
    for line in lines:
        if ";;#ASMSTART" in line:
            flag = True
        in_asm.append(flag)
        if ";;#ASMEND" in line:
            flag = False
    labels = {}
    for k, line in enumerate(lines):
        m = re.match(r"^(\.LBB\d+_\d+):", line)
        if m:
            labels[m.group(1)] = k
    problems: list[str] = []

    def walk(start: int, dest: set[int], need: int, waits: int, seen: set, origin: int) -> None:
        k = start
        while k < len(lines):
            if (k, waits) in seen:
                return
            seen.add((k, waits))
            t = lines[k].strip()
            if in_asm[k] and "s_waitcnt lgkmcnt" in t:
                waits += 1
                if waits >= need:
                    return
            elif not in_asm[k] and t and not t.startswith((".", ";")):
                hit = _insn_regs(t) & dest
                if hit:
                    problems.append(f"line {k + 1}: '{t}' touches v{sorted(hit)} before the wait of the reads "
                                    f"at line {origin + 1}")
                if t.startswith("s_endpgm"):
                    return
                m = re.match(r"s_branch (\.LBB\d+_\d+)", t)
                if m:
                    k = labels[m.group(1)]
                    continue
                m = re.match(r"s_cbranch_\w+ (\.LBB\d+_\d+)", t)
                if m:
                    walk(labels[m.group(1)], dest, need, waits, seen, origin)
            k += 1

    batches = 0
    k = 0
    while k < len(lines):
        line = lines[k]
        if in_asm[k] and "ds_read_b128" in line and re.search(r"offset:(\d+)\s*$", line):
            off = int(re.search(r"offset:(\d+)", line).group(1))
            dest: set[int] = set()
            j = k
            while "ds_read_b128" in lines[j]:
                dest |= _regs(lines[j].split()[1].rstrip(","))
                j += 1
            walk(j, dest, 1 if off == 0 else 2, 0, set(), k)
            batches += 1
            k = j
        else:
            k += 1
    return batches, problems
