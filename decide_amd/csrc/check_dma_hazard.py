#!/usr/bin/env python3
"""Build check: the global → LDS DMAs written as inline asm must not read an
SGPR that a VALU instruction wrote fewer than 5 wait states earlier.

GFX9 parts (gfx950 among them) need 5 wait states between a VALU write of an
SGPR (v_readfirstlane_b32, v_readlane_b32, a VOPC or carry-out destination)
and a VMEM instruction that reads that SGPR as its address base. The compiler
pads the distance for loads it generates itself, but a load inside an asm
string is invisible to it. This script walks back from every
`global_load_lds_dwordx4 ..., s[a:b]` in the generated assembly and fails if a
VALU write of s[a] or s[b] lies within 5 wait states on any path into the
DMA: at a block boundary the walk continues into every predecessor block (the
fall-through block and every block that branches to the label).

Usage: check_dma_hazard.py FILE.s [FILE.s ...]   (exit status 1 on a finding)
"""

import re
import sys

NEED = 5
DMA = re.compile(r"^\s*global_load_lds_dword\w*\s+v\d+,\s*s\[(\d+):(\d+)\]")
LABEL = re.compile(r"^[.\w$]+:")
FUNC = re.compile(r"^([_A-Za-z][\w$.]*):")
# VALU instructions whose destination (first operand) or carry-out is an SGPR
VALU_SDST = re.compile(r"^\s*(v_\w+)\s+(s\[\d+:\d+\]|s\d+|vcc\w*)")
VALU_CARRY = re.compile(r"^\s*(v_\w+_co\w*|v_div_scale\w*)\s+v[\[\d][^,]*,\s*(s\[\d+:\d+\]|s\d+)")


def sregs(tok):
    m = re.match(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"s(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def valu_writes(line):
    out = set()
    m = VALU_SDST.match(line)
    if m:
        out |= sregs(m.group(2))
    m = VALU_CARRY.match(line)
    if m:
        out |= sregs(m.group(2))
    return out


def wait_states(line):
    m = re.match(r"^\s*s_nop\s+(\d+)", line)
    return int(m.group(1)) + 1 if m else 1


def instructions(path):
    """(function, [lines]) with comments, directives and blank lines removed."""
    funcs, name, body = [], None, []
    for raw in open(path):
        line = raw.split(";")[0].rstrip()
        if not line.strip():
            continue
        s = line.strip()
        if s.startswith(".") and not LABEL.match(s):
            continue
        fm = FUNC.match(line)
        if fm and not line.startswith("."):
            if name is not None:
                funcs.append((name, body))
            name, body = fm.group(1), []
            continue
        if name is not None:
            body.append(line)
    if name is not None:
        funcs.append((name, body))
    return funcs


BRANCH = re.compile(r"^\s*s_(c?branch\w*)\s+([.\w$]+)")
ENDS = re.compile(r"^\s*(s_branch|s_endpgm|s_setpc_b64)\b")


def blocks(body):
    """Split a function body into basic blocks: [(label, [lines])]; predecessor map."""
    blks, label, cur = [], None, []
    for line in body:
        if LABEL.match(line.strip()):
            blks.append((label, cur))
            label, cur = line.strip()[:-1], []
        else:
            cur.append(line)
    blks.append((label, cur))
    index = {lab: k for k, (lab, _) in enumerate(blks) if lab}
    preds = {k: set() for k in range(len(blks))}
    for k, (_, lines) in enumerate(blks):
        for line in lines:
            m = BRANCH.match(line)
            if m and m.group(2) in index:
                preds[index[m.group(2)]].add(k)
        if k + 1 < len(blks) and not (lines and ENDS.match(lines[-1])):
            preds[k + 1].add(k)
    return blks, preds


def hazard(blks, preds, k, end, regs, ws, seen):
    """A VALU write of `regs` within NEED - ws wait states before line `end` of block k?"""
    lines = blks[k][1]
    for j in range(end - 1, -1, -1):
        if ws >= NEED:
            return None
        if regs & valu_writes(lines[j]):
            return "VALU write %d wait states earlier: %s" % (ws, lines[j].strip())
        ws += wait_states(lines[j])
    if ws >= NEED:
        return None
    for q in preds[k]:
        if (q, ws) in seen:
            continue
        seen.add((q, ws))
        why = hazard(blks, preds, q, len(blks[q][1]), regs, ws, seen)
        if why:
            return why + " (in a predecessor block)"
    return None


def check(path):
    bad = seen_dma = 0
    for name, body in instructions(path):
        blks, preds = blocks(body)
        for k, (_, lines) in enumerate(blks):
            for i, line in enumerate(lines):
                m = DMA.match(line)
                if not m:
                    continue
                seen_dma += 1
                regs = set(range(int(m.group(1)), int(m.group(2)) + 1))
                why = hazard(blks, preds, k, i, regs, 0, set())
                if why:
                    print("%s: %s: %s\n    %s" % (path, name, why, line.strip()))
                    bad += 1
    print("%s: %d DMA instruction(s) checked" % (path, seen_dma))
    return bad


def main(argv):
    bad = sum(check(p) for p in argv[1:])
    if bad:
        print("%d DMA(s) may read an SGPR still being written by a VALU instruction" % bad)
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
