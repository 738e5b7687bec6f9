#!/usr/bin/env python3
"""Lint for the kernels that issue global loads from inline asm with hand-counted waits.

hipcc treats an inline-asm output as defined at the asm statement.  Under register pressure it
may then copy, spill or reuse the destination of a load that is still in flight, and the late
load overwrites whatever the register holds by then (an address, for instance).  This script
compiles each HIP source for gfx950 to assembly and tracks the VGPRs written by global / buffer
loads until an `s_waitcnt vmcnt(N)` retires them (N or more vector-memory operations issued
after the load; stores and atomics count too, as on every gfx9 chip).  Any other instruction
that reads or writes such a register is reported.  A load whose destination overlaps an older
in-flight load is not reported: loads return in order.

The tracking follows the control flow of each function: basic blocks (labels, branches,
fall-through) form a graph, and the in-flight state at a block's entry is the merge of its
predecessors' exit states, iterated to a fixed point.  A register is in flight at a merge if it
is in flight on any incoming edge, with the fewest newer operations of those edges.  So load
rings carried around a loop's back edge are checked too: a copy or spill at the loop latch of a
register whose load is still in flight is reported, as is a use in the next iteration before
the wait that covers it.

Usage: python3 vmcnt_check.py [file.hip ...]   (default: every *.hip beside this script)
Exit status 1 when a hazard is found.
"""
import glob
import os
import re
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "-x", "hip", "--cuda-device-only", "-S"]
VM_PREFIXES = ("global_", "buffer_", "scratch_", "flat_")


def vgprs(tok):
    m = re.match(r"v\[(\d+):(\d+)\]$", tok)
    if m:
        return range(int(m.group(1)), int(m.group(2)) + 1)
    m = re.match(r"v(\d+)$", tok)
    return [int(m.group(1))] if m else []


def is_block_end(op):
    return op.startswith("s_branch") or op.startswith("s_cbranch") or op in ("s_endpgm", "s_setpc_b64")


VMCNT_MAX = 64  # counts saturate: vmcnt is 6 bits on gfx9


def step(state, text, report=None, ln=0):
    """Apply one instruction to the in-flight state {vgpr: newer vm ops}; return the new state."""
    parts = text.replace(",", " ").split()
    op = parts[0]
    m = re.match(r"s_waitcnt\b.*vmcnt\((\d+)\)", text)
    if m:
        n = int(m.group(1))
        return {r: k for r, k in state.items() if k < n}
    if op.startswith("s_"):
        return state
    operands = parts[1:]
    is_vm = op.startswith(VM_PREFIXES)
    # direct-to-LDS loads (global_load_lds_*, buffer_load_* ... lds) have no VGPR result
    is_load = is_vm and "_load" in op and "_lds" not in op and "lds" not in operands
    returns = is_load or (is_vm and "atomic" in op and " glc" in text)
    dst = list(vgprs(operands[0])) if operands and (returns or not is_vm) else []
    srcs = sorted({r for t in (operands[1:] if dst else operands) for r in vgprs(t)})
    if report is not None:
        for r in srcs:
            if r in state:
                report.append((ln, text, "reads v%d before its load has landed" % r))
        if not is_load:
            for r in dst:
                if r in state:
                    report.append((ln, text, "overwrites v%d while a load into it is in flight" % r))
    if not is_vm:
        return state
    new = {r: min(k + 1, VMCNT_MAX) for r, k in state.items()}
    if returns:
        for r in dst:
            new[r] = 0
    return new


def merge(a, b):
    out = dict(a)
    for r, k in b.items():
        out[r] = min(out.get(r, k), k)
    return out


def split_blocks(body):
    """body: [(ln, text)] of one function -> (blocks [(label, [(ln, text)])], successors)."""
    blocks, cur, label = [], [], None
    for ln, text in body:
        if text.endswith(":"):
            if cur or label is not None:
                blocks.append((label, cur))
            label, cur = text[:-1], []
            continue
        cur.append((ln, text))
        op = text.split()[0]
        if op.startswith("s_branch") or op.startswith("s_cbranch") or op in ("s_endpgm", "s_setpc_b64"):
            blocks.append((label, cur))
            label, cur = None, []
    if cur or label is not None:
        blocks.append((label, cur))
    index = {lab: i for i, (lab, _) in enumerate(blocks) if lab is not None}
    succ = []
    for i, (_, ins) in enumerate(blocks):
        s = []
        last = ins[-1][1] if ins else ""
        op = last.split()[0] if last else ""
        if op.startswith("s_branch") or op.startswith("s_cbranch"):
            tgt = last.split()[-1]
            if tgt in index:
                s.append(index[tgt])
        if not (op.startswith("s_branch") or op in ("s_endpgm", "s_setpc_b64")) and i + 1 < len(blocks):
            s.append(i + 1)
        succ.append(s)
    return blocks, succ


def check_function(body, report):
    blocks, succ = split_blocks(body)
    if not blocks:
        return
    entry = [None] * len(blocks)
    entry[0] = {}
    work = [0]
    while work:
        i = work.pop()
        st = entry[i]
        for _, text in blocks[i][1]:
            st = step(st, text)
        for j in succ[i]:
            m = st if entry[j] is None else merge(entry[j], st)
            if m != entry[j]:
                entry[j] = m
                work.append(j)
    for i, (_, ins) in enumerate(blocks):
        if entry[i] is None:
            continue
        st = entry[i]
        for ln, text in ins:
            st = step(st, text, report, ln)


def check_asm(path):
    lines = open(path).read().split("\n")
    found = []
    kernel, body = None, []

    def flush():
        rep = []
        check_function(body, rep)
        found.extend((kernel, *r) for r in rep)

    for ln, raw in enumerate(lines, 1):
        text = raw.split(";")[0].strip()
        m = re.match(r"^(_Z\w+|\w+):", raw)
        if (m and not raw.startswith(".")) or raw.startswith(".Lfunc_end"):
            if body:
                flush()
            body = []
            kernel = m.group(1) if m and not raw.startswith(".") else None
            continue
        if kernel is None or not text:
            continue
        if text.startswith(".") and not text.endswith(":"):
            continue
        body.append((ln, text))
    if body:
        flush()
    return found


def main(argv):
    srcs = argv[1:] or sorted(glob.glob(os.path.join(HERE, "*.hip")))
    bad = 0
    with tempfile.TemporaryDirectory() as tmp:
        for src in srcs:
            asm = os.path.join(tmp, os.path.basename(src) + ".s")
            subprocess.run([HIPCC, *FLAGS, "-I", HERE, src, "-o", asm], check=True, stderr=subprocess.DEVNULL)
            hits = check_asm(asm)
            kernels = sorted({k for k, *_ in hits})
            for k in kernels:
                mine = [h for h in hits if h[0] == k]
                print("%s: %s: %d hazard(s), first: line %d: %s (%s)" % (
                    os.path.basename(src), k, len(mine), mine[0][1], mine[0][2], mine[0][3]))
            bad += len(hits)
            print("%s: %s" % (os.path.basename(src), "ok" if not hits else "HAZARDS"))
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
