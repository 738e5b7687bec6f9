#!/usr/bin/env python3
"""Lint for the kernels that issue global loads from inline asm with hand-counted waits.

hipcc treats an inline-asm output as defined at the asm statement.  Under register pressure it
may then copy, spill or reuse the destination of a load that is still in flight, and the late
load overwrites whatever the register holds by then (an address, for instance).  This script
compiles each HIP source for gfx950 to assembly and, inside every basic block, tracks the VGPRs
written by global / buffer loads until an `s_waitcnt vmcnt(N)` retires them (N or more
vector-memory operations issued after the load; stores and atomics count too, as on every gfx9
chip).  Any other instruction that reads or writes such a register is reported.  A load whose
destination overlaps an older in-flight load is not reported: loads return in order.

The check is per block (a block starts with nothing outstanding), so it finds the straight-line
hazards a spill or copy creates; waits and loads that span blocks are the kernel's own protocol.

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


def check_block(block, report):
    pending = {}  # vgpr -> vector-memory operations issued after its load
    for ln, text in block:
        parts = text.replace(",", " ").split()
        op = parts[0]
        m = re.match(r"s_waitcnt\b.*vmcnt\((\d+)\)", text)
        if m:
            n = int(m.group(1))
            pending = {r: k for r, k in pending.items() if k < n}
            continue
        if op.startswith("s_"):
            continue
        operands = parts[1:]
        is_vm = op.startswith(VM_PREFIXES)
        is_load = is_vm and "_load" in op and "_lds" not in op  # direct-to-LDS: no VGPR result
        returns = is_load or (is_vm and "atomic" in op and " glc" in text)
        dst = list(vgprs(operands[0])) if operands and (returns or not is_vm) else []
        srcs = sorted({r for t in (operands[1:] if dst else operands) for r in vgprs(t)})
        for r in srcs:
            if r in pending:
                report.append((ln, text, "reads v%d before its load has landed" % r))
        if not is_load:
            for r in dst:
                if r in pending:
                    report.append((ln, text, "overwrites v%d while a load into it is in flight" % r))
        if is_vm:
            pending = {r: k + 1 for r, k in pending.items()}
            if returns:
                for r in dst:
                    pending[r] = 0


def check_asm(path):
    lines = open(path).read().split("\n")
    found = []
    kernel, block = None, []
    for ln, raw in enumerate(lines, 1):
        text = raw.split(";")[0].strip()
        m = re.match(r"^(_Z\w+):", raw)
        if m or text.endswith(":") or raw.startswith(".Lfunc_end"):
            if block:
                rep = []
                check_block(block, rep)
                found += [(kernel, *r) for r in rep]
            block = []
            if m:
                kernel = m.group(1)
            continue
        if not text or text.startswith("."):
            continue
        block.append((ln, text))
        if is_block_end(text.split()[0]):
            rep = []
            check_block(block, rep)
            found += [(kernel, *r) for r in rep]
            block = []
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
