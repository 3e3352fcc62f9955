#!/usr/bin/env python3
"""Build-time check of the device assembly (run by the Makefile).

Some kernels load registers with inline-asm global loads that the compiler
does not track (so that its own vmcnt waits cannot cover buffer->LDS copies
issued after them).  The compiler then treats the destination registers as
ready at once; the code is only correct if nothing reads or writes those
registers before an `s_waitcnt vmcnt(N)` that covers the loads.

From every inline-asm global load, this script follows each path of the
kernel's control flow (both sides of every conditional branch, the targets
of unconditional ones) and fails if any instruction on a path -- arithmetic,
LDS, scalar or vector memory, including the address operands of later loads
-- names a destination register of an asm load still pending on that path.
Loads are pending until a wait `vmcnt(N)` with at least N vector-memory
loads issued after the youngest pending asm load on that path (loads return
in order; stores are not counted, since they may complete earlier).  Waits
without vmcnt (lgkmcnt only) neither clear nor end the scan, and asm loads
met later join the pending set.  An indirect jump (s_setpc) with loads
pending is reported too.

Usage: isa_check_asm_loads.py FILE.s ...
"""
import re
import sys

REG = re.compile(r"v\[(\d+):(\d+)\]|\bv(\d+)\b")
LABEL = re.compile(r"^(\.?[A-Za-z_$][\w.$]*):")
VMEM_LOAD = ("global_load", "buffer_load", "flat_load", "scratch_load")


def regs(text):
    out = set()
    for m in REG.finditer(text):
        if m.group(3) is not None:
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def parse(path):
    """Instructions as (kernel, text, is_asm, line) and a label -> index map."""
    insts, labels = [], {}
    kernel, in_asm = "?", False
    for n, raw in enumerate(open(path).read().split("\n"), 1):
        t = raw.strip()
        if t == ";;#ASMSTART":
            in_asm = True
            continue
        if t == ";;#ASMEND":
            in_asm = False
            continue
        if not t or t.startswith((";", ".cfi", ".loc")):
            continue
        m = LABEL.match(t)
        if m:
            if re.match(r"^_Z\S+:", t):
                kernel = m.group(1)
            labels[m.group(1)] = len(insts)
            continue
        if t.startswith("."):
            continue
        insts.append((kernel, t.split(";")[0].strip(), in_asm, n))
    return insts, labels


def vmcnt(t):
    m = re.search(r"vmcnt\((\d+)\)", t)
    return int(m.group(1)) if m else None


def check(path):
    insts, labels = parse(path)
    bad, groups = [], 0
    for start, (_, t, is_asm, _) in enumerate(insts):
        if not (is_asm and t.startswith("global_load")):
            continue
        # start a scan only at the first asm load of a run (later ones join it)
        if start > 0 and insts[start - 1][2] and insts[start - 1][1].startswith("global_load"):
            continue
        groups += 1
        seen = set()
        stack = [(start, frozenset(), 0)]
        while stack:
            i, pending, after = stack.pop()
            while i < len(insts):
                key = (i, pending, min(after, 64))
                if key in seen:
                    break
                seen.add(key)
                kernel, t, is_asm, line = insts[i]
                op, _, rest = t.partition(" ")
                if is_asm and op.startswith("global_load"):
                    dest, _, addr = rest.partition(",")
                    if regs(addr) & pending:
                        bad.append(f"{kernel}:{line}: {t}")
                    pending = pending | regs(dest)
                    after = 0
                    i += 1
                    continue
                if op == "s_endpgm":
                    break
                if op.startswith("s_waitcnt"):
                    n = vmcnt(t)
                    if n is not None and after >= n:
                        break          # every pending asm load has landed on this path
                    i += 1
                    continue
                if pending and regs(rest) & pending:
                    bad.append(f"{kernel}:{line}: {t}")
                if op.startswith(VMEM_LOAD):
                    after += 1
                if op.startswith(("s_setpc", "s_swappc")):
                    if pending:
                        bad.append(f"{kernel}:{line}: indirect jump with asm loads pending: {t}")
                    break
                if op == "s_branch":
                    tgt = labels.get(rest.strip())
                    if tgt is None:
                        bad.append(f"{kernel}:{line}: unknown branch target: {t}")
                        break
                    i = tgt
                    continue
                if op.startswith("s_cbranch"):
                    tgt = labels.get(rest.strip())
                    if tgt is None:
                        bad.append(f"{kernel}:{line}: unknown branch target: {t}")
                        break
                    stack.append((tgt, pending, after))
                i += 1
    return groups, sorted(set(bad))


def main(paths):
    failures = []
    for p in paths:
        _, bad = check(p)
        failures += [f"{p}: {b}" for b in bad]
    if failures:
        print("registers of inline-asm loads used before their wait:", file=sys.stderr)
        for f in failures:
            print("  " + f, file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
