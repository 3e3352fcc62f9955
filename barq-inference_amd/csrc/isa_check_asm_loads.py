#!/usr/bin/env python3
"""Build-time check of the device assembly (run by the Makefile).

Some kernels load registers with inline-asm global loads that the compiler
does not track (so that its own vmcnt waits cannot cover buffer->LDS copies
issued after them).  The compiler then treats the destination registers as
ready at once; the code is only correct if nothing reads or writes those
registers before the kernel's own `s_waitcnt vmcnt` that follows the loads.
This script scans every run of inline-asm global loads in the given `.s`
files and fails if any instruction before the next `s_waitcnt vmcnt` (in
program order) names one of their destination registers.

Usage: isa_check_asm_loads.py FILE.s ...
"""
import re
import sys

REG = re.compile(r"v\[(\d+):(\d+)\]|\bv(\d+)\b")


def regs(text):
    out = set()
    for m in REG.finditer(text):
        if m.group(3) is not None:
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def check(path):
    lines = open(path).read().split("\n")
    kernel, groups, bad = "?", 0, []
    i = 0
    while i < len(lines):
        line = lines[i]
        if re.match(r"^_Z\S+:", line):
            kernel = line.split(":")[0]
        if line.strip() == ";;#ASMSTART" and i + 1 < len(lines) and lines[i + 1].strip().startswith("global_load"):
            groups += 1
            dests, j = set(), i
            # the run of asm global loads, up to the first copy or wait
            while j < len(lines):
                t = lines[j].strip()
                if t.startswith("buffer_load") or t.startswith("s_waitcnt"):
                    break
                if t.startswith("global_load"):
                    dests |= regs(t.split(None, 1)[1].split(",")[0])
                j += 1
            # every instruction before the next vmcnt wait
            while j < len(lines):
                t = lines[j].strip()
                if t.startswith("s_waitcnt") and "vmcnt" in t or t.startswith("s_endpgm"):
                    break
                if t and not t.startswith((";", ".")) and not t.startswith(("global_load", "buffer_load")):
                    parts = t.split(None, 1)
                    if len(parts) > 1 and regs(parts[1]) & dests:
                        bad.append(f"{kernel}: {t}")
                j += 1
            i = j
        i += 1
    return groups, bad


def main(paths):
    total, failures = 0, []
    for p in paths:
        n, bad = check(p)
        total += n
        failures += [f"{p}: {b}" for b in bad]
    if failures:
        print("registers of inline-asm loads used before their wait:", file=sys.stderr)
        for f in failures:
            print("  " + f, file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
