#!/usr/bin/env python3
"""Build check over hipcc's kernel resource remarks (-Rpass-analysis=kernel-resource-usage).

Fails (exit 1) when a kernel whose correctness depends on it uses scratch memory or spills
VGPRs: the dequantising GEMM in qmatmul.hip (qgemm_dq_kernel) issues its global loads as
inline asm whose register outputs the compiler treats as ready at once, and waits for them
with fixed vmcnt counts; a spill or a copy of one of those registers between the load and
its wait would read a register still being loaded, and spill traffic would break the
counts. SGPR spills fail it too: a spilled SGPR comes back by v_readlane, a VALU write,
and an asm load reading it fewer than five wait states later (a wait the compiler inserts
only for the loads it emits itself) could read the old value. Scratch use by any other
kernel is printed as a warning (it costs time, not correctness).

Also fails when a kernel declares more than 80 KiB of static LDS (half of gfx950's 160 KiB):
a decode variant whose int4 kernel declared 81 952 bytes gave wrong results, while the
same code at 78 880 bytes was correct. Kernels that need more take it as dynamic LDS,
with the launch attribute set (the prefill kernel).

usage: check_resources.py <remarks file>
"""
import re
import sys


def parse(text):
    kernels = {}
    name = None
    for line in text.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            kernels[name] = {}
            continue
        m = re.search(r"remark:\s+(ScratchSize \[bytes/lane\]|VGPRs Spill|SGPRs Spill|LDS Size \[bytes/block\]): (\d+)",
                      line)
        if m and name:
            kernels[name][m.group(1)] = int(m.group(2))
    return kernels


MAX_STATIC_LDS = 81920


def main():
    path = sys.argv[1]
    kernels = parse(open(path, errors="replace").read())
    strict = ("qgemm_dq_kernel",)
    failed = False
    for k, r in kernels.items():
        if r.get("LDS Size [bytes/block]", 0) > MAX_STATIC_LDS:
            print(f"{path}: error: kernel {k} declares {r['LDS Size [bytes/block]']} bytes of static LDS, more than "
                  f"{MAX_STATIC_LDS}", file=sys.stderr)
            failed = True
        if any(s in k for s in strict) and r.get("SGPRs Spill", 0):
            print(f"{path}: error: kernel {k} spills SGPRs ({r}); its inline-asm loads read SGPRs that a "
                  "spill reload would write just before them", file=sys.stderr)
            failed = True
        if not (r.get("ScratchSize [bytes/lane]", 0) or r.get("VGPRs Spill", 0)):
            continue
        if any(s in k for s in strict):
            print(f"{path}: error: kernel {k} uses scratch ({r}); its inline-asm loads need every "
                  "register to stay in place until its vmcnt wait", file=sys.stderr)
            failed = True
        else:
            print(f"{path}: warning: kernel {k} uses scratch ({r})", file=sys.stderr)
    if failed:
        sys.exit(1)


if __name__ == "__main__":
    main()
