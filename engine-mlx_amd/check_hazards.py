#!/usr/bin/env python3
"""Build check over the device code this build compiled (the gfx950 code object inside each
object file, disassembled with ROCm's llvm-objdump).

The compiler inserts the wait states gfx950 requires between dependent instructions only
around the instructions it emits itself, not around inline asm. Two of them concern the
asm memory instructions of these kernels (the LDS-DMA helpers and the quantised GEMM's
loader):
- an LDS-DMA (buffer_load ... lds) reads M0 no earlier than one wait state after an SALU
  write of M0;
- a memory instruction reads an SGPR (buffer resource, offset, base) no earlier than five
  wait states after a VALU instruction wrote it (v_readfirstlane, v_cmp, or the v_readlane
  that reloads a spilled SGPR).
Wait states are counted back along the instruction stream: one per instruction, N + 1 per
s_nop N, up to the start of the function. Fails (exit 1) on any shorter distance.

usage: check_hazards.py <object.o> ...
"""
import os
import re
import shutil
import subprocess
import sys
import tempfile

LLVM = "/opt/rocm/llvm/bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
SGPR_WAIT = 5
M0_WAIT = 1


def sgprs(tok):
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"s(\d+)", tok)
    return {int(m.group(1))} if m else set()


def parse(text):
    """Functions of an llvm-objdump listing: name -> [(mnemonic, [operands])]."""
    funcs, cur = {}, None
    for line in text.splitlines():
        m = re.match(r"^[0-9a-f]+ <(\S+)>:$", line)
        if m:
            cur = funcs.setdefault(m.group(1), [])
            continue
        if cur is None or not line.startswith(("\t", " ")):
            continue
        ins = line.split("//")[0].strip()
        if not ins:
            continue
        parts = ins.split(None, 1)
        ops = [o.strip() for o in parts[1].split(",")] if len(parts) > 1 else []
        cur.append((parts[0], ops))
    return funcs


def wait_states(instrs, i, hit):
    """Wait states between instruction i and the nearest earlier instruction for which
    hit(mnemonic, operands) holds (None if there is none in the function)."""
    ws = 0
    for k in range(i - 1, -1, -1):
        mn, ops = instrs[k]
        if hit(mn, ops):
            return ws
        ws += int(ops[0], 0) + 1 if mn == "s_nop" else 1
    return None


def check(funcs):
    bad = []
    for name, instrs in funcs.items():
        for i, (mn, ops) in enumerate(instrs):
            if not mn.startswith(("buffer_", "global_", "scratch_", "flat_")):
                continue
            if ops and ops[-1].split()[-1] == "lds" or mn.endswith("_lds") or " lds" in " ".join(ops):
                ws = wait_states(instrs, i, lambda m, o: m.startswith("s_") and o and o[0] == "m0")
                if ws is not None and ws < M0_WAIT:
                    bad.append((name, i, f"{mn} reads m0 {ws} wait states after its write"))
            need = set()
            for o in ops:
                for t in o.split():
                    need |= sgprs(t)
            if not need:
                continue
            ws = wait_states(instrs, i, lambda m, o: m.startswith("v_") and o and bool(sgprs(o[0]) & need))
            if ws is not None and ws < SGPR_WAIT:
                bad.append((name, i, f"{mn} {', '.join(ops)} reads an SGPR {ws} wait states after a VALU write"))
    return bad


def disassemble(obj, tmp):
    fb = os.path.join(tmp, "fatbin")
    co = os.path.join(tmp, "code.co")
    subprocess.run([f"{LLVM}/llvm-objcopy", f"--dump-section=.hip_fatbin={fb}", obj], check=True,
                   capture_output=True)
    subprocess.run([f"{LLVM}/clang-offload-bundler", "--unbundle", "--type=o", f"--input={fb}", f"--targets={TARGET}",
                    f"--output={co}"], check=True, capture_output=True)
    return subprocess.run([f"{LLVM}/llvm-objdump", "-d", "--mcpu=gfx950", co], check=True, capture_output=True,
                          text=True).stdout


def main():
    if not all(shutil.which(f"{LLVM}/{t}") for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump")):
        print("check_hazards: ROCm llvm tools not found; skipped", file=sys.stderr)
        return
    failed = False
    with tempfile.TemporaryDirectory() as tmp:
        for obj in sys.argv[1:]:
            if not obj.endswith(".hip.o"):
                continue
            for name, i, what in check(parse(disassemble(obj, tmp))):
                print(f"{obj}: error: {name} instruction {i}: {what}", file=sys.stderr)
                failed = True
    if failed:
        sys.exit(1)


if __name__ == "__main__":
    main()
