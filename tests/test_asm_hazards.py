"""CPU tests of the build's wait-state check (engine-mlx_amd/check_hazards.py) over the
disassembled device code: an LDS-DMA must come at least one wait state after the SALU write
of M0 it reads, and a memory instruction at least five after a VALU write of an SGPR it
reads. The compiler keeps both for its own instructions; the check covers the asm ones."""
import glob
import os
import shutil
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "engine-mlx_amd"))
import check_hazards  # noqa: E402

HEAD = "0000000000001000 <_ZN3ema6kernelEv>:\n"


def listing(*lines):
    return HEAD + "".join(f"\t{l}  // 000000001000: 00000000\n" for l in lines)


def problems(*lines):
    return check_hazards.check(check_hazards.parse(listing(*lines)))


def test_dma_right_after_the_m0_write_is_flagged():
    bad = problems("s_mov_b32 m0, s13", "buffer_load_dwordx4 v106, s[72:75], s3 offen nt lds")
    assert len(bad) == 1 and "m0" in bad[0][2]


def test_dma_one_wait_state_after_the_m0_write_passes():
    assert problems("s_mov_b32 m0, s13", "s_nop 0", "buffer_load_dwordx4 v106, s[72:75], s3 offen nt lds") == []


def test_sgpr_read_soon_after_a_valu_write_is_flagged():
    bad = problems("v_readlane_b32 s3, v178, 6", "s_mov_b32 m0, s13", "s_nop 0",
                   "buffer_load_dwordx4 v106, s[72:75], s3 offen nt lds")
    assert len(bad) == 1 and "SGPR" in bad[0][2]
    # the resource of a plain load as well
    assert len(problems("v_readfirstlane_b32 s73, v4", "buffer_load_dwordx4 v[0:3], v1, s[72:75], 0 offen")) == 1


def test_sgpr_read_five_wait_states_after_a_valu_write_passes():
    assert problems("v_readlane_b32 s3, v178, 6", "s_nop 2", "s_mov_b32 m0, s13", "s_nop 0",
                    "buffer_load_dwordx4 v106, s[72:75], s3 offen nt lds") == []
    # an SALU read of the VALU-written SGPR (here the M0 copy) needs no wait
    assert problems("v_readlane_b32 s13, v178, 6", "s_add_i32 s3, s3, s1", "s_mov_b32 m0, s13", "s_nop 0",
                    "buffer_load_dwordx4 v106, s[72:75], s3 offen nt lds") == []


def test_built_objects_keep_the_waits():
    objs = sorted(glob.glob(os.path.join(ROOT, "engine-mlx_amd", "_build", "*.hip.o")))
    if not objs:
        pytest.skip("library not built")
    if not shutil.which(os.path.join(check_hazards.LLVM, "llvm-objdump")):
        pytest.skip("ROCm llvm tools not found")
    import tempfile

    dmas = 0
    with tempfile.TemporaryDirectory() as tmp:
        for obj in objs:
            funcs = check_hazards.parse(check_hazards.disassemble(obj, tmp))
            assert check_hazards.check(funcs) == [], obj
            dmas += sum(1 for ins in funcs.values() for mn, ops in ins if mn.startswith("buffer_") and ops
                        and ops[-1].split()[-1] == "lds")
    assert dmas > 100  # the LDS-DMA helpers of decode, prefill, qmatmul and the WY scan are in the code
