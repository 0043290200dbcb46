"""CPU tests of the build's resource check (engine-mlx_amd/check_resources.py): hipcc's
kernel resource remarks must show no scratch and no VGPR or SGPR spills for the dequantising GEMM,
whose inline-asm loads need their registers left in place until their vmcnt waits."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECK = os.path.join(ROOT, "engine-mlx_amd", "check_resources.py")

REMARKS = """\
csrc/qmatmul.hip:812:1: remark: Function Name: _ZN3ema12_GLOBAL__N_115qgemm_dq_kernelILi4ELi64ELb1EEEvNS0_7QmmArgsENS0_6DqPlanE [-Rpass-analysis=kernel-resource-usage]
csrc/qmatmul.hip:812:1: remark:     VGPRs: 97 [-Rpass-analysis=kernel-resource-usage]
csrc/qmatmul.hip:812:1: remark:     ScratchSize [bytes/lane]: {scratch} [-Rpass-analysis=kernel-resource-usage]
csrc/qmatmul.hip:812:1: remark:     VGPRs Spill: {spill} [-Rpass-analysis=kernel-resource-usage]
csrc/qmatmul.hip:812:1: remark:     SGPRs Spill: {sspill} [-Rpass-analysis=kernel-resource-usage]
csrc/qmatmul.hip:187:1: remark: Function Name: _ZN3ema12_GLOBAL__N_110qmm_kernelILi4ELi64ELb1ELi1EEEvNS0_7QmmArgsE [-Rpass-analysis=kernel-resource-usage]
csrc/qmatmul.hip:187:1: remark:     ScratchSize [bytes/lane]: {other} [-Rpass-analysis=kernel-resource-usage]
csrc/qmatmul.hip:187:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
csrc/qmatmul.hip:187:1: remark:     SGPRs Spill: {osspill} [-Rpass-analysis=kernel-resource-usage]
"""


def run_check(tmp_path, sspill=0, osspill=0, **kw):
    kw.update(sspill=sspill, osspill=osspill)
    p = tmp_path / "x.res"
    p.write_text(REMARKS.format(**kw))
    return subprocess.run([sys.executable, CHECK, str(p)], capture_output=True, text=True)


def test_clean_remarks_pass(tmp_path):
    r = run_check(tmp_path, scratch=0, spill=0, other=0)
    assert r.returncode == 0 and r.stderr == ""


def test_spilling_dequantising_gemm_fails_the_build(tmp_path):
    r = run_check(tmp_path, scratch=16, spill=0, other=0)
    assert r.returncode == 1 and "qgemm_dq_kernel" in r.stderr and "error" in r.stderr
    r = run_check(tmp_path, scratch=0, spill=3, other=0)
    assert r.returncode == 1


def test_sgpr_spills_of_the_dequantising_gemm_fail_the_build(tmp_path):
    """A spilled SGPR returns by v_readlane (a VALU write); an asm load reading it within five
    wait states gets no wait from the compiler."""
    r = run_check(tmp_path, scratch=0, spill=0, other=0, sspill=2)
    assert r.returncode == 1 and "spills SGPRs" in r.stderr
    r = run_check(tmp_path, scratch=0, spill=0, other=0, osspill=5)
    assert r.returncode == 0


def test_other_kernels_only_warn(tmp_path):
    r = run_check(tmp_path, scratch=0, spill=0, other=64)
    assert r.returncode == 0 and "warning" in r.stderr and "qmm_kernel" in r.stderr


def test_built_library_remarks():
    """The remarks of the last build (written next to the objects) hold the dequantising
    GEMM's instantiations, all without scratch."""
    res = os.path.join(ROOT, "engine-mlx_amd", "_build", "qmatmul.hip.res")
    if not os.path.exists(res):
        import pytest

        pytest.skip("library not built")
    sys.path.insert(0, os.path.dirname(CHECK))
    import check_resources

    ks = {k: v for k, v in check_resources.parse(open(res).read()).items() if "qgemm_dq_kernel" in k}
    assert len(ks) >= 6
    for k, v in ks.items():
        assert v["ScratchSize [bytes/lane]"] == 0 and v["VGPRs Spill"] == 0 and v["SGPRs Spill"] == 0, k
