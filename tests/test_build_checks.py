"""Device-code checks that run at build time (no GPU needed: hipcc cross-compiles).

The skinny decoder GEMM stages its activation rows with buffer loads that write
LDS directly; the wait before each k-block's MFMAs is correct only while the
compiler keeps the issue order the source pins. build_lib.check_kblock_waits
re-derives that from the generated assembly; these tests show it passes on the
real kernels and rejects a wait that would let the MFMAs read LDS too early.
"""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "flash-vla_amd"))
import build_lib  # noqa: E402

pytestmark = pytest.mark.skipif(not os.path.exists(build_lib.HIPCC) and not shutil.which("hipcc"),
                                reason="needs hipcc")


@pytest.fixture(scope="module")
def gemm_asm():
    src = os.path.join(build_lib.CSRC, "pi0_gemm.hip")
    res = subprocess.run([build_lib.HIPCC, *build_lib.FLAGS, "--cuda-device-only", "-S", src,
                          "-o", "-"], capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    return res.stdout


def test_kblock_waits_hold(gemm_asm):
    assert "skinny_gemm_kernel" in gemm_asm
    assert build_lib.check_kblock_waits(gemm_asm) == []


# the gate kernel (x rows then weights per k-block), the QKV kernel (all weights first),
# each also with 56 of the 64 rows staged
@pytest.mark.parametrize("name", [
    "_ZN3pi018skinny_gemm_kernelILi4ELb1ELi8ELi4ELin1ELi64EEEvNS_8GemmArgsE",
    "_ZN3pi018skinny_gemm_kernelILi4ELb1ELi8ELi4ELin1ELi56EEEvNS_8GemmArgsE",
    "_ZN3pi018skinny_gemm_kernelILi3ELb0ELi8ELi4ELi4ELi64EEEvNS_8GemmArgsE",
    "_ZN3pi018skinny_gemm_kernelILi3ELb0ELi8ELi4ELi4ELi56EEEvNS_8GemmArgsE"])
def test_kblock_waits_reject_a_loose_wait(gemm_asm, name):
    start = gemm_asm.index(name + ":")
    body = gemm_asm[start:gemm_asm.index("s_endpgm", start)]
    first = body.index("s_waitcnt vmcnt(", body.index(" lds\n"))   # first k-block wait
    loose = body[:first] + "s_waitcnt vmcnt(60)" + body[body.index(")", first) + 1:]
    assert build_lib.check_kblock_waits(gemm_asm.replace(body, loose)) == [name]


def test_no_packed_fp32(gemm_asm):
    assert not build_lib._PACKED_FP32.search(gemm_asm)


def test_no_kernel_uses_scratch():
    """Every kernel runs without a scratch segment: a runtime-indexed kernel argument
    (copied to the stack) or a register spill shows up here before it shows up as a
    slowdown on the GPU."""
    src = os.path.join(build_lib.CSRC, "pi0_attention.hip")
    res = subprocess.run([build_lib.HIPCC, *build_lib.FLAGS, "--cuda-device-only", "-S", src,
                          "-o", "-"], capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    assert "attn_kernel" in res.stdout
    assert build_lib.scratch_kernels(res.stdout) == []
    fake = ("\t.amdhsa_kernel k_spills\n\t\t.amdhsa_private_segment_fixed_size 192\n"
            "\t.end_amdhsa_kernel\n\t.amdhsa_kernel k_clean\n"
            "\t\t.amdhsa_private_segment_fixed_size 0\n\t.end_amdhsa_kernel\n")
    assert build_lib.scratch_kernels(fake) == ["k_spills"]
