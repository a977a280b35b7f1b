"""Build libpi0hip.so (gfx950) from csrc/*.hip with hipcc, in-tree.

Usage: python flash-vla_amd/build_lib.py   (or __graft_entry__.build())
Objects go to flash-vla_amd/_build/, the library to flash_vla_amd/lib/.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "flash_vla_amd", "lib")
LIB = os.path.join(LIBDIR, "libpi0hip.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", f"-I{INCLUDE}",
    # packed fp32 VALU ops are kept out of generated code on this hardware
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src).replace(".hip", ".o"))
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


# packed fp32 VALU forms must not appear in the device code (see FLAGS)
_PACKED_FP32 = re.compile(r"\bv_pk_(add|mul|fma)_f32\b")


def check_kblock_waits(asm: str) -> list[str]:
    """Names of skinny GEMM kernels whose k-block waits do not cover their LDS copies.

    skinny_gemm_kernel issues, per k-block, buffer loads that write x straight into
    LDS and that k-block's weight loads (x first, or the weights some k-blocks ahead:
    one k-block's copies are contiguous, the k-blocks' copies go out in order, and the
    loop waits once per k-block); before the MFMAs of k-block j it waits with vmcnt(N). Vector-memory operations complete in issue order, so the wait is
    sufficient only if N is at most the number of operations issued after k-block j's
    last LDS copy. This re-checks that order in the generated code (the scheduling
    barriers in the source are what keep it).
    """
    bad = []
    for m in re.finditer(r"^(_ZN3pi018skinny_gemm_kernelI\w+):", asm, re.M):
        body = asm[m.end():asm.index("s_endpgm", m.end())]
        lines = [ln.strip() for ln in body.split("\n")]
        first_ds = next(i for i, ln in enumerate(lines) if ln.startswith("ds_read"))
        issue = [i for i, ln in enumerate(lines[:first_ds])
                 if ln.startswith(("global_load", "buffer_load"))]
        kinds = ["lds" if lines[i].endswith(" lds") else "reg" for i in issue]
        waits = [int(w) for w in re.findall(r"s_waitcnt vmcnt\((\d+)\)",
                                            "\n".join(lines[issue[-1] + 1:]))]
        tail = lines[issue[-1] + 1:]
        loop = "\n".join(tail[:next((i for i, ln in enumerate(tail) if ln.startswith("s_barrier")),
                                     len(tail))])
        nkb = len(re.findall(r"s_waitcnt vmcnt\(\d+\)", loop))
        copies = [j for j, k in enumerate(kinds) if k == "lds"]
        per = len(copies) // nkb if nkb and len(copies) % nkb == 0 else 0
        last_copy = copies[per - 1::per] if per else []
        ok = bool(last_copy) and len(waits) >= len(last_copy) and all(
            waits[j] <= len(kinds) - 1 - c for j, c in enumerate(last_copy))
        if not ok:
            bad.append(m.group(1))
    return bad


def scratch_kernels(asm: str) -> list[str]:
    """Kernels whose private (scratch) segment is not empty: a spill, or a kernel argument
    indexed at run time and so copied to the stack -- both silent slowdowns."""
    bad = []
    for m in re.finditer(r"^\s*\.amdhsa_kernel\s+(\S+)(.*?)^\s*\.end_amdhsa_kernel", asm, re.M | re.S):
        size = re.search(r"\.amdhsa_private_segment_fixed_size\s+(\d+)", m.group(2))
        if size and int(size.group(1)) > 0:
            bad.append(m.group(1))
    return bad


def check_device_code(src: str) -> None:
    """Compile `src` to device assembly and fail if any packed fp32 VALU op was
    generated, if any kernel uses scratch memory, or (pi0_gemm.hip) if a skinny GEMM's
    k-block waits are unsafe."""
    cmd = [HIPCC, *FLAGS, "--cuda-device-only", "-S", src, "-o", "-"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc -S failed for {src}:\n{res.stderr}")
    if _PACKED_FP32.search(res.stdout):
        raise RuntimeError(f"{src}: packed fp32 VALU instructions in the device code")
    scratch = scratch_kernels(res.stdout)
    if scratch:
        raise RuntimeError(f"{src}: kernels with a scratch segment: {scratch}")
    if os.path.basename(src) == "pi0_gemm.hip":
        bad = check_kblock_waits(res.stdout)
        if bad:
            raise RuntimeError(f"{src}: k-block vmcnt waits do not cover the LDS copies in {bad}")


def build(verbose: bool = False, check_isa: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(_compile, sources))
        if check_isa:
            list(ex.map(check_device_code, sources))
    tmp = LIB + ".tmp"
    # --no-undefined: a kernel whose host stub was not emitted fails here, not at load time
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", *objs,
           "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
