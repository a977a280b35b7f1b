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


def check_no_packed_fp32(src: str) -> None:
    """Compile `src` to device assembly and fail if any packed fp32 VALU op was generated."""
    cmd = [HIPCC, *FLAGS, "--cuda-device-only", "-S", src, "-o", "-"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc -S failed for {src}:\n{res.stderr}")
    if _PACKED_FP32.search(res.stdout):
        raise RuntimeError(f"{src}: packed fp32 VALU instructions in the device code")


def build(verbose: bool = False, check_isa: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(_compile, sources))
        if check_isa:
            list(ex.map(check_no_packed_fp32, sources))
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
