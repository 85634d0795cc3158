"""Build libmamba3_hip.so (the C ABI in include/mamba3_ssm.h) for gfx950.

Every source is compiled with hipcc for --offload-arch=gfx950 only and linked
into mamba3/libmamba3_hip.so inside this package directory (in-tree, so the
library travels with the source tree).  Run directly or via
__graft_entry__.build().  Needs no GPU: hipcc cross-compiles.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "mamba3", "libmamba3_hip.so")

SOURCES = ["m3_api.cpp", "m3_mixer_api.cpp", "linear.cpp", "checkpoint.cpp", "ssd_scan.hip",
           "ssd_scan_fast.hip", "ssd_scan_chunked.hip", "ssd_scan_backward.hip",
           "ssd_scan_backward_generic.hip", "decode_step.hip", "mfma_selftest.hip",
           "mixer_ops.hip", "skinny_gemm.hip"]
ARCH = "gfx950"
# Packed-FP32 instructions stay off: hipcc derives them from plain float code
# and some forms have been unreliable; scalar FP32 is used instead.
HIPFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


def hipcc() -> str:
    return shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    lang = ["-x", "hip"] if src.endswith(".cpp") else []
    cmd = [hipcc()] + HIPFLAGS + lang + ["-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    jobs = min(len(SOURCES), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-o", tmp] + objs + [
        "-L/opt/rocm/lib", "-lhipblaslt", "-Wl,-rpath,/opt/rocm/lib", "-pthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
