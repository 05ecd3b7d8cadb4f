"""Build libvolta_mi355x_backend.so (HIP for gfx950) in-tree.

Usage: python volta-zk_amd/build.py [--jobs N]

Every HIP source is compiled with hipcc for gfx950 only, with packed-FP32
instruction selection disabled, and linked into one shared library next to
this file.  No CUDA, no hipify, no multi-target build.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "libvolta_mi355x_backend.so"
# Host build of the device arithmetic headers for the CPU tests (not shipped).
CHECK_LIB = HERE / "libgl64_check.so"
SOURCES = ["context.cpp", "ntt.hip", "ntt_reg.hip", "encode_fast.hip", "ntt15.hip", "ntt_rr.hip", "pcs.hip", "merkle.hip", "x4.hip", "abi_pcs.cpp",
           "abi_stubs.cpp"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CFLAGS = [
    "-x", "hip", "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-fvisibility=hidden", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", str(CSRC), "-I", str(HERE.parent / "include"),
]


def _compile(src: str) -> pathlib.Path:
    obj = BUILD / (src + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed for {src}")
    return obj


def build(jobs: int | None = None) -> pathlib.Path:
    if shutil.which(HIPCC) is None and not pathlib.Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD.mkdir(exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("link failed")
    os.replace(tmp, LIB)
    # host-only compile of the same headers: no device code in this library
    cmd = [HIPCC, "-x", "hip", "--cuda-host-only", "-O2", "-std=c++17", "-fPIC", "-shared",
           "-I", str(CSRC), str(CSRC / "host_check.cpp"), "-o", str(CHECK_LIB)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("host check library failed to build")
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    a = ap.parse_args()
    print(build(a.jobs))
