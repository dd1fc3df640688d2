"""Ahead-of-time build of the gfx950 libraries (hipcc, in-tree).

Outputs (git-ignored, shipped to the GPU box with the tree):
  lc_parallel_primitive_amd/liblcpp_amd.so      the primitives behind include/lcpp_amd.h
  lc_parallel_primitive_amd/liblcpp_datagen.so  synthetic-input generators (bench/tests)
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "liblcpp_amd.so")
DATAGEN_LIB = os.path.join(PKG, "liblcpp_datagen.so")

LIB_SOURCES = ["runtime.hip", "reduce.hip", "scan.hip", "radix_sort.hip", "segment_reduce.hip",
               "scan_by_key.hip", "reduce_by_key.hip"]
DATAGEN_SOURCES = ["datagen.hip"]

ARCH = os.environ.get("LCPP_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
CXXFLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # packed-FP32 VALU forms are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *CXXFLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def _link(objs: list[str], out: str) -> None:
    tmp = out + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed for {out}:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)


def build(verbose: bool = False) -> None:
    os.makedirs(BUILD, exist_ok=True)
    sources = LIB_SOURCES + DATAGEN_SOURCES
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = dict(zip(sources, ex.map(_compile, sources)))
    _link([objs[s] for s in LIB_SOURCES], LIB)
    _link([objs[s] for s in DATAGEN_SOURCES], DATAGEN_LIB)
    if verbose:
        print(f"built {LIB} and {DATAGEN_LIB} for {ARCH}")


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
