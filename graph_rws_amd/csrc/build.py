"""Builds graph_rws_amd/libgrws.so with hipcc for gfx950 (in-tree).

    python -m graph_rws_amd.csrc.build        # or: python graph_rws_amd/csrc/build.py

Every translation unit is compiled with
  --offload-arch=gfx950 -O3 -fPIC -std=c++17
  -Xclang -target-feature -Xclang -packed-fp32-ops -mllvm -amdgpu-mfma-vgpr-form
(the feature pair keeps the compiler from emitting packed fp32 VALU ops; the
last option keeps MFMA accumulators in ordinary VGPRs, which avoids copies
between accumulator registers in the pipelined loops), then
linked into one shared library that exports the C ABI of include/grws.h.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
OUT = os.path.join(PKG, "libgrws.so")
OBJ_DIR = os.path.join(HERE, "_build")

SOURCES = [
    "abi.cpp",
    "scan.hip",
    "sort.hip",
    "spmm.hip",
    "group.hip",
    "bcsr_build.hip",
    "reindex.hip",
    "sample.hip",
    "window_sample.hip",
    "gemm_tn.hip",
    "repack.hip",
    "fused.hip",
    "probe.hip",
]

ARCH = os.environ.get("GRWS_OFFLOAD_ARCH", "gfx950")


def _hipcc() -> str:
    p = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(p):
        raise RuntimeError("hipcc not found")
    return p


def _flags():
    return [f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall",
            "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-result",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-mllvm", "-amdgpu-mfma-vgpr-form",
            f"-I{os.path.join(ROOT, 'include')}"]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    cmd = [_hipcc()] + _flags() + ["-c", os.path.join(HERE, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> str:
    """Compiles every source and links libgrws.so; returns its path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4, 16)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = OUT + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs + ["-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(OUT)
    return OUT


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
