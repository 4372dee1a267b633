"""Resource checks on the built library's gfx950 code objects (CPU only: the
kernels' metadata is read from libgrws.so, nothing runs on a GPU).

The slab-pair SpMM kernels stage X through LDS by direct loads and keep 80
accumulator registers per lane; a build of the 320-column kernel that spilled
registers to scratch summed wrongly (run-dependent results), the spill-free
build is bit-identical to the register-staged kernel.  So the grouped-tile
kernels must use no scratch memory at all, and must fit the register budget
that keeps three waves per SIMD (168 VGPRs, 512 per SIMD lane)."""
import os
import re
import shutil
import struct
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "graph_rws_amd", "libgrws.so")
LLVM = "/opt/rocm/llvm/bin"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _tool(name):
    p = os.path.join(LLVM, name)
    return p if os.path.exists(p) else shutil.which(name)


def _code_objects(fatbin: bytes):
    """The gfx950 code objects of a .hip_fatbin section: one clang offload
    bundle per source file, each {magic, entry count, entries of (offset,
    size, triple length, triple)}, offsets relative to the bundle."""
    out = []
    pos = fatbin.find(MAGIC)
    while pos >= 0:
        p = pos + len(MAGIC)
        (n,) = struct.unpack_from("<Q", fatbin, p)
        p += 8
        for _ in range(n):
            off, size, tlen = struct.unpack_from("<QQQ", fatbin, p)
            p += 24
            triple = fatbin[p:p + tlen].decode()
            p += tlen
            if "gfx950" in triple and size:
                out.append(fatbin[pos + off:pos + off + size])
        pos = fatbin.find(MAGIC, pos + len(MAGIC))
    return out


def _kernel_metadata(tmp_path):
    objcopy, readelf = _tool("llvm-objcopy"), _tool("llvm-readelf")
    if not (objcopy and readelf):
        pytest.skip("llvm-objcopy / llvm-readelf not found")
    if not os.path.exists(LIB):
        pytest.skip("libgrws.so not built")
    fat = tmp_path / "fat.bin"
    subprocess.run([objcopy, f"--dump-section=.hip_fatbin={fat}", LIB, str(tmp_path / "host.so")], check=True,
                   capture_output=True)
    kernels = {}
    for i, co in enumerate(_code_objects(fat.read_bytes())):
        f = tmp_path / f"co{i}.o"
        f.write_bytes(co)
        notes = subprocess.run([readelf, "--notes", str(f)], check=True, capture_output=True, text=True).stdout
        # one YAML block per kernel: its keys, then `.name:` among them
        for blk in re.split(r"\n\s+- \.", notes):
            name = re.search(r"\bname:\s+(\S+)", blk)
            if not name:
                continue
            vals = {k: int(v) for k, v in re.findall(r"\.(private_segment_fixed_size|vgpr_count|vgpr_spill_count):\s+(\d+)", blk)}
            if vals:
                kernels[name.group(1)] = vals
    return kernels


def test_grouped_spmm_kernels_use_no_scratch(tmp_path):
    kernels = _kernel_metadata(tmp_path)
    grouped = {k: v for k, v in kernels.items() if re.search(r"spmm_grp2?d?_kernel", k)}
    assert any("spmm_grp2d_kernel" in k for k in grouped), "no direct-load slab-pair kernel in the library"
    for k, v in grouped.items():
        assert v.get("private_segment_fixed_size", 0) == 0, f"{k} uses scratch: {v}"
    # the slab-pair kernels (the product's default for 4-window groups): no
    # spills at all (a tuning-only 2-windows-per-wave kernel parks a few
    # registers in AGPRs, which is no memory traffic)
    for k, v in grouped.items():
        if re.search(r"spmm_grp2d?_kernel", k):
            assert v.get("vgpr_spill_count", 0) == 0, f"{k} spills: {v}"
        if re.search(r"spmm_grp2d?_kernelILi[12]ELi20E", k):
            assert v["vgpr_count"] <= 168, f"{k} leaves fewer than three waves per SIMD: {v}"
