"""Builds the gfx950 shared library ``_liblocomp_amd.so`` in-tree with hipcc.

Usage: ``python -m locomp_amd.build`` (also called by ``__graft_entry__.build``).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJDIR = PKG / "_build"
LIB = PKG / "_liblocomp_amd.so"
SOURCES = ["dequant.hip", "gemv_w4.hip", "gemv_w8.hip", "gemv_x4.hip", "gemv_x8.hip", "gemv_xsilu.hip", "gemv_generic.hip", "gemv_group.hip", "gemv_rows16.hip", "gemv_fused.hip", "gemm.hip", "quantize.hip",
           "stream.hip", "norm.hip", "capi.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    # Packed-fp32 VALU ops are disabled for every device compile on this target.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", str(ROOT / "include"),
    "-Wall", "-Wno-unused-function",
]


# Per-source extra flags.  gemm.hip: select the VGPR-destination MFMA form;
# with AGPR destinations the allocator does not tie each MFMA's accumulator
# input to its output and copies accumulators between VGPRs and AGPRs.
EXTRA = {"gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src: str) -> Path:
    obj = OBJDIR / (Path(src).stem + ".o")
    cmd = [HIPCC, *FLAGS, *EXTRA.get(src, []), "-c", str(CSRC / src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    OBJDIR.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build()
