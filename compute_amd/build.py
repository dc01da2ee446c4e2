"""Builds libmxrt.so (the C-ABI backend library) in-tree with hipcc for gfx950.

Run as ``python -m compute_amd.build`` or through ``__graft_entry__.build()``.  Object files go
to ``_build/`` at the repository root; the shared library to ``compute_amd/_lib/libmxrt.so``.
"""
from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = ROOT / "_build" / "mxrt"
LIB = PKG / "_lib" / "libmxrt.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed-fp32 VALU ops are disabled for every kernel (the compiler would otherwise form them
# from scalar/float2 code); the host pass warns that it does not know the feature.
COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
SOURCES = ["runtime.cpp", "graph.cpp", "qdense.hip", "qdense_skinny.hip", "qdense_gemv.hip", "qdense_gemm.hip", "qdense_refgemm.hip", "qdense_noalloc.hip", "ggml.hip", "dot.hip", "elementwise.hip"]


# The skinny kernel takes one arrival ticket per workgroup from a single lane; LLVM's atomic
# optimizer would turn that atomic into a wave-wide one whose result is waited for at once.  Its
# leading scalar arguments are preloaded into SGPRs at wave launch.
EXTRA = {"qdense_skinny.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
                               "-mllvm", "-amdgpu-kernarg-preload-count=8"]}


def _compile(src: str) -> Path:
    out = OBJ / (src + ".o")
    cmd = [HIPCC, *COMMON, *EXTRA.get(src, []), "-x", "hip", "-c", str(CSRC / src), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stderr}")
    return out


def build(verbose: bool = False) -> Path:
    """Compiles every source (always) and links libmxrt.so; returns the library path."""
    OBJ.mkdir(parents=True, exist_ok=True)
    LIB.parent.mkdir(parents=True, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(os.cpu_count() or 8, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
