"""Build libqmoe.so (all HIP sources under csrc/) for gfx950 with hipcc.

The library is built in-tree, next to this file, so it travels with the
repository tree; nothing is JIT-compiled at import time.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG.parent / "csrc"
INCLUDE = PKG.parent.parent / "include"
LIB = PKG / "libqmoe.so"
ARCH = os.environ.get("QMOE_OFFLOAD_ARCH", "gfx950")

# Packed-FP32 VALU ops are disabled for all device code.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


# Per-file additions. w4_gemv.hip: atomics stay as written (the decode and
# projection kernels bump counters from one lane; the wave-aggregating
# rewrite reads the result back at once, which stalls the wave on the
# atomic's round trip).
# w8_gemm.hip: MFMA accumulators stay in VGPRs (the AGPR form moved the group
# sums to VGPRs and back for every scale-group fma).
FILE_FLAGS = {"w4_gemv.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
              "w8_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def flags_for(src: Path) -> list:
    return [*HIPCC_FLAGS, *FILE_FLAGS.get(src.name, [])]


def sources():
    return sorted(CSRC.glob("*.hip"))


def _hipcc():
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; cannot build libqmoe.so")
    return exe


def build(verbose: bool = False) -> Path:
    """Compile every csrc/*.hip to an object file and link libqmoe.so."""
    hipcc = _hipcc()
    objdir = PKG.parent / "_build"
    objdir.mkdir(exist_ok=True)
    srcs = sources()

    def compile_one(src: Path) -> Path:
        obj = objdir / (src.stem + ".o")
        cmd = [hipcc, *flags_for(src), "-I", str(CSRC), "-I", str(INCLUDE), "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr}")
        return obj

    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link of libqmoe.so failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
