"""Build libqwen4mix.so (the HIP kernels + C ABI) in-tree for gfx950.

One hipcc invocation over csrc/*.hip, output next to this file. Every HIP
translation unit is compiled with packed-FP32 instruction selection disabled
(``-Xclang -target-feature -Xclang -packed-fp32-ops``); hipcc's host pass warns
that it does not know that feature, which is harmless. Kernels whose arguments
are plain scalars get their first 16 argument dwords preloaded into scalar
registers at wave start (``-amdgpu-kernarg-preload-count=16``; firmware without
preloading runs the kernel's own argument loads instead).
"""

from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
LIB_NAME = "libqwen4mix.so"
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the qwen4mix HIP library cannot be built")


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(PKG, "csrc", "*.hip")))


def build(verbose: bool = False) -> str:
    """Compile every kernel source into the package's shared library; return its path."""
    out = os.path.join(PKG, LIB_NAME)
    tmp = out + ".tmp"
    cmd = [
        hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-mllvm", "-amdgpu-kernarg-preload-count=16",
        "-I", os.path.join(ROOT, "include"), "-I", os.path.join(PKG, "csrc"),
        "-o", tmp, *sources(),
    ]
    if verbose:
        print(" ".join(cmd), file=sys.stderr)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-8000:]}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
