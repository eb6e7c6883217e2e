"""In-tree build of ``librnrqr.so`` for gfx950 with hipcc (no CMake, no JIT cache).

The library goes next to this file so it travels with the repository snapshot.
Packed-FP32 instructions are disabled for every HIP translation unit
(``-Xclang -target-feature -Xclang -packed-fp32-ops``).
"""
from __future__ import annotations

import os
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
SOURCES = ["rnrqr.hip"]
HEADERS = ["common.hpp", "gemm_tn.hpp", "lu.hpp", "chol.hpp", "trsm.hpp"]
OUT = os.path.join(HERE, "librnrqr.so")
ARCH = os.environ.get("RNR_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build librnrqr.so)")


def command(out: str = OUT) -> list[str]:
    return [hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-I", INCLUDE, "-o", out] + [os.path.join(CSRC, s) for s in SOURCES]


def build_library(verbose: bool = False) -> str:
    """Compile the library (always, also when it exists) and return its path."""
    tmp = OUT + ".tmp"
    cmd = command(tmp)
    proc = subprocess.run(cmd, cwd=CSRC, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + " ".join(cmd) + "\n" + proc.stdout + proc.stderr)
    if verbose:
        print(" ".join(cmd))
    os.replace(tmp, OUT)
    return OUT
