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
SOURCES = ["rnrqr.hip", "small.hip", "check.hip", "orgqr.hip", "gen.hip", "hhqr.hip"]
HEADERS = ["common.hpp", "gemm_tn.hpp", "lu.hpp", "chol.hpp", "trsm.hpp", "small.hpp", "applyq.hpp", "wy.hpp"]
OUT = os.path.join(HERE, "librnrqr.so")
ARCH = os.environ.get("RNR_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build librnrqr.so)")


def compile_command(src: str, obj: str) -> list[str]:
    """hipcc line for one translation unit (device code for gfx950 only)."""
    return [hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-I", INCLUDE, "-c", "-o", obj, os.path.join(CSRC, src)]


def command(out: str = OUT) -> list[str]:
    """One-line equivalent of the build (every source compiled and linked in one call)."""
    return [hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-I", INCLUDE, "-o", out] + [os.path.join(CSRC, s) for s in SOURCES]


def build_library(verbose: bool = False) -> str:
    """Compile the library (always, also when it exists) and return its path.

    The translation units compile in parallel to objects under ``_build/`` and are linked
    into ``librnrqr.so`` next to this file."""
    bdir = os.path.join(HERE, "_build")
    os.makedirs(bdir, exist_ok=True)
    jobs = []
    for src in SOURCES:
        obj = os.path.join(bdir, os.path.splitext(src)[0] + ".o")
        cmd = compile_command(src, obj)
        if verbose:
            print(" ".join(cmd), flush=True)
        jobs.append((cmd, obj, subprocess.Popen(cmd, cwd=CSRC, stdout=subprocess.PIPE,
                                                stderr=subprocess.STDOUT, text=True)))
    objs, errors = [], []
    for cmd, obj, proc in jobs:
        out, _ = proc.communicate()
        if proc.returncode != 0:
            errors.append(" ".join(cmd) + "\n" + out)
        objs.append(obj)
    if errors:
        raise RuntimeError("hipcc failed:\n" + "\n".join(errors))
    tmp = OUT + ".tmp"
    link = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    proc = subprocess.run(link, cwd=CSRC, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("link failed:\n" + " ".join(link) + "\n" + proc.stdout + proc.stderr)
    if verbose:
        print(" ".join(link))
    os.replace(tmp, OUT)
    return OUT
