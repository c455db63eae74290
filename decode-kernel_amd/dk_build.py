"""Ahead-of-time build of libdk_decode.so (HIP for gfx950) into this directory.

Replaces the reference's nvcc JIT loader (src/cuda_/build.py:38-282): the library is
compiled once, in-tree, with hipcc, and loaded by ctypes (dk_lib.py). The host-only
argument checker (csrc/dk_args.cpp) is compiled with g++ and linked in.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
INCLUDE = HERE.parent / "include"
LIB_NAME = "libdk_decode.so"
LIB_PATH = HERE / LIB_NAME
BUILD_DIR = HERE / "_build"
ARCH = "gfx950"

# -packed-fp32-ops is disabled for all device code: the compiler may otherwise form
# v_pk_{add,mul,fma}_f32 from scalar float code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass reports the device-only feature flag as unknown; drop that noise.
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build(verbose: bool = False) -> Path:
    """Compile csrc/ into libdk_decode.so (always rebuilds). Returns the library path."""
    BUILD_DIR.mkdir(exist_ok=True)
    args_o = BUILD_DIR / "dk_args.o"
    dec_o = BUILD_DIR / "dk_decode.o"
    _run(["g++", "-std=c++17", "-O2", "-fPIC", "-Wall", "-Wextra", f"-I{INCLUDE}",
          "-c", str(CSRC / "dk_args.cpp"), "-o", str(args_o)])
    hipcc = _hipcc()
    _run([hipcc, *HIP_FLAGS, f"-I{INCLUDE}", "-c", str(CSRC / "dk_decode.hip"), "-o", str(dec_o)])
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", str(dec_o), str(args_o),
          "-o", str(tmp)])
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
