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


HIP_SOURCES = ("dk_api.hip", "dk_f16.hip", "dk_bf16.hip")


def _filter(out: str) -> str:
    # hipcc's host pass reports the device-only feature flag as unknown; drop that noise.
    return "\n".join(l for l in out.splitlines() if "packed-fp32-ops" not in l)


def _run_all(cmds: list[list[str]]) -> None:
    """Run compile commands in parallel; raise with the output of the first failure."""
    procs = [(c, subprocess.Popen(c, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True))
             for c in cmds]
    failed = None
    for cmd, proc in procs:
        out = _filter(proc.communicate()[0])
        if proc.returncode != 0 and failed is None:
            failed = f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}"
        elif out.strip():
            print(out, file=sys.stderr)
    if failed:
        raise RuntimeError(failed)


def build(verbose: bool = False) -> Path:
    """Compile csrc/ into libdk_decode.so (always rebuilds). Returns the library path."""
    BUILD_DIR.mkdir(exist_ok=True)
    hipcc = _hipcc()
    objs = [BUILD_DIR / "dk_args.o"]
    cmds = [["g++", "-std=c++17", "-O2", "-fPIC", "-Wall", "-Wextra", f"-I{INCLUDE}",
             "-c", str(CSRC / "dk_args.cpp"), "-o", str(objs[0])]]
    for src in HIP_SOURCES:
        obj = BUILD_DIR / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([hipcc, *HIP_FLAGS, f"-I{INCLUDE}", "-c", str(CSRC / src), "-o", str(obj)])
    _run_all(cmds)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run_all([[hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs),
               "-o", str(tmp)]])
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
