"""Ahead-of-time build of libdk_decode.so (HIP for gfx950) into this directory.

Replaces the reference's nvcc JIT loader (src/cuda_/build.py:38-282): the library is
compiled once, in-tree, with hipcc, and loaded by ctypes (dk_lib.py). The host-only
argument checker (csrc/dk_args.cpp) is compiled with g++ and linked in.
"""
from __future__ import annotations

import os
import re
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


HIP_SOURCES = ("dk_api.hip", "dk_paging.hip", "dk_append.hip")
# pass-1 kernel tables: each compiled once per head_dim (-DDK_HEAD_DIM=...)
KERNEL_SOURCES = ("dk_f16.hip", "dk_bf16.hip", "dk_f16_mfma.hip", "dk_bf16_mfma.hip",
                  "dk_f16_kv8.hip", "dk_bf16_kv8.hip", "dk_f16_kv8_mfma.hip",
                  "dk_bf16_kv8_mfma.hip")
HEAD_DIMS = (64, 128, 256)


# Per-kernel resource report of the device compiler (VGPRs, scratch, occupancy).
RESOURCE_FLAG = "-Rpass-analysis=kernel-resource-usage"


def _filter(out: str) -> str:
    # hipcc's host pass reports the device-only feature flag as unknown; the resource
    # remarks are parsed separately. Drop both, and the source lines the compiler echoes
    # under each remark (" 1179 | ..."), from what is echoed.
    return "\n".join(l for l in out.splitlines()
                     if "packed-fp32-ops" not in l and "kernel-resource-usage" not in l
                     and not l.startswith(("  ", "In file included from"))
                     and not re.match(r"\s*\d*\s*\|", l))


def kernel_resources(out: str) -> dict:
    """{kernel: {"VGPRs": n, "ScratchSize": bytes per lane, "Occupancy": waves/SIMD}}."""
    res, cur = {}, None
    for line in out.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            cur = res.setdefault(m.group(1), {})
            continue
        m = re.search(r"(VGPRs|ScratchSize \[bytes/lane\]|Occupancy \[waves/SIMD\]): (\d+)",
                      line)
        if m and cur is not None:
            cur[m.group(1).split()[0]] = int(m.group(2))
    return res


def _jobs() -> int:
    """Parallel compiles: MAX_JOBS if set, else the CPU count (at most 16)."""
    env = os.environ.get("MAX_JOBS")
    if env and env.isdigit() and int(env) > 0:
        return int(env)
    return max(1, min(16, os.cpu_count() or 1))


def _run_all(cmds: list[list[str]]) -> str:
    """Run compile commands, _jobs() at a time; raise with the output of the first failure.
    Returns the concatenated raw output (for the resource remarks)."""
    from concurrent.futures import ThreadPoolExecutor

    def run(c):
        p = subprocess.run(c, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        return p.returncode, p.stdout

    with ThreadPoolExecutor(max_workers=_jobs()) as pool:
        results = list(pool.map(run, cmds))
    procs = [(c, r) for c, r in zip(cmds, results)]
    failed = None
    raw = []
    for cmd, (returncode, text) in procs:
        raw.append(text)
        out = _filter(text)
        if returncode != 0 and failed is None:
            failed = f"build step failed ({returncode}): {' '.join(cmd)}\n{out}"
        elif out.strip():
            print(out, file=sys.stderr)
    if failed:
        raise RuntimeError(failed)
    return "\n".join(raw)


def build(verbose: bool = False, defines: tuple = (), out: Path = LIB_PATH,
          build_dir: Path = BUILD_DIR) -> Path:
    """Compile csrc/ into libdk_decode.so (always rebuilds). Returns the library path.
    `defines` (e.g. ("DK_PREFETCH_DEPTH=4",)) and another `out` / `build_dir` make a side
    build for comparisons, loadable through the DK_DECODE_LIB environment variable."""
    build_dir = Path(build_dir)
    out = Path(out)
    build_dir.mkdir(parents=True, exist_ok=True)
    hipcc = _hipcc()
    dflags = [f"-D{d}" for d in defines]
    objs = [build_dir / "dk_args.o"]
    cmds = [["g++", "-std=c++17", "-O2", "-fPIC", "-Wall", "-Wextra", *dflags, f"-I{INCLUDE}",
             "-c", str(CSRC / "dk_args.cpp"), "-o", str(objs[0])]]
    for src in HIP_SOURCES:
        obj = build_dir / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([hipcc, *HIP_FLAGS, *dflags, RESOURCE_FLAG, f"-I{INCLUDE}", "-c",
                     str(CSRC / src), "-o", str(obj)])
    for src in KERNEL_SOURCES:
        for d in HEAD_DIMS:
            obj = build_dir / f"{Path(src).stem}.d{d}.o"
            objs.append(obj)
            cmds.append([hipcc, *HIP_FLAGS, *dflags, f"-DDK_HEAD_DIM={d}", RESOURCE_FLAG,
                         f"-I{INCLUDE}", "-c", str(CSRC / src), "-o", str(obj)])
    res = kernel_resources(_run_all(cmds))
    (build_dir / "kernel_resources.txt").write_text("".join(
        f"{k} VGPRs={v.get('VGPRs')} scratch={v.get('ScratchSize')} "
        f"occupancy={v.get('Occupancy')}\n" for k, v in sorted(res.items())))
    # Every kernel keeps its state in registers and LDS: scratch memory here would mean an
    # array indexed by a lane-dependent value or a spill, both a large slowdown.
    scratch = sorted(k for k, v in res.items() if v.get("ScratchSize", 0) > 0)
    if scratch:
        raise RuntimeError(f"{len(scratch)} kernels use scratch memory: {scratch[:4]}")
    tmp = out.with_suffix(".so.tmp")
    _run_all([[hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs),
               "-o", str(tmp)]])
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build(verbose=True)
