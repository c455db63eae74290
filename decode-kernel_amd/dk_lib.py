"""ctypes binding of libdk_decode.so (the C ABI declared in include/dk_decode.h).

This module replaces the reference's pybind11/JIT boundary (src/cuda_/build.py:256-282,
src/cuda_/attention_ext.cu:613-626) with plain C calls: no torch types cross the
boundary, only device pointers, sizes, element strides and a hipStream_t.

Loading fails loudly: there is no CPU or PyTorch fallback for the decode path.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("DK_DECODE_LIB", HERE / "libdk_decode.so"))

DK_F16 = 0
DK_BF16 = 1
DK_KV_SAME = 0
DK_KV_FP8_E4M3 = 2
ABI_VERSION = 3
STATIC_SCRATCH_BYTES = 32 << 20     # DK_STATIC_SCRATCH_BYTES: dk_decode_attention_noalloc

DK_OK = 0
DK_EINVAL = -1
DK_ENULL = -2
DK_EWORKSPACE = -3
DK_EUNSUPPORTED = -4


class DecodeArgumentError(ValueError, RuntimeError):
    """Invalid argument rejected before any launch.

    Subclasses both ValueError and RuntimeError: the reference reports these through
    TORCH_CHECK (a RuntimeError in Python, src/cuda_/attention_ext.cu:506-509,549-552),
    while layout validation speaks of ValueError (src/layout.py:18).
    """


class DecodeLaunchError(RuntimeError):
    """A HIP error returned by a kernel launch."""


class DkStrides(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in
                ("q_b", "q_h", "kv_p", "kv_r", "kv_s", "kv_h", "o_b", "o_h")]


class DkOptions(ctypes.Structure):
    _fields_ = [("qk_path", ctypes.c_int32), ("waves_per_group", ctypes.c_int32),
                ("waves_per_cu", ctypes.c_int32), ("schedule", ctypes.c_int32),
                ("max_pages_per_seq", ctypes.c_int32), ("sm_scale", ctypes.c_float),
                ("kv_dtype", ctypes.c_int32), ("k_scale", ctypes.c_float),
                ("v_scale", ctypes.c_float), ("logit_cap", ctypes.c_float),
                ("window", ctypes.c_int32), ("reserved", ctypes.c_int32 * 1),
                ("sinks", ctypes.c_void_p)]


_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); must match include/dk_decode.h
SIGNATURES = {
    "dk_abi_version": (ctypes.c_int, []),
    "dk_last_error": (ctypes.c_char_p, []),
    "dk_workspace_bytes": (_SZ, [_I32, _I32, _I32, _I32, _I32]),
    "dk_partials_layout": (ctypes.c_int, [_I32, _I32, _I32, _I32, ctypes.POINTER(_SZ),
                                          ctypes.POINTER(_SZ), ctypes.POINTER(_SZ),
                                          ctypes.POINTER(_SZ)]),
    "dk_choose_split": (ctypes.c_int, [_I32, _I32, _I32, _I32, _I32, _I64, _I32]),
    "dk_plan_schedule": (ctypes.c_int, [_I32, _I32, _I32, _I32, _I64, _I32, _I32,
                                        ctypes.POINTER(DkOptions), _I32]),
    "dk_decode_attention": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _SZ, _I32, _I32, _I32,
                                           _I32, _I32, _I64, _I64, _I32,
                                           ctypes.POINTER(DkStrides), _I32, _P]),
    "dk_decode_attention_ex": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _SZ, _I32, _I32,
                                              _I32, _I32, _I32, _I64, _I64, _I32,
                                              ctypes.POINTER(DkStrides), _I32,
                                              ctypes.POINTER(DkOptions), _P]),
    "dk_decode_attention_noalloc": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _I32, _I32, _I32,
                                                   _I32, _I32, _I64, _I64, _I32,
                                                   ctypes.POINTER(DkStrides), _I32,
                                                   ctypes.POINTER(DkOptions), _P]),
    "dk_decode_attention_kv": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _SZ, _I32, _I32,
                                              _I32, _I32, _I32, _I64, _I64, _I32,
                                              ctypes.POINTER(DkStrides), _I32,
                                              ctypes.POINTER(DkOptions), _P]),
    "dk_build_page_table": (ctypes.c_int, [_P, _I64, _P, _P, _I32, _I32, _P, _P, _I64, _P, _P]),
    "dk_expand_page_table": (ctypes.c_int, [_P, _P, _P, _I32, _I32, _I32, _I64, _I64, _P, _P,
                                            _I64, _P, _P]),
    "dk_append_kv": (ctypes.c_int, [_P, _P, _P, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _I32,
                                    _I32, _I32, _I32, _I32, _I32, _I64, _I64, _I32,
                                    ctypes.POINTER(DkStrides), _P]),
    "dk_append_kv_fp8": (ctypes.c_int, [_P, _P, _P, _I64, _I64, _P, _P, _P, _P, _P, _P, _P,
                                        _I32, _I32, _I32, _I32, _I32, _I32, _I64, _I64, _I32,
                                        ctypes.c_float, ctypes.c_float,
                                        ctypes.POINTER(DkStrides), _P]),
    "dk_decode_partials": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _SZ, _I32, _I32, _I32, _I32,
                                          _I32, _I64, _I64, _I32, ctypes.POINTER(DkStrides),
                                          _I32, ctypes.POINTER(DkOptions), _P]),
    "dk_merge_partials": (ctypes.c_int, [_P, _SZ, _P, _I32, _I32, _I32, _I32, _I64, _I64, _I32,
                                         _P]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load the library once; raise ImportError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: the HIP decode-attention library has not been built "
            "(run `python __graft_entry__.py build` or decode-kernel_amd/dk_build.py)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.dk_abi_version()
    if ver != ABI_VERSION:
        raise ImportError(f"{LIB_PATH}: ABI version {ver}, expected {ABI_VERSION}")
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    """Map a C-ABI return code to a Python exception."""
    if rc == DK_OK:
        return
    msg = load().dk_last_error().decode(errors="replace")
    if rc < 0:
        raise DecodeArgumentError(f"{what}: {msg}")
    raise DecodeLaunchError(f"{what}: HIP error {rc}: {msg}")


def workspace_bytes(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                    split_kv: int) -> int:
    """Scratch bytes for split_kv (0 = balanced mode, 1 = none, > 1 = explicit partials)."""
    return int(load().dk_workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim, split_kv))


def partials_layout(batch: int, num_q_heads: int, head_dim: int, split_kv: int):
    """(off_o, off_m, off_l, total) byte offsets of the fp32 partials in a workspace."""
    o, m, l, t = _SZ(), _SZ(), _SZ(), _SZ()
    check(load().dk_partials_layout(batch, num_q_heads, head_dim, split_kv, ctypes.byref(o),
                                    ctypes.byref(m), ctypes.byref(l), ctypes.byref(t)),
          "dk_partials_layout")
    return o.value, m.value, l.value, t.value


def choose_split(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                 dtype_code: int, avg_pages_per_seq: int, device: int) -> int:
    rc = load().dk_choose_split(batch, num_q_heads, num_kv_heads, head_dim, dtype_code,
                                avg_pages_per_seq, device)
    if rc < 1:
        check(rc if rc != 0 else DK_EINVAL, "dk_choose_split")
    return int(rc)


def plan_schedule(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                  num_indices: int, dtype_code: int, split_kv: int,
                  opts: "DkOptions | None" = None, device: int = -1) -> int:
    """Schedule a full call runs: 1 one pass, 0 balanced + merge, > 1 explicit split."""
    rc = load().dk_plan_schedule(batch, num_q_heads, num_kv_heads, head_dim, num_indices,
                                 dtype_code, split_kv,
                                 ctypes.byref(opts) if opts is not None else None, device)
    if rc < 0:
        check(rc, "dk_plan_schedule")
    return int(rc)


SCHEDULE_AUTO = 0
SCHEDULE_BALANCED = 1
SCHEDULE_ONE_PASS = 2


def options(qk_path: int = 0, waves_per_group: int = 0, waves_per_cu: int = 0,
            schedule: int = SCHEDULE_AUTO, max_pages_per_seq: int = 0,
            sm_scale: float = 0.0, kv_dtype: int = DK_KV_SAME, k_scale: float = 0.0,
            v_scale: float = 0.0, logit_cap: float = 0.0, window: int = 0,
            sinks: int = 0) -> DkOptions:
    o = DkOptions()
    o.sinks = sinks or None       # device address of num_q_heads fp32 sink logits
    o.logit_cap = logit_cap
    o.window = window
    o.sm_scale = sm_scale
    o.kv_dtype = kv_dtype
    o.k_scale = k_scale
    o.v_scale = v_scale
    o.qk_path = qk_path
    o.waves_per_group = waves_per_group
    o.waves_per_cu = waves_per_cu
    o.schedule = schedule
    o.max_pages_per_seq = max_pages_per_seq
    return o
