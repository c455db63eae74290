"""Decode attention over a FlashInfer-NHD paged KV cache, on MI355X through HIP.

Drop-in for the reference dispatch (src/attention.py:26-58):

    from attention import decode_attention
    out = decode_attention(q, kv_data, kv_indptr, kv_indices, kv_last_page_len, split_kv=4)

Same arguments and meaning; the reference's two pybind entry points
(`decode_attention_naive`, `decode_attention_split_kv`, src/cuda_/attention_ext.cu:613-626)
are provided too, behind `get_hip_ext()` (the counterpart of `get_cuda_ext()`,
src/cuda_/build.py:256). Every call goes to libdk_decode.so (HIP, gfx950); there is no
PyTorch or CPU fallback, and a missing library raises ImportError.

Differences from the reference, all extensions: bf16 as well as fp16; an fp8 (E4M3) cache
under fp16/bf16 queries, with per-tensor k_scale / v_scale; any split_kv >= 1
(the reference allows 1..32), and split_kv=0 or None selects the balanced mode, in which
a persistent grid gives every wavefront an equal share of all (sequence, kv head, page)
work whatever the sequence lengths; work runs on torch's current stream of q's device
(the reference used the legacy default stream); empty sequences (no pages) produce zeros.
"""
from __future__ import annotations

import ctypes
import math
from types import SimpleNamespace
from typing import Optional

import torch

import dk_lib
from dk_lib import DecodeArgumentError

PAGE_SIZE = 16
SUPPORTED_HEAD_DIMS = (64, 128, 256)
_DTYPE_CODE = {torch.float16: dk_lib.DK_F16, torch.bfloat16: dk_lib.DK_BF16}
KV_FP8 = torch.float8_e4m3fn            # OCP E4M3: the fp8 cache format the kernel reads


def _fail(msg: str) -> None:
    raise DecodeArgumentError(msg)


def _kv_layout(kv_data):
    """The paged cache in either FlashInfer NHD form: one tensor
    (num_pages, 2, page_size, num_kv_heads, head_dim) with K at [:, 0] and V at [:, 1]
    (src/layout.md:41-69), or a (k_cache, v_cache) pair of (num_pages, page_size,
    num_kv_heads, head_dim) tensors with equal strides (SGLang's token pools)."""
    if isinstance(kv_data, (tuple, list)):
        if len(kv_data) != 2 or not all(isinstance(t, torch.Tensor) for t in kv_data):
            raise TypeError("kv_data must be a tensor or a (k_cache, v_cache) pair of tensors")
        k, v = kv_data
        if k.dim() != 4 or v.shape != k.shape:
            _fail("k_cache and v_cache must both be (num_pages, page_size, num_kv_heads, "
                  f"head_dim); got {tuple(k.shape)} and {tuple(v.shape)}")
        if v.stride() != k.stride() or v.dtype != k.dtype or v.device != k.device:
            _fail("k_cache and v_cache must have the same strides, dtype and device")
        return SimpleNamespace(k=k, v=v, num_pages=k.shape[0], page_size=k.shape[1],
                               hkv=k.shape[2], d=k.shape[3], dtype=k.dtype, device=k.device,
                               strides=(k.stride(0), 0, k.stride(1), k.stride(2)),
                               d_stride=k.stride(3))
    if not isinstance(kv_data, torch.Tensor):
        raise TypeError(f"kv_data must be a torch.Tensor, got {type(kv_data).__name__}")
    if kv_data.dim() != 5:
        _fail("kv_data must be 5-D")
    if kv_data.shape[1] != 2:
        _fail("kv_data dim-1 must be 2 (K/V)")
    return SimpleNamespace(k=kv_data, v=None, num_pages=kv_data.shape[0],
                           page_size=kv_data.shape[2], hkv=kv_data.shape[3],
                           d=kv_data.shape[4], dtype=kv_data.dtype, device=kv_data.device,
                           strides=(kv_data.stride(0), kv_data.stride(1), kv_data.stride(2),
                                    kv_data.stride(3)),
                           d_stride=kv_data.stride(4))


def _check(q, kv_data, kv_indptr, kv_indices, kv_last_page_len, wide_pages=False):
    """Host-side checks: the reference's TORCH_CHECKs (attention_ext.cu:506-509,549-552)
    plus the layout invariants that need no device read (src/layout.md:171-178).
    wide_pages: pages of any multiple of 16 tokens pass (the checks that run before such a
    table is rewritten over 16-token sub-pages on the device). Returns the cache layout."""
    for name, t in (("q", q), ("kv_indptr", kv_indptr),
                    ("kv_indices", kv_indices), ("kv_last_page_len", kv_last_page_len)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    kv = _kv_layout(kv_data)
    if wide_pages:
        if kv.page_size <= 0 or kv.page_size % PAGE_SIZE:
            _fail(f"pages must hold a multiple of 16 tokens, got {kv.page_size}")
    elif kv.page_size != PAGE_SIZE:
        _fail(f"page_size must be 16 for the HIP kernel (decode_attention also takes a "
              f"multiple of 16), got {kv.page_size}")
    if not q.is_cuda:
        _fail("q must be on CUDA")
    if q.dtype not in _DTYPE_CODE:
        _fail(f"q must be fp16 or bf16, got {q.dtype}")
    if q.dim() != 3:
        _fail(f"q must be 3-D (batch, num_q_heads, head_dim), got shape {tuple(q.shape)}")
    if kv.dtype != q.dtype and kv.dtype != KV_FP8:
        _fail(f"kv_data dtype {kv.dtype} must match q dtype {q.dtype} (or be "
              f"torch.float8_e4m3fn)")
    if q.shape[2] != kv.d:
        _fail(f"head_dim mismatch: q has {q.shape[2]}, kv_data has {kv.d}")
    if q.shape[2] not in SUPPORTED_HEAD_DIMS:
        _fail(f"head_dim must be 64, 128, or 256; got {q.shape[2]}")
    if q.shape[1] % kv.hkv != 0:
        _fail(f"num_q_heads ({q.shape[1]}) must be divisible by num_kv_heads ({kv.hkv})")
    for name, t in (("kv_indptr", kv_indptr), ("kv_indices", kv_indices),
                    ("kv_last_page_len", kv_last_page_len)):
        if t.dtype != torch.int32:
            _fail(f"{name} must be int32, got {t.dtype}")
        if t.dim() != 1:
            _fail(f"{name} must be 1-D")
        if t.device != q.device:
            _fail(f"{name} must be on {q.device}, got {t.device}")
    if kv.device != q.device:
        _fail(f"kv_data must be on {q.device}, got {kv.device}")
    if q.shape[0] != kv_indptr.shape[0] - 1:
        _fail(f"q.shape[0] ({q.shape[0]}) must equal kv_indptr.shape[0] - 1 "
              f"({kv_indptr.shape[0] - 1})")
    if kv_last_page_len.shape[0] != q.shape[0]:
        _fail("kv_last_page_len must have one entry per sequence")
    if q.stride(2) != 1 or kv.d_stride != 1:
        _fail("the head_dim stride of q and kv_data must be 1")
    return kv


def _check_sinks(sinks, q) -> None:
    """Attention sinks: None, or one fp32 logit per q head on q's device (contiguous)."""
    if sinks is None:
        return
    if not isinstance(sinks, torch.Tensor):
        raise TypeError(f"sinks must be a torch.Tensor, got {type(sinks).__name__}")
    if sinks.dtype != torch.float32 or sinks.dim() != 1 or sinks.shape[0] != q.shape[1] or \
            not sinks.is_contiguous() or sinks.device != q.device:
        _fail(f"sinks must be a contiguous float32 tensor of num_q_heads ({q.shape[1]}) "
              f"logits on {q.device}; got {tuple(sinks.shape)} {sinks.dtype} on "
              f"{sinks.device}")


def _contig1d(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() else t.contiguous()


def _kv_options(kv, k_scale, v_scale):
    """(kv_dtype, k_scale, v_scale) for dk_options: an fp8 cache takes positive finite
    per-tensor scales (default 1); a cache of q's type takes none."""
    if kv.dtype != KV_FP8:
        if k_scale not in (None, 1.0) or v_scale not in (None, 1.0):
            _fail("k_scale / v_scale apply to a torch.float8_e4m3fn cache only")
        return dk_lib.DK_KV_SAME, 0.0, 0.0
    scales = []
    for name, x in (("k_scale", k_scale), ("v_scale", v_scale)):
        x = 1.0 if x is None else float(x)
        if not math.isfinite(x) or x <= 0.0:
            _fail(f"{name} must be finite and > 0, got {x}")
        scales.append(x)
    return dk_lib.DK_KV_FP8_E4M3, scales[0], scales[1]


def _logit_cap(logit_cap) -> float:
    """logit_cap as dk_options takes it: 0.0 for off (None or 0), else finite and > 0."""
    if logit_cap is None:
        return 0.0
    cap = float(logit_cap)
    if not math.isfinite(cap) or cap < 0.0:
        _fail(f"logit_cap must be finite and >= 0 (0 = off), got {logit_cap}")
    return cap


def _window(window) -> int:
    """window as dk_options takes it: 0 for all tokens (None or 0), else >= 1."""
    if window is None:
        return 0
    if isinstance(window, bool) or not isinstance(window, int) or window < 0:
        _fail(f"window must be an int >= 0 (0 = all tokens), got {window!r}")
    return window


def _strides(q, kv_data, out) -> dk_lib.DkStrides:
    s = dk_lib.DkStrides()
    s.q_b, s.q_h = q.stride(0), q.stride(1)
    s.kv_p, s.kv_r, s.kv_s, s.kv_h = _kv_layout(kv_data).strides
    if out is not None:
        s.o_b, s.o_h = out.stride(0), out.stride(1)
    return s


def resolve_split(split_kv: Optional[int]) -> int:
    """split_kv as the C ABI takes it: 0 for the balanced mode (None or 0), else >= 1."""
    if split_kv is None:
        return 0
    if isinstance(split_kv, bool) or not isinstance(split_kv, int):
        raise TypeError(f"split_kv must be an int, got {type(split_kv).__name__}")
    if split_kv < 0:
        _fail(f"split_kv must be >= 1 (or 0/None for the balanced mode), got {split_kv}")
    return split_kv


def plan_hint(kv_indptr_host) -> int:
    """max_pages_per_seq for decode_attention from a HOST copy of kv_indptr (a list, numpy
    array or CPU tensor), computed once per batch outside the decode call, as serving
    frameworks keep sequence lengths on the host. Never reads device memory."""
    if isinstance(kv_indptr_host, torch.Tensor):
        if kv_indptr_host.device.type != "cpu":
            raise ValueError("plan_hint takes a host copy of kv_indptr")
        kv_indptr_host = kv_indptr_host.tolist()
    ip = [int(x) for x in kv_indptr_host]
    return max((b - a for a, b in zip(ip[:-1], ip[1:])), default=0)


def choose_split(q: torch.Tensor, kv_data: torch.Tensor, kv_indices: torch.Tensor) -> int:
    """An explicit split count chosen from occupancy (for callers that want one)."""
    batch = q.shape[0]
    avg = kv_indices.shape[0] // batch if batch else 0
    return dk_lib.choose_split(batch, q.shape[1], _kv_layout(kv_data).hkv, q.shape[2],
                               _DTYPE_CODE[q.dtype], avg, q.device.index or 0)


def _tensor_sig(t):
    """What the host-side checks of one tensor argument depend on."""
    return (t.shape, t.stride(), t.dtype, t.device)


def _kv_sig(kv_data):
    if isinstance(kv_data, torch.Tensor):
        return _tensor_sig(kv_data)
    if isinstance(kv_data, (tuple, list)) and len(kv_data) == 2 and \
            all(isinstance(t, torch.Tensor) for t in kv_data):
        return (_tensor_sig(kv_data[0]), _tensor_sig(kv_data[1]))
    return None          # not cacheable: the slow path raises the type error


class _CallPlan:
    """Everything decode_attention derives from its arguments' shapes, dtypes, devices,
    strides and options -- validated once, then reused by every call with the same
    signature (a model's layers share one): the ctypes argument tuple (strides and options
    structs included), the scratch sizes, the entry point."""

    __slots__ = ("shape", "ws_need", "split_kv", "pair", "contig", "out_shape", "dtype",
                 "device", "batch", "opts", "sinks")

    def __init__(self, q, kv_data, kv_indptr, kv_indices, kv_last_page_len, split_kv, out,
                 workspace, qk_path, waves_per_group, waves_per_cu, schedule,
                 max_pages_per_seq, sm_scale, k_scale, v_scale, logit_cap, window,
                 sinks=None):
        kv = _check(q, kv_data, kv_indptr, kv_indices, kv_last_page_len)
        _check_sinks(sinks, q)
        self.sinks = None if sinks is None else (sinks.shape, sinks.dtype, sinks.device)
        if sm_scale is not None and (not math.isfinite(sm_scale) or sm_scale <= 0.0):
            _fail(f"sm_scale must be finite and > 0, got {sm_scale}")
        kv_dtype, k_sc, v_sc = _kv_options(kv, k_scale, v_scale)
        cap = _logit_cap(logit_cap)
        win = _window(window)
        split = resolve_split(split_kv)
        batch, hq, d = q.shape
        if out is not None and (out.shape != q.shape or out.dtype != q.dtype or
                                out.device != q.device or out.stride(2) != 1):
            _fail("out must match q's shape, dtype and device with unit head_dim stride")
        self.batch, self.out_shape, self.dtype, self.device = batch, (batch, hq, d), q.dtype, \
            q.device
        self.split_kv = split
        self.pair = kv.v is not None
        self.contig = (kv_indptr.is_contiguous(), kv_indices.is_contiguous(),
                       kv_last_page_len.is_contiguous())
        self.ws_need = dk_lib.workspace_bytes(batch, hq, kv.hkv, d, split) if batch else 0
        if self.ws_need and workspace is not None and (
                workspace.numel() * workspace.element_size() < self.ws_need or
                workspace.device != q.device):
            _fail(f"workspace must hold {self.ws_need} bytes on {q.device}")
        strides = dk_lib.DkStrides()
        strides.q_b, strides.q_h = q.stride(0), q.stride(1)
        strides.kv_p, strides.kv_r, strides.kv_s, strides.kv_h = kv.strides
        # out's strides: those of the caller's out, else of a fresh contiguous tensor
        strides.o_b, strides.o_h = (out.stride(0), out.stride(1)) if out is not None else \
            (hq * d, d)
        opts = dk_lib.options(qk_path, waves_per_group, waves_per_cu, schedule,
                              max_pages_per_seq, sm_scale or 0.0, kv_dtype, k_sc, v_sc, cap, win,
                              0 if sinks is None else sinks.data_ptr())
        self.opts = opts
        self.shape = (batch, hq, kv.hkv, d, kv.page_size, kv.num_pages, kv_indices.shape[0],
                      _DTYPE_CODE[q.dtype], ctypes.byref(strides), split, ctypes.byref(opts),
                      strides, opts)      # the structs last, kept alive with the plan


class _LibraryScratch:
    """The workspace the library owns for calls made without a caller workspace, one per
    (device, stream): a call allocates only when its problem outgrows it (calls on one
    stream never overlap, and a replaced buffer is freed in stream order). Calls under
    graph capture do not use it (a captured call keeps its own; see decode_attention)."""

    def __init__(self):
        self._by_stream = {}

    def get(self, device, stream: int, ws_need: int):
        key = (device, stream)
        ws = self._by_stream.get(key)
        if ws is None or ws.numel() < ws_need:
            ws = self._by_stream[key] = torch.empty(ws_need, dtype=torch.uint8, device=device)
        return ws


_SCRATCH = _LibraryScratch()
_PLANS: dict = {}
_PLANS_MAX = 512


def _raw_stream(device) -> int:
    """hipStream_t of torch's current stream on `device`."""
    try:
        return torch._C._cuda_getCurrentRawStream(device.index)
    except (AttributeError, TypeError):
        return torch.cuda.current_stream(device).cuda_stream


def _page_size_of(kv_data) -> Optional[int]:
    """Tokens per page of a cache in either form (None if it is neither)."""
    if isinstance(kv_data, torch.Tensor):
        return kv_data.shape[2] if kv_data.dim() == 5 else None
    if isinstance(kv_data, (tuple, list)) and len(kv_data) == 2 and \
            isinstance(kv_data[0], torch.Tensor) and kv_data[0].dim() == 4:
        return kv_data[0].shape[1]
    return None


def _sub_page_view(t: torch.Tensor, page_dim: int, page_size: int):
    """A view of the cache tensor `t` (pages of page_size = 16 s token rows along
    page_dim, pages along dim 0) as 16-token pages: page p's sub-page j is view page
    p * mult + j, mult = (page stride) / (16 token rows). The view ends at the last real
    sub-page. Returns (view, mult)."""
    row = t.stride(page_dim)
    step = PAGE_SIZE * row
    if row <= 0 or t.stride(0) % step != 0:
        _fail(f"pages of {page_size} tokens are read as 16-token sub-pages, so the page "
              f"stride ({t.stride(0)}) must be a multiple of 16 token rows ({step})")
    mult = t.stride(0) // step
    n = t.shape[0]
    shape = list(t.shape)
    shape[0] = (n - 1) * mult + page_size // PAGE_SIZE if n > 0 else 0
    shape[page_dim] = PAGE_SIZE
    stride = list(t.stride())
    stride[0] = step
    return t.as_strided(shape, stride), mult


def sixteen_token_pages(kv_data, kv_indptr=None, kv_indices=None, kv_last_page_len=None):
    """A cache with pages of a multiple of 16 tokens, as decode_attention reads it: the
    same memory viewed as 16-token pages (no copy) and, when the page table is given, that
    table rewritten over the 16-token sub-pages on the device (paging.expand_page_table,
    one small kernel, no host sync). Returns (view, kv_indptr, kv_indices,
    kv_last_page_len) (the tables None when not given). decode_attention does this on
    every call with such a cache; a model whose layers share one page table can rewrite
    it once per step and call decode_attention on each layer's view with that table."""
    import paging
    page_size = _page_size_of(kv_data)
    if page_size is None or page_size <= 0 or page_size % PAGE_SIZE:
        _fail(f"pages must hold a multiple of 16 tokens, got {page_size}")
    if isinstance(kv_data, torch.Tensor):
        view, mult = _sub_page_view(kv_data, 2, page_size)
        num_pages = kv_data.shape[0]
    else:
        k, v = kv_data
        if k.stride() != v.stride() or k.shape != v.shape:
            _fail("k_cache and v_cache must have the same shape and strides")
        (kv_k, mult), (kv_v, _) = _sub_page_view(k, 1, page_size), _sub_page_view(v, 1, page_size)
        view, num_pages = (kv_k, kv_v), k.shape[0]
    if kv_indptr is None:
        return view, None, None, None
    cache_dev = kv_data.device if isinstance(kv_data, torch.Tensor) else kv_data[0].device
    for name, t in (("kv_indptr", kv_indptr), ("kv_indices", kv_indices),
                    ("kv_last_page_len", kv_last_page_len)):
        if not isinstance(t, torch.Tensor) or t.dtype != torch.int32 or t.dim() != 1:
            _fail(f"{name} must be a 1-D int32 tensor")
        if t.device != cache_dev:
            _fail(f"{name} must be on the cache's device {cache_dev}, got {t.device}")
    indptr, indices, last = paging.expand_page_table(
        _contig1d(kv_indptr), _contig1d(kv_indices), _contig1d(kv_last_page_len), page_size,
        mult, num_pages)
    return view, indptr, indices, last


def _decode_over_sub_pages(q, kv_data, kv_indptr, kv_indices, kv_last_page_len, split_kv,
                           page_size, kw):
    """decode_attention over a cache of pages of a multiple of 16 tokens (see
    sixteen_token_pages); the plan hint scales to sub-pages. The arguments pass the host
    checks before the expansion kernel reads the tables."""
    _check(q, kv_data, kv_indptr, kv_indices, kv_last_page_len, wide_pages=True)
    view, indptr, indices, last = sixteen_token_pages(kv_data, kv_indptr, kv_indices,
                                                      kv_last_page_len)
    kw = dict(kw)
    if kw.get("max_pages_per_seq"):
        kw["max_pages_per_seq"] *= page_size // PAGE_SIZE
    return decode_attention(q, view, indptr, indices, last, split_kv, **kw)


def decode_attention(
    q: torch.Tensor,
    kv_data: torch.Tensor,
    kv_indptr: torch.Tensor,
    kv_indices: torch.Tensor,
    kv_last_page_len: torch.Tensor,
    split_kv: Optional[int] = 1,
    *,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
    qk_path: int = 0,
    waves_per_group: int = 0,
    waves_per_cu: int = 0,
    schedule: int = 0,
    max_pages_per_seq: int = 0,
    sm_scale: Optional[float] = None,
    k_scale: Optional[float] = None,
    v_scale: Optional[float] = None,
    logit_cap: Optional[float] = None,
    window: Optional[int] = None,
    sinks: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Decode attention over a paged KV cache (reference src/attention.py:26-58).

    Args:
        q                : (batch, num_q_heads, head_dim), fp16 or bf16, on a GPU
        kv_data          : (num_pages, 2, 16, num_kv_heads, head_dim), q's dtype or
                           torch.float8_e4m3fn (NHD), or a (k_cache, v_cache) pair of
                           (num_pages, 16, num_kv_heads, head_dim) tensors with equal
                           strides
        kv_indptr        : (batch + 1,) int32 CSR row pointer into kv_indices
        kv_indices       : (kv_indptr[-1],) int32 physical page ids
        kv_last_page_len : (batch,) int32 valid tokens in each sequence's last page
        split_kv         : KV partitions per (sequence, head). 1 -> one pass writing the
                           output directly; > 1 -> the reference's ceil(N/S)-page split
                           partials + log-sum-exp merge; 0 / None -> automatic: the
                           one-pass kernel when batch * kv heads fills the device, else the
                           balanced schedule (equal pages per workgroup) + merge.
        out, workspace   : optional preallocated output (batch, num_q_heads, head_dim) and
                           uint8 scratch of dk_lib.workspace_bytes(...) bytes. Without a
                           workspace the library uses its own (one per device and stream,
                           grown as needed); under graph capture it allocates one for the
                           captured call.
        qk_path, waves_per_group, waves_per_cu, schedule : tuning knobs (0 =
                           defaults; qk_path 1 = MFMA q.k, 2 = VALU q.k, 0 = VALU up to
                           4 q heads per kv head and MFMA (up to 16 heads per wavefront)
                           beyond and for fp8 at D=256; schedule (for
                           split_kv 0) 1 = always balanced, 2 = always one pass)
        max_pages_per_seq: plan hint for split_kv 0 (see plan_hint): the longest
                           sequence's page count, 0 = unknown. Affects speed only.
        sm_scale         : softmax scale; None = 1/sqrt(head_dim) as in the reference
        k_scale, v_scale : fp8 cache only: K = k_scale * fp8 value, V = v_scale * fp8 value
                           (per tensor; None = 1)
        logit_cap        : logit soft-capping: each scaled score s becomes
                           logit_cap * tanh(s / logit_cap) before the softmax (Gemma 2);
                           None or 0 = off
        window           : sliding window: attend to the last `window` tokens of each
                           sequence (the new one and window - 1 before it; Mistral,
                           Gemma); None or 0 = all tokens
        sinks            : attention sinks (gpt-oss): (num_q_heads,) float32 logits on the
                           device; head h's softmax gets one more term e^{sinks[h]} that
                           takes weight and carries no value; None = off

    The argument checks run once per call signature (shapes, strides, dtypes, devices and
    options); later calls with the same signature reuse the validated plan, so a model's
    layers pay only for the pointers and the library call.

    Pages of a multiple of 16 tokens (32, 64, ...; FlashInfer allows any page size, the
    reference only 16) are read in place as 16-token sub-pages: the page table is
    rewritten over them on the device first (one more small kernel, no host sync; see
    sixteen_token_pages to do that once for many layers), and an explicit split_kv then
    partitions sub-pages.

    Returns:
        (batch, num_q_heads, head_dim) tensor, same dtype as q.
    """
    ps = _page_size_of(kv_data)
    if ps is not None and ps != PAGE_SIZE and ps > 0 and ps % PAGE_SIZE == 0:
        return _decode_over_sub_pages(
            q, kv_data, kv_indptr, kv_indices, kv_last_page_len, split_kv, ps,
            dict(out=out, workspace=workspace, qk_path=qk_path,
                 waves_per_group=waves_per_group, waves_per_cu=waves_per_cu,
                 schedule=schedule, max_pages_per_seq=max_pages_per_seq, sm_scale=sm_scale,
                 k_scale=k_scale, v_scale=v_scale, logit_cap=logit_cap, window=window,
                 sinks=sinks))
    kvs = _kv_sig(kv_data) if isinstance(q, torch.Tensor) else None
    key = None
    # scalar options given as tensors are read on every call (a cached plan would keep the
    # value they had when it was made)
    scalars_plain = not any(isinstance(x, torch.Tensor)
                            for x in (sm_scale, k_scale, v_scale, logit_cap, window))
    if kvs is not None and scalars_plain and all(isinstance(t, torch.Tensor) for t in
                                                 (kv_indptr, kv_indices, kv_last_page_len)):
        key = (_tensor_sig(q), kvs, _tensor_sig(kv_indptr), _tensor_sig(kv_indices),
               _tensor_sig(kv_last_page_len),
               None if out is None else _tensor_sig(out),
               None if workspace is None else (workspace.numel() * workspace.element_size(),
                                               workspace.device),
               split_kv, qk_path, waves_per_group, waves_per_cu, schedule, max_pages_per_seq,
               sm_scale, k_scale, v_scale, logit_cap, window,
               None if sinks is None else (sinks.data_ptr(), _tensor_sig(sinks)))
    plan = _PLANS.get(key) if key is not None else None
    if plan is None:
        plan = _CallPlan(q, kv_data, kv_indptr, kv_indices, kv_last_page_len, split_kv, out,
                         workspace, qk_path, waves_per_group, waves_per_cu, schedule,
                         max_pages_per_seq, sm_scale, k_scale, v_scale, logit_cap, window,
                         sinks)
        if key is not None:
            if len(_PLANS) >= _PLANS_MAX:
                _PLANS.clear()
            _PLANS[key] = plan
    return _launch(plan, q, kv_data, kv_indptr, kv_indices, kv_last_page_len, out, workspace)


def _launch(plan, q, kv_data, kv_indptr, kv_indices, kv_last_page_len, out, workspace):
    """One library call with a validated plan: pointers, `out`, the workspace, the stream."""
    lib = dk_lib.load()
    if out is None:
        out = torch.empty(plan.out_shape, dtype=plan.dtype, device=plan.device)
    if plan.batch == 0:
        return out
    if not all(plan.contig):
        kv_indptr, kv_indices, kv_last_page_len = (
            _contig1d(kv_indptr), _contig1d(kv_indices), _contig1d(kv_last_page_len))
    dev = plan.device
    switch = dev.index != torch.cuda.current_device()
    if switch:
        prev = torch.cuda.current_device()
        torch.cuda.set_device(dev)
    try:
        stream = _raw_stream(dev)
        if plan.ws_need and workspace is None:
            if torch.cuda.is_current_stream_capturing():
                # a captured call keeps this allocation (the graph's pool)
                workspace = torch.empty(plan.ws_need, dtype=torch.uint8, device=dev)
            else:
                workspace = _SCRATCH.get(dev, stream, plan.ws_need)
            # pass the bytes this call needs, not the buffer's size (grown by earlier,
            # larger calls), so that what a workspace size can steer (the explicit splits
            # of a sliding window) never depends on history
            ws_ptr, ws_bytes = workspace.data_ptr(), plan.ws_need
        elif plan.ws_need:
            ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
        else:
            ws_ptr, ws_bytes = None, 0
        k, v = (kv_data[0], kv_data[1]) if plan.pair else (kv_data, None)
        tables = (kv_indptr.data_ptr(), kv_indices.data_ptr(), kv_last_page_len.data_ptr(),
                  out.data_ptr(), ws_ptr, ws_bytes)
        if v is None:
            rc = lib.dk_decode_attention_ex(q.data_ptr(), k.data_ptr(), *tables,
                                            *plan.shape[:11], stream)
        else:
            rc = lib.dk_decode_attention_kv(q.data_ptr(), k.data_ptr(), v.data_ptr(), *tables,
                                            *plan.shape[:11], stream)
    finally:
        if switch:
            torch.cuda.set_device(prev)
    dk_lib.check(rc, "decode_attention")
    return out


class DecodePlan:
    """decode_attention split into plan and run, as FlashInfer's decode wrappers are:
    the plan validates the arguments once (shapes, strides, dtypes, devices, options) and
    keeps the library call's argument tuple; run() then passes only the pointers, so a
    model's layers, which share one shape, pay little more than the C ABI call.

        plan = DecodePlan(q, kv_data, kv_indptr, kv_indices, kv_last_page_len, split_kv=0,
                          max_pages_per_seq=hint)
        for layer in layers:
            out = plan.run(q_l, kv_l, kv_indptr, kv_indices, kv_last_page_len, out=out_l)

    run() takes tensors with the planned shapes, strides, dtypes and devices: those of q,
    the cache, the page tables, `out` and the workspace's device are compared with the
    plan's (the strides are what the kernels address memory with; a tensor on another
    device would be addressed as if it were on the planned one). `out` may be None (a
    contiguous one is allocated; then the plan must have been made without one) and
    `workspace` must hold at least the planned bytes (the library checks its size on every
    call). Keyword options are those of decode_attention.

    A cache of pages of a multiple of 16 tokens is planned over its 16-token view. run()
    then takes either that cache with its own page table, which it rewrites over the
    sub-pages on every call (one more small kernel, about 6-8 us per call), or the view
    and rewritten table that sixteen_token_pages returns: a model whose layers share one
    page table rewrites it once per step and passes each layer's view,

        _, ip16, ids16, last16 = sixteen_token_pages(kv_0, kv_indptr, kv_indices, last)
        for layer in layers:
            view, *_ = sixteen_token_pages(kv_l)
            out = plan.run(q_l, view, ip16, ids16, last16, out=out_l)
    """

    def __init__(self, q, kv_data, kv_indptr, kv_indices, kv_last_page_len, split_kv=1, *,
                 out=None, workspace=None, qk_path=0, waves_per_group=0, waves_per_cu=0,
                 schedule=0, max_pages_per_seq=0, sm_scale=None, k_scale=None, v_scale=None,
                 logit_cap=None, window=None, sinks=None):
        # pages of a multiple of 16 tokens: planned (and run) over the 16-token view, with
        # the page table rewritten on the device by every run (sixteen_token_pages)
        ps = _page_size_of(kv_data)
        self._wide = ps is not None and ps != PAGE_SIZE and ps > 0 and ps % PAGE_SIZE == 0
        if self._wide:
            _check(q, kv_data, kv_indptr, kv_indices, kv_last_page_len, wide_pages=True)
            kv_data, kv_indptr, kv_indices, kv_last_page_len = sixteen_token_pages(
                kv_data, kv_indptr, kv_indices, kv_last_page_len)
            max_pages_per_seq *= ps // PAGE_SIZE
        self._plan = _CallPlan(q, kv_data, kv_indptr, kv_indices, kv_last_page_len, split_kv,
                               out, workspace, qk_path, waves_per_group, waves_per_cu,
                               schedule, max_pages_per_seq, sm_scale, k_scale, v_scale,
                               logit_cap, window, sinks)
        self._guard = self._layout(q, kv_data, kv_indptr, kv_indices, kv_last_page_len)
        self._out_strides = None if out is None else out.stride()
        self.workspace_bytes = self._plan.ws_need

    @staticmethod
    def _layout(q, kv_data, kv_indptr, kv_indices, kv_last_page_len):
        kv = (kv_data.shape, kv_data.stride(), kv_data.dtype, kv_data.device) \
            if isinstance(kv_data, torch.Tensor) else \
            tuple((t.shape, t.stride(), t.dtype, t.device) for t in kv_data)
        return (q.shape, q.stride(), q.dtype, q.device, kv, kv_indptr.shape, kv_indptr.stride(),
                kv_indptr.device, kv_indices.shape, kv_indices.stride(), kv_indices.device,
                kv_last_page_len.shape, kv_last_page_len.stride(), kv_last_page_len.device)

    def run(self, q, kv_data, kv_indptr, kv_indices, kv_last_page_len, out=None,
            workspace=None, sinks=None):
        """One call with the plan. A plan made with sinks takes each call's sinks (a
        layer's own; same shape, dtype and device as the planned ones); one made without
        takes none."""
        if getattr(self, "_wide", False) and _page_size_of(kv_data) != PAGE_SIZE:
            # the wide cache and its own table: rewritten here, on every run
            kv_data, kv_indptr, kv_indices, kv_last_page_len = sixteen_token_pages(
                kv_data, kv_indptr, kv_indices, kv_last_page_len)
        if self._layout(q, kv_data, kv_indptr, kv_indices, kv_last_page_len) != self._guard:
            _fail("DecodePlan.run: the tensors differ in shape, strides, dtype or device from "
                  "the planned call")
        if out is None:
            if self._out_strides is not None:
                _fail("DecodePlan.run: the plan was made with an out tensor")
        elif out.stride() != self._out_strides or out.shape != q.shape or \
                out.dtype != q.dtype or out.device != q.device:
            _fail("DecodePlan.run: out differs from the planned call (none, or its shape, "
                  "strides, dtype or device)")
        if workspace is not None and workspace.device != q.device:
            _fail(f"DecodePlan.run: workspace must be on {q.device}, got {workspace.device}")
        if (sinks is None) != (self._plan.sinks is None):
            _fail("DecodePlan.run: pass sinks exactly when the plan was made with them")
        if sinks is not None:
            if not isinstance(sinks, torch.Tensor) or \
                    (sinks.shape, sinks.dtype, sinks.device) != self._plan.sinks or \
                    not sinks.is_contiguous():
                _fail("DecodePlan.run: sinks differ from the planned ones (shape, dtype, "
                      "device) or are not contiguous")
            self._plan.opts.sinks = sinks.data_ptr()
        return _launch(self._plan, q, kv_data, kv_indptr, kv_indices, kv_last_page_len, out,
                       workspace)


def decode_partials(q, kv_data, kv_indptr, kv_indices, kv_last_page_len, split_kv: int,
                    *, qk_path: int = 0, waves_per_group: int = 0,
                    k_scale: Optional[float] = None, v_scale: Optional[float] = None,
                    logit_cap: Optional[float] = None, window: Optional[int] = None):
    """Pass 1 only. Returns (partial_O (B,Hq,S,D), partial_m (B,Hq,S), partial_l (B,Hq,S)),
    fp32, with the semantics of the reference partition kernel
    (src/cuda_/attention_ext.cu:207-349): m is the split's max of q.k*scale (-1e9 when the
    split is empty), l = sum exp(score - m), O = sum exp(score - m) * V (unnormalised)."""
    kv = _check(q, kv_data, kv_indptr, kv_indices, kv_last_page_len)
    if kv.v is not None:
        _fail("decode_partials takes the combined (num_pages, 2, 16, Hkv, D) cache")
    kv_dtype, k_sc, v_sc = _kv_options(kv, k_scale, v_scale)
    lib = dk_lib.load()
    split = choose_split(q, kv_data, kv_indices) if split_kv in (None, 0) else \
        resolve_split(split_kv)
    batch, hq, d = q.shape
    off_o, off_m, off_l, total = dk_lib.partials_layout(batch, hq, d, split)
    ws = torch.empty(total, dtype=torch.uint8, device=q.device)
    strides = _strides(q, kv_data, None)
    opts = dk_lib.options(qk_path, waves_per_group, kv_dtype=kv_dtype, k_scale=k_sc,
                          v_scale=v_sc, logit_cap=_logit_cap(logit_cap),
                          window=_window(window))
    with torch.cuda.device(q.device):
        stream = torch.cuda.current_stream(q.device).cuda_stream
        rc = lib.dk_decode_partials(
            q.data_ptr(), kv_data.data_ptr(), _contig1d(kv_indptr).data_ptr(),
            _contig1d(kv_indices).data_ptr(), _contig1d(kv_last_page_len).data_ptr(),
            ws.data_ptr(), total, batch, hq, kv_data.shape[3], d, kv_data.shape[2],
            kv_data.shape[0], kv_indices.shape[0], _DTYPE_CODE[q.dtype], ctypes.byref(strides),
            split, ctypes.byref(opts), stream)
    dk_lib.check(rc, "decode_partials")
    rows = batch * hq * split
    po = ws[off_o:off_o + rows * d * 4].view(torch.float32).view(batch, hq, split, d)
    pm = ws[off_m:off_m + rows * 4].view(torch.float32).view(batch, hq, split)
    pl = ws[off_l:off_l + rows * 4].view(torch.float32).view(batch, hq, split)
    return po, pm, pl


def merge_partials(partial_o: torch.Tensor, partial_m: torch.Tensor, partial_l: torch.Tensor,
                   dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """Pass 2 only: log-sum-exp merge of fp32 partials (reference decode_attn_reduce_kernel,
    src/cuda_/attention_ext.cu:363-406) into a (B, Hq, D) tensor of `dtype`."""
    if dtype not in _DTYPE_CODE:
        _fail(f"dtype must be fp16 or bf16, got {dtype}")
    if not isinstance(partial_o, torch.Tensor) or partial_o.dim() != 4:
        _fail("partial_o must be a (B, Hq, S, D) tensor")
    batch, hq, split, d = partial_o.shape
    if partial_m.shape != (batch, hq, split) or partial_l.shape != (batch, hq, split):
        _fail("partial_m / partial_l must be (B, Hq, S)")
    if not partial_o.is_cuda:
        _fail("partial_o must be on CUDA (the merge runs on its device)")
    if d not in SUPPORTED_HEAD_DIMS:
        _fail(f"head_dim must be 64, 128, or 256; got {d}")
    lib = dk_lib.load()
    off_o, off_m, off_l, total = dk_lib.partials_layout(batch, hq, d, split)
    ws = torch.empty(total, dtype=torch.uint8, device=partial_o.device)
    rows = batch * hq * split
    ws[off_o:off_o + rows * d * 4].view(torch.float32).copy_(partial_o.reshape(-1))
    ws[off_m:off_m + rows * 4].view(torch.float32).copy_(partial_m.reshape(-1))
    ws[off_l:off_l + rows * 4].view(torch.float32).copy_(partial_l.reshape(-1))
    out = torch.empty((batch, hq, d), dtype=dtype, device=partial_o.device)
    with torch.cuda.device(partial_o.device):
        stream = torch.cuda.current_stream(partial_o.device).cuda_stream
        rc = lib.dk_merge_partials(ws.data_ptr(), total, out.data_ptr(), batch, hq, d,
                                   _DTYPE_CODE[dtype], out.stride(0), out.stride(1), split,
                                   stream)
    dk_lib.check(rc, "merge_partials")
    return out


# ---- the reference's extension-module surface (src/cuda_/attention_ext.cu:613-626)

def decode_attention_naive(q, kv_data, kv_indptr, kv_indices, kv_last_page_len):
    """One pass per (sequence, kv head): the split_kv == 1 route."""
    return decode_attention(q, kv_data, kv_indptr, kv_indices, kv_last_page_len, split_kv=1)


def decode_attention_split_kv(q, kv_data, kv_indptr, kv_indices, kv_last_page_len,
                              split_kv: int = 4):
    """Split-KV partials + log-sum-exp merge."""
    return decode_attention(q, kv_data, kv_indptr, kv_indices, kv_last_page_len,
                            split_kv=split_kv)


_EXT = None


def get_hip_ext():
    """Object with the reference extension's two entry points (cf. get_cuda_ext())."""
    global _EXT
    if _EXT is None:
        dk_lib.load()
        _EXT = SimpleNamespace(decode_attention_naive=decode_attention_naive,
                               decode_attention_split_kv=decode_attention_split_kv)
    return _EXT
