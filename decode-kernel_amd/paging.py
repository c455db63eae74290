"""Page tables and cache writes around the decode path, on the device.

`build_page_table` turns a serving framework's per-request token-slot map (SGLang's
ReqToTokenPool.req_to_token) into the CSR page table of src/layout.md:27-138 with one
kernel launch (libdk_decode.so: dk_build_page_table), so a decode step needs no host round
trip. Tokens are assumed to sit in 16-token pages: token t of a request at slot
16 * page + t % 16, as a paged allocator with page_size 16 places them (or one with a
page_size that is a multiple of 16: each of its pages is a run of aligned 16-slot pages).
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional

import torch

import dk_lib
from dk_lib import DecodeArgumentError

PAGE_SIZE = 16


def page_capacity(seq_lens_sum: int, batch: int) -> int:
    """kv_indices entries that always suffice: sum(ceil(len / 16)) <= (sum + 15 B) / 16."""
    return (int(seq_lens_sum) + (PAGE_SIZE - 1) * int(batch)) // PAGE_SIZE


def build_page_table(req_to_token: torch.Tensor, req_pool_indices: torch.Tensor,
                     seq_lens: torch.Tensor, capacity: Optional[int] = None,
                     seq_lens_sum: Optional[int] = None, out=None):
    """(kv_indptr (B+1,), kv_indices (capacity,), kv_last_page_len (B,)) int32 on the device.

    req_to_token     : (rows, max_tokens) int32 cache slot of each request's tokens
    req_pool_indices : (B,) row of each request (int32 or int64)
    seq_lens         : (B,) tokens per request (int32 or int64)
    capacity         : size of kv_indices; default page_capacity(seq_lens_sum, B), with
                       seq_lens_sum (a host integer) required then. Entries past the
                       table's total are left uninitialised.
    out              : optional persistent (kv_indptr, kv_indices, kv_last_page_len)
                       buffers to fill in place (at least B + 1, capacity and B entries),
                       e.g. for tables a captured HIP graph reads; capacity defaults to
                       the kv_indices buffer's size then
    """
    if req_to_token.dtype != torch.int32 or req_to_token.dim() != 2:
        raise DecodeArgumentError("req_to_token must be a 2-D int32 tensor")
    if req_to_token.stride(1) != 1:
        raise DecodeArgumentError("req_to_token rows must be contiguous")
    dev = req_to_token.device
    batch = int(seq_lens.shape[0])
    if req_pool_indices.shape[0] != batch:
        raise DecodeArgumentError("req_pool_indices and seq_lens must have one entry per request")
    if out is not None:
        kv_indptr, kv_indices, kv_last = out
        if capacity is None:
            capacity = kv_indices.numel()
        if (kv_indptr.numel() < batch + 1 or kv_indices.numel() < capacity or
                kv_last.numel() < batch or
                any(t.dtype != torch.int32 or t.device != dev or not t.is_contiguous()
                    for t in out)):
            raise DecodeArgumentError("out buffers must be contiguous int32 on the table's "
                                      "device, with B + 1, capacity and B entries")
    elif capacity is None:
        if seq_lens_sum is None:
            raise DecodeArgumentError("give capacity or seq_lens_sum (a host integer)")
        capacity = page_capacity(seq_lens_sum, batch)
    rpi = req_pool_indices.to(device=dev, dtype=torch.int32).contiguous()
    lens = seq_lens.to(device=dev, dtype=torch.int32).contiguous()
    if out is None:
        kv_indptr = torch.empty(batch + 1, dtype=torch.int32, device=dev)
        kv_indices = torch.empty(max(int(capacity), 1), dtype=torch.int32, device=dev)
        kv_last = torch.empty(batch, dtype=torch.int32, device=dev)
    if batch == 0:
        kv_indptr[:1].zero_()
        return kv_indptr[:1], kv_indices[:0], kv_last[:0]
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        rc = dk_lib.load().dk_build_page_table(
            req_to_token.data_ptr(), req_to_token.stride(0), rpi.data_ptr(), lens.data_ptr(),
            batch, PAGE_SIZE, kv_indptr.data_ptr(), kv_indices.data_ptr(), int(capacity),
            kv_last.data_ptr(), stream)
    dk_lib.check(rc, "build_page_table")
    return kv_indptr[:batch + 1], kv_indices[:int(capacity)], kv_last[:batch]


def expand_page_table(kv_indptr: torch.Tensor, kv_indices: torch.Tensor,
                      kv_last_page_len: torch.Tensor, page_size: int, pages_mult: int,
                      num_pages: int):
    """The page table of a cache with pages of page_size = 16 * s tokens, rewritten over
    its 16-token sub-pages (dk_expand_page_table): sub-page j of page p is id
    p * pages_mult + j. Returns (kv_indptr (B+1,), kv_indices (len(kv_indices) * s,),
    kv_last_page_len (B,)) int32 on the same device; entries past the new table's total
    are left uninitialised. No host synchronisation."""
    for name, t in (("kv_indptr", kv_indptr), ("kv_indices", kv_indices),
                    ("kv_last_page_len", kv_last_page_len)):
        if not isinstance(t, torch.Tensor) or t.dtype != torch.int32 or t.dim() != 1 or \
                not t.is_contiguous():
            raise DecodeArgumentError(f"{name} must be a contiguous 1-D int32 tensor")
    if page_size <= 0 or page_size % PAGE_SIZE:
        raise DecodeArgumentError(f"page_size must be a positive multiple of 16, got {page_size}")
    if kv_indptr.shape[0] < 1 or kv_last_page_len.shape[0] != kv_indptr.shape[0] - 1:
        raise DecodeArgumentError(
            f"kv_last_page_len must have one entry per sequence (len(kv_indptr) - 1 = "
            f"{kv_indptr.shape[0] - 1}); got {kv_last_page_len.shape[0]}")
    dev = kv_indptr.device
    # the kernel reads all three tables on one GPU: host memory there would fault it
    if dev.type != "cuda" or kv_indices.device != dev or kv_last_page_len.device != dev:
        raise DecodeArgumentError(
            f"kv_indptr, kv_indices and kv_last_page_len must be on one GPU; got "
            f"{kv_indptr.device}, {kv_indices.device}, {kv_last_page_len.device}")
    batch = int(kv_indptr.shape[0]) - 1
    sub = page_size // PAGE_SIZE
    capacity = int(kv_indices.shape[0]) * sub
    out_indptr = torch.empty(batch + 1, dtype=torch.int32, device=dev)
    out_indices = torch.empty(max(capacity, 1), dtype=torch.int32, device=dev)
    out_last = torch.empty(max(batch, 0), dtype=torch.int32, device=dev)
    if batch <= 0:
        out_indptr.zero_()
        return out_indptr, out_indices[:0], out_last
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        rc = dk_lib.load().dk_expand_page_table(
            kv_indptr.data_ptr(), kv_indices.data_ptr(), kv_last_page_len.data_ptr(), batch,
            int(page_size), int(pages_mult), int(num_pages), int(kv_indices.shape[0]),
            out_indptr.data_ptr(), out_indices.data_ptr(), capacity, out_last.data_ptr(),
            stream)
    dk_lib.check(rc, "expand_page_table")
    return out_indptr, out_indices[:capacity], out_last


def rope_inv_freq(head_dim: int, theta: float = 10000.0, device="cuda") -> torch.Tensor:
    """Plain rotary frequencies theta^(-2i/head_dim), i < head_dim/2, fp32. Frequency
    scalings (Llama 3's, YaRN, ...) produce their own inv_freq and pass it instead."""
    i = torch.arange(0, head_dim, 2, dtype=torch.float64)
    return (1.0 / (theta ** (i / head_dim))).to(device=device, dtype=torch.float32)


def append_kv(q: Optional[torch.Tensor], k_new: torch.Tensor, v_new: torch.Tensor, kv_data,
              kv_indptr: torch.Tensor, kv_indices: torch.Tensor, kv_last_page_len: torch.Tensor,
              inv_freq: Optional[torch.Tensor] = None, positions: Optional[torch.Tensor] = None,
              rope_style: int = 0, k_scale: Optional[float] = None,
              v_scale: Optional[float] = None) -> None:
    """Write each sequence's new token into the paged cache (dk_append_kv), in place.

    The token's slot is the last one the page table describes (grow the table first).
    q (batch, num_q_heads, head_dim) or None is rotated in place; k_new / v_new
    (batch, num_kv_heads, head_dim) are the token's K (rotated on the way in) and V rows;
    kv_data is the combined cache or a (k_cache, v_cache) pair as for decode_attention.
    inv_freq (head_dim/2,) fp32 on the device, or None for no rotation; positions (batch,)
    int32, or None for each token's index in its sequence; rope_style 0 = rotate-half
    pairs (i, i + D/2) (Llama), 1 = interleaved pairs (2i, 2i + 1).
    A torch.float8_e4m3fn cache (q, k_new, v_new fp16 or bf16) stores each element as
    RNE(clamp(x / scale, -448, 448)) with k_scale for K and v_scale for V (None = 1), the
    scales decode_attention then takes.
    """
    import attention                     # local: attention imports nothing from here
    kv = attention._kv_layout(kv_data)
    batch, hkv, d = k_new.shape
    kv8 = kv.dtype == attention.KV_FP8
    act = k_new.dtype if kv8 else kv.dtype          # type of q, k_new and v_new
    if kv8 and act not in (torch.float16, torch.bfloat16):
        raise DecodeArgumentError("over an fp8 cache k_new and v_new must be fp16 or bf16")
    if v_new.shape != k_new.shape or k_new.dtype != act or v_new.dtype != act:
        raise DecodeArgumentError("k_new and v_new must be (batch, num_kv_heads, head_dim) in "
                                  "the cache's dtype (fp16 / bf16 over an fp8 cache)")
    scales = []
    for name, x in (("k_scale", k_scale), ("v_scale", v_scale)):
        if not kv8:
            if x not in (None, 1.0):
                raise DecodeArgumentError(f"{name} applies to a torch.float8_e4m3fn cache only")
            continue
        x = 1.0 if x is None else float(x)
        if not math.isfinite(x) or x <= 0.0:
            raise DecodeArgumentError(f"{name} must be finite and > 0, got {x}")
        scales.append(x)
    if v_new.stride() != k_new.stride() or k_new.stride(2) != 1:
        raise DecodeArgumentError("k_new and v_new need equal strides and a unit head_dim stride")
    if hkv != kv.hkv or d != kv.d or kv.page_size != PAGE_SIZE or kv.d_stride != 1:
        raise DecodeArgumentError("k_new does not match the cache's heads / head_dim")
    if q is not None and (q.dim() != 3 or q.shape[0] != batch or q.shape[2] != d or
                          q.dtype != act or q.stride(2) != 1):
        raise DecodeArgumentError("q must be (batch, num_q_heads, head_dim) in k_new's dtype")
    if inv_freq is not None and (inv_freq.dtype != torch.float32 or inv_freq.numel() != d // 2
                                 or not inv_freq.is_contiguous()):
        raise DecodeArgumentError("inv_freq must be a contiguous fp32 tensor of head_dim/2")
    if positions is not None:
        positions = positions.to(dtype=torch.int32).contiguous()
    s = dk_lib.DkStrides()
    if q is not None:
        s.q_b, s.q_h = q.stride(0), q.stride(1)
    s.kv_p, s.kv_r, s.kv_s, s.kv_h = kv.strides
    code = dk_lib.DK_F16 if act == torch.float16 else dk_lib.DK_BF16
    ptr = lambda t: t.data_ptr() if t is not None else None  # noqa: E731
    lib = dk_lib.load()
    with torch.cuda.device(k_new.device):
        stream = torch.cuda.current_stream(k_new.device).cuda_stream
        args = (ptr(q), k_new.data_ptr(), v_new.data_ptr(), k_new.stride(0), k_new.stride(1),
                kv.k.data_ptr(), ptr(kv.v), kv_indptr.data_ptr(), kv_indices.data_ptr(),
                kv_last_page_len.data_ptr(), ptr(positions), ptr(inv_freq), rope_style, batch,
                q.shape[1] if q is not None else 1, hkv, d, PAGE_SIZE, kv.num_pages,
                kv_indices.shape[0], code)
        if kv8:
            rc = lib.dk_append_kv_fp8(*args, *scales, ctypes.byref(s), stream)
        else:
            rc = lib.dk_append_kv(*args, ctypes.byref(s), stream)
    dk_lib.check(rc, "append_kv")
