"""Page tables for the decode path built on the device from a token-slot map.

`build_page_table` turns a serving framework's per-request token-slot map (SGLang's
ReqToTokenPool.req_to_token) into the CSR page table of src/layout.md:27-138 with one
kernel launch (libdk_decode.so: dk_build_page_table), so a decode step needs no host round
trip. Tokens are assumed to sit in 16-token pages: token t of a request at slot
16 * page + t % 16, as a paged allocator with page_size 16 places them.
"""
from __future__ import annotations

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
                     seq_lens_sum: Optional[int] = None):
    """(kv_indptr (B+1,), kv_indices (capacity,), kv_last_page_len (B,)) int32 on the device.

    req_to_token     : (rows, max_tokens) int32 cache slot of each request's tokens
    req_pool_indices : (B,) row of each request (int32 or int64)
    seq_lens         : (B,) tokens per request (int32 or int64)
    capacity         : size of kv_indices; default page_capacity(seq_lens_sum, B), with
                       seq_lens_sum (a host integer) required then. Entries past the
                       table's total are left uninitialised.
    """
    if req_to_token.dtype != torch.int32 or req_to_token.dim() != 2:
        raise DecodeArgumentError("req_to_token must be a 2-D int32 tensor")
    if req_to_token.stride(1) != 1:
        raise DecodeArgumentError("req_to_token rows must be contiguous")
    dev = req_to_token.device
    batch = int(seq_lens.shape[0])
    if req_pool_indices.shape[0] != batch:
        raise DecodeArgumentError("req_pool_indices and seq_lens must have one entry per request")
    if capacity is None:
        if seq_lens_sum is None:
            raise DecodeArgumentError("give capacity or seq_lens_sum (a host integer)")
        capacity = page_capacity(seq_lens_sum, batch)
    rpi = req_pool_indices.to(device=dev, dtype=torch.int32).contiguous()
    lens = seq_lens.to(device=dev, dtype=torch.int32).contiguous()
    kv_indptr = torch.empty(batch + 1, dtype=torch.int32, device=dev)
    kv_indices = torch.empty(max(int(capacity), 1), dtype=torch.int32, device=dev)
    kv_last = torch.empty(batch, dtype=torch.int32, device=dev)
    if batch == 0:
        kv_indptr.zero_()
        return kv_indptr, kv_indices[:0], kv_last
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        rc = dk_lib.load().dk_build_page_table(
            req_to_token.data_ptr(), req_to_token.stride(0), rpi.data_ptr(), lens.data_ptr(),
            batch, PAGE_SIZE, kv_indptr.data_ptr(), kv_indices.data_ptr(), int(capacity),
            kv_last.data_ptr(), stream)
    dk_lib.check(rc, "build_page_table")
    return kv_indptr, kv_indices[:int(capacity)], kv_last
