"""FlashInfer-NHD paged KV layout: validation, block tables and seeded synthetic inputs.

Mirrors the reference's src/layout.py (PagedKVLayout.validate :11-32,
build_block_table :35-69, synthesize :72-126) and adds generators for the
benchmark configurations: permuted page tables, ragged batches drawn from a shuffled
free list, and q scaling.

kv_data is (num_pages, 2, page_size, num_kv_heads, head_dim): [:, 0] K, [:, 1] V.
Sequence b owns pages kv_indices[kv_indptr[b]:kv_indptr[b+1]]; all of them hold
page_size tokens except the last, which holds kv_last_page_len[b] (src/layout.md).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Sequence, Tuple, Union

import torch


class LayoutError(ValueError, AssertionError):
    """Layout invariant violated. A ValueError (as the reference's docstring says,
    src/layout.py:18) that is also an AssertionError (as its asserts raise)."""


@dataclass
class PagedKVLayout:
    page_size: int
    head_dim: int
    num_kv_heads: int
    dtype: torch.dtype = torch.float16

    def validate(self, kv_data, kv_indptr, kv_indices, kv_last_page_len) -> None:
        """Raise LayoutError on any invariant violation (src/layout.md:171-178)."""
        def need(cond, msg):
            if not cond:
                raise LayoutError(msg)
        need(kv_data.dim() == 5, "kv_data must be 5-D")
        need(kv_data.shape[1] == 2, "kv_data dim-1 must be 2 (K/V)")
        need(kv_data.shape[2] == self.page_size, "kv_data page_size mismatch")
        need(kv_data.shape[3] == self.num_kv_heads, "kv_data num_kv_heads mismatch")
        need(kv_data.shape[4] == self.head_dim, "kv_data head_dim mismatch")
        need(kv_data.dtype == self.dtype, f"kv_data dtype {kv_data.dtype} != {self.dtype}")
        need(int(kv_indptr[-1]) == kv_indices.shape[0],
             f"kv_indptr[-1]={int(kv_indptr[-1])} != kv_indices.shape[0]={kv_indices.shape[0]}")
        need(bool((kv_indptr[1:] >= kv_indptr[:-1]).all()), "kv_indptr must be non-decreasing")
        need(bool((kv_last_page_len > 0).all()), "kv_last_page_len must be > 0")
        need(bool((kv_last_page_len <= self.page_size).all()),
             "kv_last_page_len must be <= page_size")
        if kv_indices.numel():
            need(int(kv_indices.min()) >= 0 and int(kv_indices.max()) < kv_data.shape[0],
                 "kv_indices out of range of kv_data pages")


def build_block_table(batch: int, context_length: int, page_size: int,
                      device: Union[str, torch.device] = "cuda"
                      ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """kv_indptr, kv_indices, kv_last_page_len for a uniform context
    (src/layout.py:35-69): sequence b owns physical pages [b*K_p, (b+1)*K_p)."""
    pages_per_seq = math.ceil(context_length / page_size)
    last_len = context_length - (pages_per_seq - 1) * page_size
    if last_len == 0:
        last_len = page_size
    kv_indptr = torch.arange(0, batch + 1, dtype=torch.int32, device=device) * pages_per_seq
    kv_indices = torch.arange(0, batch * pages_per_seq, dtype=torch.int32, device=device)
    kv_last_page_len = torch.full((batch,), last_len, dtype=torch.int32, device=device)
    return kv_indptr, kv_indices, kv_last_page_len


def synthesize(batch: int, context_length: int, num_q_heads: int, num_kv_heads: int,
               head_dim: int, page_size: int = 16, dtype: torch.dtype = torch.float16,
               device: Union[str, torch.device] = "cuda", seed: int = 42):
    """Random q and NHD paged K/V for a uniform context (src/layout.py:72-126).

    One seeded generator on `device`; q is drawn first, then kv_data, both N(0, 1) in
    `dtype`. Returns (q, kv_data, kv_indptr, kv_indices, kv_last_page_len, layout).
    """
    if num_q_heads % num_kv_heads != 0:
        raise ValueError(f"num_q_heads ({num_q_heads}) must be divisible by "
                         f"num_kv_heads ({num_kv_heads})")
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    q = torch.randn(batch, num_q_heads, head_dim, dtype=dtype, device=device, generator=gen)
    kv_indptr, kv_indices, kv_last_page_len = build_block_table(batch, context_length,
                                                                page_size, device)
    total_pages = int(kv_indices.shape[0])
    kv_data = torch.randn(total_pages, 2, page_size, num_kv_heads, head_dim, dtype=dtype,
                          device=device, generator=gen)
    layout = PagedKVLayout(page_size=page_size, head_dim=head_dim, num_kv_heads=num_kv_heads,
                           dtype=dtype)
    return q, kv_data, kv_indptr, kv_indices, kv_last_page_len, layout


def synthesize_paged(batch: int, context_lengths: Union[int, Sequence[int]], num_q_heads: int,
                     num_kv_heads: int, head_dim: int, page_size: int = 16,
                     dtype: torch.dtype = torch.float16,
                     device: Union[str, torch.device] = "cuda", seed: int = 0,
                     page_table: str = "contiguous", pool_pages: int = 0,
                     q_scale: float = 1.0):
    """Synthetic decode inputs with a chosen page-table shape.

    context_lengths : one length for all sequences, or one per sequence (ragged; a length
                      of 0 gives a sequence with no pages)
    page_table      : "contiguous" (identity, as build_block_table), "permuted" (a seeded
                      random permutation of the pool) or "freelist" (pages drawn without
                      replacement from a shuffled free list of `pool_pages` pages)
    pool_pages      : page-pool size (>= pages needed; 0 = exactly the pages needed)
    q_scale         : multiplier applied to q after drawing it (e.g. 1/sqrt(d))

    Page indices and lengths are computed on the CPU with a seeded torch generator, so
    the page table is the same on every device. kv_data of every pool page is N(0, 1).
    Returns (q, kv_data, kv_indptr, kv_indices, kv_last_page_len, layout).
    """
    if num_q_heads % num_kv_heads != 0:
        raise ValueError(f"num_q_heads ({num_q_heads}) must be divisible by "
                         f"num_kv_heads ({num_kv_heads})")
    if isinstance(context_lengths, int):
        lens = [context_lengths] * batch
    else:
        lens = [int(x) for x in context_lengths]
        if len(lens) != batch:
            raise ValueError("need one context length per sequence")
    pages = [math.ceil(n / page_size) for n in lens]
    last = [(n - (p - 1) * page_size) if p > 0 else page_size for n, p in zip(lens, pages)]
    needed = sum(pages)
    pool = max(pool_pages, needed, 1)
    cpu = torch.Generator(device="cpu")
    cpu.manual_seed(seed)
    if page_table == "contiguous":
        ids = torch.arange(needed, dtype=torch.int32)
    elif page_table in ("permuted", "freelist"):
        ids = torch.randperm(pool, generator=cpu)[:needed].to(torch.int32)
    else:
        raise ValueError(f"unknown page_table {page_table!r}")
    indptr = torch.zeros(batch + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(torch.tensor(pages, dtype=torch.int64), 0).to(torch.int32)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    q = torch.randn(batch, num_q_heads, head_dim, dtype=dtype, device=device, generator=gen)
    if q_scale != 1.0:
        q = (q.float() * q_scale).to(dtype)
    kv_data = torch.randn(pool, 2, page_size, num_kv_heads, head_dim, dtype=dtype,
                          device=device, generator=gen)
    layout = PagedKVLayout(page_size=page_size, head_dim=head_dim, num_kv_heads=num_kv_heads,
                           dtype=dtype)
    return (q, kv_data, indptr.to(device), ids.to(device),
            torch.tensor(last, dtype=torch.int32, device=device), layout)


def ragged_lengths(batch: int, lo: int, hi: int, seed: int = 0):
    """Per-sequence context lengths uniform in [lo, hi] (seeded, CPU)."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return torch.randint(lo, hi + 1, (batch,), generator=g).tolist()


def seq_lens(kv_indptr: torch.Tensor, kv_last_page_len: torch.Tensor, page_size: int = 16):
    """Tokens per sequence: (pages - 1) * page_size + last_page_len (0 for no pages)."""
    n = (kv_indptr[1:] - kv_indptr[:-1]).long()
    lens = (n - 1) * page_size + kv_last_page_len.long()
    return torch.where(n > 0, lens, torch.zeros_like(lens))


def attention_bytes(batch: int, context_length, num_q_heads: int, num_kv_heads: int,
                    head_dim: int, elem_bytes: int = 2, page_size: int = 16,
                    kv_elem_bytes: int = 0) -> int:
    """Algorithmic HBM bytes of one decode call: K and V of the valid tokens, q read and
    the output written (the reference's bytes model, bench/microbench_cuda.py:114-121),
    plus the int32 page tables. `context_length` is an int or a per-sequence list;
    kv_elem_bytes is the cache's element size when it differs from q's (1 for fp8)."""
    lens = [context_length] * batch if isinstance(context_length, int) else list(context_length)
    kv = sum(lens) * num_kv_heads * head_dim * (kv_elem_bytes or elem_bytes) * 2
    qo = 2 * batch * num_q_heads * head_dim * elem_bytes
    tables = 4 * (batch + 1) + 4 * sum(math.ceil(n / page_size) for n in lens) + 4 * batch
    return kv + qo + tables
