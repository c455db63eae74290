"""CPU restatement of the page-table build from a token-slot map (test infrastructure only).

The CSR page-table format is src/layout.md:27-138 (kv_indptr, kv_indices,
kv_last_page_len; page_size 16). The token-slot map is the one SGLang's ReqToTokenPool
keeps (req_to_token[row][t] = cache slot of token t; the reference adapter,
integration/sglang_backend.py:85-101, receives page tables already built from it). A paged
allocator puts token t at slot 16 * page + t % 16, so page p of a request is
req_to_token[row][16 p] // 16. `expand_page_table` rewrites a table of larger pages (a
multiple of 16 tokens) over 16-token sub-pages.
"""
from __future__ import annotations

import numpy as np

PAGE = 16


def build_page_table(req_to_token: np.ndarray, req_pool_indices, seq_lens):
    """(kv_indptr (B+1,), kv_indices (sum pages,), kv_last_page_len (B,)) int32."""
    req_pool_indices = np.asarray(req_pool_indices, dtype=np.int64)
    seq_lens = np.asarray(seq_lens, dtype=np.int64)
    indptr = [0]
    indices = []
    last = []
    for row, n_tok in zip(req_pool_indices, seq_lens):
        n_tok = max(int(n_tok), 0)
        n = -(-n_tok // PAGE)
        for p in range(n):
            indices.append(int(req_to_token[row, p * PAGE]) // PAGE)
        indptr.append(indptr[-1] + n)
        last.append(n_tok - (n - 1) * PAGE if n else 0)
    return (np.asarray(indptr, np.int32), np.asarray(indices, np.int32),
            np.asarray(last, np.int32))


def token_slots(kv_indptr, kv_indices, kv_last_page_len, b: int) -> np.ndarray:
    """Cache slots of request b's tokens as the page table describes them."""
    s, e = int(kv_indptr[b]), int(kv_indptr[b + 1])
    out = []
    for i, page in enumerate(kv_indices[s:e]):
        n = int(kv_last_page_len[b]) if i == e - s - 1 else PAGE
        out.extend(int(page) * PAGE + t for t in range(n))
    return np.asarray(out, np.int64)


def expand_page_table(kv_indptr, kv_indices, kv_last_page_len, page_size: int,
                      pages_mult: int, num_pages: int):
    """The table of pages of page_size = 16 s tokens rewritten over 16-token sub-pages
    (the format above, FlashInfer's layout at another page size): sub-page j of page id p
    is p * pages_mult + j; a sequence of n pages whose last holds `last` tokens (clamped
    to [0, page_size]) has (n - 1) s + ceil(last / 16) sub-pages, the last holding the
    remainder (16 when last is a multiple of 16, 0 included). Ids outside [0, num_pages)
    become 2^31 - 1. kv_indptr is clamped to [0, len(kv_indices)] entry by entry, so the
    ranges of an invalid table may overlap; the rewritten table then holds only its first
    capacity = len(kv_indices) * s entries and its offsets saturate there (a valid table
    never reaches it). Returns (indptr, indices, last) int32. No counterpart in the
    reference (whose page_size is 16); pinned by token order: the sub-page table must
    describe the same token rows of the cache as the page table it came from."""
    s = page_size // PAGE
    indptr = np.asarray(kv_indptr, np.int64)
    indices = np.asarray(kv_indices, np.int64)
    lastv = np.asarray(kv_last_page_len, np.int64)
    capacity = len(indices) * s
    out_ptr, out_idx, out_last = [0], [], []
    total = 0
    for b in range(len(indptr) - 1):
        s0 = min(max(int(indptr[b]), 0), len(indices))
        s1 = min(max(int(indptr[b + 1]), s0), len(indices))
        n = s1 - s0
        last = min(max(int(lastv[b]), 0), page_size)
        m = (n - 1) * s + -(-last // PAGE) if n > 0 else 0
        for t in range(m):
            if len(out_idx) >= capacity:
                break
            pid = int(indices[s0 + t // s])
            out_idx.append(pid * pages_mult + t % s if 0 <= pid < num_pages else 2**31 - 1)
        total += m
        out_ptr.append(min(total, capacity))
        out_last.append(0 if m == 0 else (PAGE if last % PAGE == 0 else last % PAGE))
    return (np.asarray(out_ptr, np.int32), np.asarray(out_idx, np.int32),
            np.asarray(out_last, np.int32))
