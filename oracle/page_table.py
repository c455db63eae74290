"""CPU restatement of the page-table build from a token-slot map (test infrastructure only).

The CSR page-table format is src/layout.md:27-138 (kv_indptr, kv_indices,
kv_last_page_len; page_size 16). The token-slot map is the one SGLang's ReqToTokenPool
keeps (req_to_token[row][t] = cache slot of token t; the reference adapter,
integration/sglang_backend.py:85-101, receives page tables already built from it). A paged
allocator puts token t at slot 16 * page + t % 16, so page p of a request is
req_to_token[row][16 p] // 16.
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
