"""CPU restatement of the reference's two-pass split-KV algorithm.

TEST INFRASTRUCTURE ONLY (see oracle/reference.py's header for who may import it).

  * partition        page range of each split: ceil(N/S) contiguous pages, the last
                     split short or empty (src/cuda_/attention_ext.cu:243-252)
  * split_partials   pass 1's fp32 partials per (sequence, q head, split): m = max of
                     q.k*scale over the split's valid tokens, l = sum exp(score - m),
                     O = sum exp(score - m) * V, unnormalised; an empty split gives
                     m = -1e9, l = 0, O = 0 (attention_ext.cu:254-256,342-348;
                     contract src/layout.md:142-167)
  * merge_partials   pass 2: M = max_s m_s (starting from -1e9), w_s = exp(m_s - M),
                     out = sum w_s O_s / sum w_s l_s (attention_ext.cu:363-406); a row whose
                     splits are all empty gives 0 (the reference divides 0 by 0 there)

Computed in float64 so that it can stand as the exact value the fp32 kernels round.
Pinned in tests/test_oracle.py by the primer's two-split example
(writeup/cuda_primer.md:505-540), by brute-force fixtures, and by the identity
merge(split_partials(S)) == reference_attention_paged for every S.
"""
from __future__ import annotations

import math

import numpy as np

from oracle.reference import _sequence_kv

EMPTY_M = -1e9


def partition(num_pages: int, split_kv: int):
    """[(start, end)] page ranges of the splits of one sequence."""
    pps = (num_pages + split_kv - 1) // split_kv if num_pages > 0 else 0
    out = []
    for s in range(split_kv):
        start = min(s * pps, num_pages)
        out.append((start, min(start + pps, num_pages)))
    return out


def split_partials(Q, kv_data, kv_indptr, kv_indices, kv_last_page_len, split_kv: int,
                   scale=None):
    """(O (B,Hq,S,D), m (B,Hq,S), l (B,Hq,S)) float64 partials of pass 1.

    `scale` defaults to 1/sqrt(head_dim) (attention_ext.cu:515); the argument exists so
    that tests can plant a wrong scale and show that the checks catch it."""
    Q = np.asarray(Q, dtype=np.float64)
    kv = np.asarray(kv_data)
    B, Hq, D = Q.shape
    P, Hkv = kv.shape[2], kv.shape[3]
    G = Hq // Hkv
    scale = D ** -0.5 if scale is None else scale
    O = np.zeros((B, Hq, split_kv, D))
    m = np.full((B, Hq, split_kv), EMPTY_M)
    l = np.zeros((B, Hq, split_kv))
    for b in range(B):
        k, v = _sequence_kv(kv, kv_indptr, kv_indices, kv_last_page_len, b)
        k = k.astype(np.float64)
        v = v.astype(np.float64)
        npages = int(kv_indptr[b + 1]) - int(kv_indptr[b])
        for s, (p0, p1) in enumerate(partition(npages, split_kv)):
            t0, t1 = p0 * P, min(p1 * P, len(k))
            if t1 <= t0:
                continue
            for h in range(Hq):
                kvh = h // G
                sc = (k[t0:t1, kvh] @ Q[b, h]) * scale
                mx = sc.max()
                p = np.exp(sc - mx)
                m[b, h, s] = mx
                l[b, h, s] = p.sum()
                O[b, h, s] = p @ v[t0:t1, kvh]
    return O, m, l


def merge_partials(O, m, l) -> np.ndarray:
    """(B, Hq, D) float64 result of the log-sum-exp merge."""
    O = np.asarray(O, dtype=np.float64)
    m = np.asarray(m, dtype=np.float64)
    l = np.asarray(l, dtype=np.float64)
    M = np.maximum(m.max(axis=2, initial=EMPTY_M), EMPTY_M)
    w = np.exp(m - M[..., None])
    L = (w * l).sum(axis=2)
    acc = (w[..., None] * O).sum(axis=2)
    out = np.zeros_like(acc)
    nz = L > 0
    out[nz] = acc[nz] / L[nz][:, None]
    return out


def split_kv_attention(Q, kv_data, kv_indptr, kv_indices, kv_last_page_len,
                       split_kv: int) -> np.ndarray:
    """merge_partials(split_partials(...)): the two-pass result."""
    return merge_partials(*split_partials(Q, kv_data, kv_indptr, kv_indices,
                                          kv_last_page_len, split_kv))

