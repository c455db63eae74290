"""Writes the golden decode-attention fixtures in this directory.

Each fixture holds seeded inputs (q, kv_data as float16 or as bfloat16 bit patterns,
page tables) and float64 expected outputs computed here by brute force in plain Python
loops (math.exp, no numpy arithmetic), directly from the definition of decode attention
over a FlashInfer-NHD paged cache (reference src/layout.md, src/reference.py:61-96):

    tokens of sequence b: pages kv_indices[kv_indptr[b]:kv_indptr[b+1]], all full except
                          the last, which holds kv_last_page_len[b] tokens
    out[b, h] = sum_t softmax_t(q[b,h] . K[t, h//G] / sqrt(D)) * V[t, h//G]

and, for the split cases, the reference's per-split partials (m = split max of the
scaled scores, l = sum exp(s - m), O = sum exp(s - m) V; empty split: -1e9, 0, 0 —
src/cuda_/attention_ext.cu:243-256,342-348).

This code is deliberately independent of oracle/ so that the fixtures check it.
Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def _bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 -> bfloat16 (nearest-even), returned as uint16 bit patterns."""
    b = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    return b.astype(np.uint16)


def _bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def _tokens(kv, indptr, indices, last, b, page_size):
    """List of (k_vec_per_head, v_vec_per_head) for sequence b, in token order."""
    toks = []
    start, end = int(indptr[b]), int(indptr[b + 1])
    for ptr in range(start, end):
        page = int(indices[ptr])
        n = int(last[b]) if ptr == end - 1 else page_size
        for pos in range(n):
            toks.append((kv[page][0][pos], kv[page][1][pos]))
    return toks


def brute_attention(q, kv, indptr, indices, last, page_size):
    B, Hq, D = len(q), len(q[0]), len(q[0][0])
    Hkv = len(kv[0][0][0])
    G = Hq // Hkv
    scale = 1.0 / math.sqrt(D)
    out = [[[0.0] * D for _ in range(Hq)] for _ in range(B)]
    for b in range(B):
        toks = _tokens(kv, indptr, indices, last, b, page_size)
        for h in range(Hq):
            if not toks:
                continue
            g = h // G
            s = [sum(q[b][h][d] * k[g][d] for d in range(D)) * scale for k, _ in toks]
            mx = max(s)
            p = [math.exp(x - mx) for x in s]
            lsum = sum(p)
            for d in range(D):
                out[b][h][d] = sum(p[t] * toks[t][1][g][d] for t in range(len(toks))) / lsum
    return out


def brute_partials(q, kv, indptr, indices, last, page_size, split):
    B, Hq, D = len(q), len(q[0]), len(q[0][0])
    Hkv = len(kv[0][0][0])
    G = Hq // Hkv
    scale = 1.0 / math.sqrt(D)
    O = np.zeros((B, Hq, split, D))
    m = np.full((B, Hq, split), -1e9)
    l = np.zeros((B, Hq, split))
    for b in range(B):
        start, end = int(indptr[b]), int(indptr[b + 1])
        npages = end - start
        pps = (npages + split - 1) // split
        for s in range(split):
            p0 = s * pps
            p1 = min(p0 + pps, npages)
            toks = []
            for ptr in range(start + p0, start + p1):
                page = int(indices[ptr])
                n = int(last[b]) if ptr == end - 1 else page_size
                for pos in range(n):
                    toks.append((kv[page][0][pos], kv[page][1][pos]))
            if not toks:
                continue
            for h in range(Hq):
                g = h // G
                sc = [sum(q[b][h][d] * k[g][d] for d in range(D)) * scale for k, _ in toks]
                mx = max(sc)
                p = [math.exp(x - mx) for x in sc]
                m[b, h, s] = mx
                l[b, h, s] = sum(p)
                for d in range(D):
                    O[b, h, s, d] = sum(p[t] * toks[t][1][g][d] for t in range(len(toks)))
    return O, m, l


def make_case(name, seed, lens, Hq, Hkv, D, P, pool, dtype, splits=(), qscale=1.0):
    rng = np.random.default_rng(seed)
    B = len(lens)
    pages = [math.ceil(n / P) for n in lens]
    last = [n - (p - 1) * P if p else P for n, p in zip(lens, pages)]
    need = sum(pages)
    pool = max(pool, need)
    ids = rng.permutation(pool)[:need].astype(np.int32)
    indptr = np.zeros(B + 1, np.int32)
    indptr[1:] = np.cumsum(pages)
    q32 = (rng.standard_normal((B, Hq, D)) * qscale).astype(np.float32)
    kv32 = rng.standard_normal((pool, 2, P, Hkv, D)).astype(np.float32)
    if dtype == "f16":
        q_store, kv_store = q32.astype(np.float16), kv32.astype(np.float16)
        qv, kvv = q_store.astype(np.float64), kv_store.astype(np.float64)
    else:
        q_store, kv_store = _bf16_bits(q32), _bf16_bits(kv32)
        qv = _bf16_to_f32(q_store).astype(np.float64)
        kvv = _bf16_to_f32(kv_store).astype(np.float64)
    lastv = np.array(last, np.int32)
    out = brute_attention(qv.tolist(), kvv.tolist(), indptr, ids, lastv, P)
    arrays = dict(q=q_store, kv_data=kv_store, kv_indptr=indptr, kv_indices=ids,
                  kv_last_page_len=lastv, out=np.array(out, np.float64),
                  dtype=np.array(dtype), page_size=np.array(P))
    for S in splits:
        O, m, l = brute_partials(qv.tolist(), kvv.tolist(), indptr, ids, lastv, P, S)
        arrays[f"partial_o_s{S}"] = O
        arrays[f"partial_m_s{S}"] = m
        arrays[f"partial_l_s{S}"] = l
    np.savez_compressed(HERE / f"{name}.npz", **arrays)
    print(f"wrote {name}.npz: lens={lens} Hq={Hq} Hkv={Hkv} D={D} P={P} pool={pool} {dtype}")


def main():
    # tiny shapes for the CPU oracle (any page size / head_dim)
    make_case("tiny_f16", 1, [1, 5, 11, 0], 4, 2, 8, 4, 8, "f16", splits=(2, 3, 8))
    # shapes the HIP kernel takes: page_size 16, head_dim 64 / 128
    make_case("gqa4_d64_f16", 2, [17, 40, 16], 8, 2, 64, 16, 9, "f16", splits=(2, 4))
    make_case("gqa8_d128_bf16", 3, [33, 3], 8, 1, 128, 16, 6, "bf16", splits=(2, 3))
    make_case("mha_d128_f16", 4, [30, 1], 4, 4, 128, 16, 4, "f16", splits=(4,))


if __name__ == "__main__":
    main()
