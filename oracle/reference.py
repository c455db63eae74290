"""CPU fp32 restatement of the reference oracle `reference_attention_paged`.

TEST INFRASTRUCTURE ONLY. This module is the checker for the HIP decode path: it may be
imported by tests/, by __graft_entry__.smoke() and by bench.py's CPU-baseline leg, and
never by the product code under decode-kernel_amd/.

It restates /root/reference src/reference.py in numpy:
  * gather_paged_to_dense   follows src/reference.py:9-58
  * reference_attention     follows src/reference.py:61-96 (GQA by grouping q heads,
                            which equals repeat_interleave: kv_head = q_head // G)
  * reference_attention_paged follows src/reference.py:99-108
with one deliberate difference in the default: each sequence attends over exactly its
own tokens. The reference zero-pads shorter sequences to the batch maximum and then
softmaxes over the padding with no mask (src/reference.py:40-43,91-94); that equals the
masked result whenever all sequences have the same length and is wrong for ragged
batches. `literal=True` reproduces the padded form.

Pinned by tests/test_oracle.py against: the hand-worked example of
writeup/cuda_primer.md:31-43,505-540; closed forms (ctx=1, constant V, equal K);
torch.nn.functional.scaled_dot_product_attention(enable_gqa=True) in float64;
brute-force float64 golden fixtures (tests/golden/); the soft-capped form against
transformers' Gemma 2 eager attention (softcap) in float64; the attention-sink form
against transformers' gpt-oss eager attention (sinks) in float64.

Inputs are numpy arrays: q (B, Hq, D) and kv_data (N_p, 2, P, Hkv, D) as float16 /
float32 (bfloat16 callers pass float32 upcasts — exact), and int32 page tables.
"""
from __future__ import annotations

import numpy as np


def seq_lens_of(kv_indptr, kv_last_page_len, page_size: int) -> np.ndarray:
    """(n_pages - 1) * P + last_len, floored at 0 (src/reference.py:31-38)."""
    indptr = np.asarray(kv_indptr, dtype=np.int64)
    last = np.asarray(kv_last_page_len, dtype=np.int64)
    n = indptr[1:] - indptr[:-1]
    return np.maximum(0, (n - 1) * page_size + last)


def _sequence_kv(kv_data, kv_indptr, kv_indices, kv_last_page_len, b: int):
    """K, V (len_b, Hkv, D) float32 of sequence b, in token order."""
    kv = np.asarray(kv_data)
    page_size = kv.shape[2]
    start, end = int(kv_indptr[b]), int(kv_indptr[b + 1])
    n = max(0, (end - start - 1) * page_size + int(kv_last_page_len[b])) if end > start else 0
    if n == 0:
        shape = (0,) + kv.shape[3:]
        return np.zeros(shape, np.float32), np.zeros(shape, np.float32)
    pages = np.asarray(kv_indices[start:end], dtype=np.int64)
    blk = kv[pages]                                   # (n_pages, 2, P, Hkv, D)
    k = blk[:, 0].reshape((-1,) + kv.shape[3:])[:n]   # full pages, then the last page's prefix
    v = blk[:, 1].reshape((-1,) + kv.shape[3:])[:n]
    return k.astype(np.float32), v.astype(np.float32)


def gather_paged_to_dense(kv_data, kv_indptr, kv_indices, kv_last_page_len):
    """Dense float32 K, V (B, max_len, Hkv, D), zero-padded past each sequence's length
    (src/reference.py:9-58)."""
    kv = np.asarray(kv_data)
    batch = len(kv_indptr) - 1
    lens = seq_lens_of(kv_indptr, kv_last_page_len, kv.shape[2])
    max_len = int(lens.max()) if batch else 0
    K = np.zeros((batch, max_len) + kv.shape[3:], np.float32)
    V = np.zeros_like(K)
    for b in range(batch):
        k, v = _sequence_kv(kv, kv_indptr, kv_indices, kv_last_page_len, b)
        K[b, :len(k)] = k
        V[b, :len(v)] = v
    return K, V


def _softmax_attend(qs: np.ndarray, k: np.ndarray, v: np.ndarray,
                    logit_cap=None, sinks=None) -> np.ndarray:
    """qs (Hkv, G, D) already scaled; k, v (S, Hkv, D) -> (Hkv, G, D), fp32 throughout.
    logit_cap: scores s become cap * tanh(s / cap) before the softmax (an extension).
    sinks (Hkv, G): one more logit per q head in the softmax, with no value (an extension,
    gpt-oss's attention sinks): its weight only enlarges the denominator."""
    if k.shape[0] == 0:
        return np.zeros(qs.shape, np.float32)
    kt = np.ascontiguousarray(k.transpose(1, 2, 0))            # (Hkv, D, S)
    scores = np.matmul(qs, kt)                                 # (Hkv, G, S)
    if logit_cap:
        cap = np.float32(logit_cap)
        scores = (cap * np.tanh(scores / cap)).astype(np.float32)
    top = scores.max(axis=-1, keepdims=True)
    if sinks is not None:
        sk = np.asarray(sinks, np.float32)[..., None]          # (Hkv, G, 1)
        top = np.maximum(top, sk)
    w = np.exp(scores - top, dtype=np.float32)
    den = w.sum(axis=-1, keepdims=True, dtype=np.float32)
    if sinks is not None:
        den = den + np.exp(sk - top, dtype=np.float32)
    w /= den
    return np.matmul(w, np.ascontiguousarray(v.transpose(1, 0, 2)))  # (Hkv, G, D)


def reference_attention(Q, K, V, seq_lens=None, sm_scale=None, logit_cap=None,
                        sinks=None) -> np.ndarray:
    """fp32 decode attention with GQA (src/reference.py:61-96).

    Q (B, Hq, D); K, V (B, S, Hkv, D). With `seq_lens`, sequence b attends over its first
    seq_lens[b] positions only (a length of 0 gives zeros); without, over all S positions
    (the reference's unmasked form). Returns (B, Hq, D) float32. sm_scale, logit_cap and
    sinks are the extensions of reference_attention_paged.
    """
    Q = np.asarray(Q, dtype=np.float32)
    B, Hq, D = Q.shape
    Hkv = K.shape[2]
    G = Hq // Hkv
    scale = np.float32(D ** -0.5 if sm_scale is None else sm_scale)
    out = np.zeros((B, Hq, D), np.float32)
    for b in range(B):
        n = K.shape[1] if seq_lens is None else int(seq_lens[b])
        qs = (Q[b] * scale).reshape(Hkv, G, D)                 # q head h -> kv head h // G
        sk = None if sinks is None else np.asarray(sinks, np.float32).reshape(Hkv, G)
        out[b] = _softmax_attend(qs, np.asarray(K[b, :n], np.float32),
                                 np.asarray(V[b, :n], np.float32), logit_cap,
                                 sk).reshape(Hq, D)
    return out


def reference_attention_paged(Q, kv_data, kv_indptr, kv_indices, kv_last_page_len,
                              literal: bool = False, batch_subset=None, sm_scale=None,
                              logit_cap=None, window=None, sinks=None) -> np.ndarray:
    """Paged decode attention (src/reference.py:99-108), per-sequence masked by default.

    literal=True gathers to the zero-padded dense form and attends over all positions,
    exactly as the reference does. batch_subset restricts the work to some sequences
    (the other rows of the result are NaN); it is only meaningful with literal=False.
    sm_scale (default 1/sqrt(D), the reference's), logit_cap (scores s -> cap *
    tanh(s / cap) before the softmax, Gemma 2 style), window (attend to each
    sequence's last `window` tokens only) and sinks ((Hq,) logits, one more softmax term
    per q head with no value, gpt-oss style) are extensions beyond the reference, for the
    masked form only.
    """
    Q = np.asarray(Q, dtype=np.float32)
    if literal:
        K, V = gather_paged_to_dense(kv_data, kv_indptr, kv_indices, kv_last_page_len)
        return reference_attention(Q, K, V)
    B, Hq, D = Q.shape
    kv = np.asarray(kv_data)
    Hkv = kv.shape[3]
    G = Hq // Hkv
    scale = np.float32(D ** -0.5 if sm_scale is None else sm_scale)
    out = np.full((B, Hq, D), np.nan, np.float32)
    for b in (range(B) if batch_subset is None else batch_subset):
        k, v = _sequence_kv(kv, kv_indptr, kv_indices, kv_last_page_len, b)
        if window:
            k, v = k[-window:], v[-window:]
        qs = (Q[b] * scale).reshape(Hkv, G, D)
        sk = None if sinks is None else np.asarray(sinks, np.float32).reshape(Hkv, G)
        out[b] = _softmax_attend(qs, k, v, logit_cap, sk).reshape(Hq, D)
    return out
