"""CPU restatement of the cache write before a decode step (test infrastructure only).

Format written: src/layout.md:41-69 (K at kv_data[page, 0, slot, h], V at [page, 1, slot,
h]). Rotary position embedding as Llama models apply it (transformers'
LlamaRotaryEmbedding + apply_rotary_pos_emb: angles position * inv_freq formed in fp32,
rotate_half pairs (i, i + D/2)); the GPT-J interleaved pairing (2i, 2i + 1) as option.
The rotation itself is evaluated in float64 here and stored at the inputs' float width
(at least float32). `append_kv_fp8` writes an OCP E4M3 cache instead: each element is the
rotated (K) or copied (V) value rounded to float32, divided by its scale in float32,
clamped to +-448 and rounded to the nearest code (ties to even), as oracle/fp8.py encodes.
"""
from __future__ import annotations

import numpy as np

PAGE = 16


def rope(x, pos, inv_freq, style: int = 0) -> np.ndarray:
    """x (..., D) rotated at position pos; float64 result."""
    x = np.asarray(x, np.float64)
    d = x.shape[-1]
    ang = (np.float32(pos) * np.asarray(inv_freq, np.float32)).astype(np.float64)  # fp32 angles
    c, s = np.cos(ang), np.sin(ang)
    out = x.copy()
    if style == 0:
        x0, x1 = x[..., : d // 2], x[..., d // 2:]
        out[..., : d // 2] = x0 * c - x1 * s
        out[..., d // 2:] = x1 * c + x0 * s
    else:
        x0, x1 = x[..., 0::2], x[..., 1::2]
        out[..., 0::2] = x0 * c - x1 * s
        out[..., 1::2] = x1 * c + x0 * s
    return out


def append_kv(kv_data, q, k_new, v_new, kv_indptr, kv_indices, kv_last_page_len,
              inv_freq=None, positions=None, style: int = 0):
    """(kv_data with the new tokens written, rotated q) as float copies.
    kv_data (pages, 2, 16, Hkv, D); q (B, Hq, D) or None; k_new, v_new (B, Hkv, D)."""
    # float32 inputs stay float32 (a rotated value rounded to fp32 is off by 2^-24 at most);
    # anything narrower is widened to float32, wider stays float64
    wide = lambda a: np.result_type(np.asarray(a).dtype, np.float32)  # noqa: E731
    kv = np.array(kv_data, wide(kv_data))
    qo = None if q is None else np.array(q, wide(q))
    for b in range(len(kv_last_page_len)):
        s, e = int(kv_indptr[b]), int(kv_indptr[b + 1])
        if e <= s:
            continue
        page, slot = int(kv_indices[e - 1]), int(kv_last_page_len[b]) - 1
        pos = positions[b] if positions is not None else (e - s - 1) * PAGE + slot
        k = np.asarray(k_new[b], np.float64)
        if inv_freq is not None:
            k = rope(k, pos, inv_freq, style)
            if qo is not None:
                qo[b] = rope(qo[b], pos, inv_freq, style)
        kv[page, 0, slot] = k
        kv[page, 1, slot] = np.asarray(v_new[b], np.float64)
    return kv, qo


def append_kv_fp8(codes, q, k_new, v_new, kv_indptr, kv_indices, kv_last_page_len,
                  k_scale: float, v_scale: float, inv_freq=None, positions=None,
                  style: int = 0):
    """(uint8 E4M3 cache (pages, 2, 16, Hkv, D) with the new tokens written, rotated q)."""
    from oracle import fp8
    out = np.array(codes, np.uint8)
    qo = None if q is None else np.array(q, np.result_type(np.asarray(q).dtype, np.float32))
    ks, vs = np.float32(k_scale), np.float32(v_scale)
    for b in range(len(kv_last_page_len)):
        s, e = int(kv_indptr[b]), int(kv_indptr[b + 1])
        if e <= s:
            continue
        page, slot = int(kv_indices[e - 1]), int(kv_last_page_len[b]) - 1
        pos = positions[b] if positions is not None else (e - s - 1) * PAGE + slot
        k = np.asarray(k_new[b], np.float64)
        if inv_freq is not None:
            k = rope(k, pos, inv_freq, style)
            if qo is not None:
                qo[b] = rope(qo[b], pos, inv_freq, style)
        v = np.asarray(v_new[b], np.float32)
        out[page, 0, slot] = fp8.encode_saturating(k.astype(np.float32) / ks)
        out[page, 1, slot] = fp8.encode_saturating(v / vs)
    return out, qo
