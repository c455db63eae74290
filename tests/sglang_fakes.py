"""Minimal stand-ins for the SGLang objects the backend adapter reads (SGLang is not
installed here): a token pool with per-layer K/V buffers, a request-to-token map filled
by a paged allocator, a forward batch and a RadixAttention-like layer. Field
names follow SGLang's (ForwardBatch, MHATokenToKVPool, ReqToTokenPool, RadixAttention);
the allocator's page size is the server's page_size (16 by default).
"""
from __future__ import annotations

import math
from types import SimpleNamespace

import torch

PAGE = 16


class Mode:
    def __init__(self, decode: bool):
        self._decode = decode

    def is_decode(self) -> bool:
        return self._decode


class TokenPool:
    """MHATokenToKVPool-like: k_buffer[layer] / v_buffer[layer] of (slots, Hkv, D). An fp8
    pool stores uint8 and hands out float8_e4m3fn views; set_kv_buffer divides by the
    layer's scales and casts, as SGLang's pool does."""

    def __init__(self, slots, layers, hkv, d, dtype, device, gen):
        self.dtype = dtype
        self.store_dtype = torch.uint8 if dtype == torch.float8_e4m3fn else dtype
        mk = lambda: torch.randn(slots, hkv, d, generator=gen, device=device).to(dtype)  # noqa: E731
        self.k_buffer = [mk().view(self.store_dtype) for _ in range(layers)]
        self.v_buffer = [mk().view(self.store_dtype) for _ in range(layers)]

    def get_key_buffer(self, layer_id):
        return self.k_buffer[layer_id].view(self.dtype)

    def get_value_buffer(self, layer_id):
        return self.v_buffer[layer_id].view(self.dtype)

    def get_kv_buffer(self, layer_id):
        return self.get_key_buffer(layer_id), self.get_value_buffer(layer_id)

    def set_kv_buffer(self, layer, loc, cache_k, cache_v, k_scale=None, v_scale=None):
        kb, vb = self.k_buffer[layer.layer_id], self.v_buffer[layer.layer_id]
        if cache_k.dtype != self.dtype:
            if k_scale is not None:
                cache_k = cache_k / k_scale
            if v_scale is not None:
                cache_v = cache_v / v_scale
            cache_k, cache_v = cache_k.to(self.dtype), cache_v.to(self.dtype)
        kb[loc.long()] = cache_k.reshape(-1, kb.shape[1], kb.shape[2]).view(self.store_dtype)
        vb[loc.long()] = cache_v.reshape(-1, vb.shape[1], vb.shape[2]).view(self.store_dtype)


def make_batch(lens, hq=32, hkv=8, d=128, layers=2, dtype=torch.float16, device="cuda",
               seed=0, pool_pages=None, rows=None, decode=True, kv_dtype=None, k_scale=None,
               v_scale=None, server_page=PAGE):
    """Requests of `lens` tokens (the decode token included) with pages of
    `server_page` slots (the server's page_size) drawn from a shuffled free list; returns
    (forward_batch, layer list, pool, req_to_token)."""
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    sp = server_page
    need = sum(math.ceil(n / sp) for n in lens)
    pool_pages = pool_pages or need + 8
    perm = torch.randperm(pool_pages, generator=gen).tolist()
    max_ctx = max(lens) + sp if lens else sp
    n_rows = rows or len(lens) + 3
    req_to_token = torch.zeros(n_rows, max_ctx, dtype=torch.int32)
    row_ids = torch.randperm(n_rows, generator=gen)[:len(lens)].tolist()
    for r, n in zip(row_ids, lens):
        for p in range(math.ceil(n / sp)):
            page = perm.pop()
            for t in range(p * sp, min(n, (p + 1) * sp)):
                req_to_token[r, t] = page * sp + t % sp
    dgen = torch.Generator(device=device)
    dgen.manual_seed(seed + 1)
    pool = TokenPool(pool_pages * sp, layers, hkv, d, kv_dtype or dtype, device, dgen)
    seq_lens = torch.tensor(lens, dtype=torch.int64)
    out_cache_loc = torch.tensor([int(req_to_token[r, n - 1]) for r, n in zip(row_ids, lens)],
                                 dtype=torch.int64)
    fb = SimpleNamespace(
        forward_mode=Mode(decode), batch_size=len(lens),
        req_pool_indices=torch.tensor(row_ids, dtype=torch.int64, device=device),
        seq_lens=seq_lens.to(device), seq_lens_sum=int(seq_lens.sum()), seq_lens_cpu=seq_lens,
        out_cache_loc=out_cache_loc.to(device),
        req_to_token_pool=SimpleNamespace(req_to_token=req_to_token.to(device)),
        token_to_kv_pool=pool)
    layer_objs = [SimpleNamespace(layer_id=i, tp_q_head_num=hq, tp_k_head_num=hkv,
                                  tp_v_head_num=hkv, head_dim=d, scaling=d ** -0.5,
                                  logit_cap=0.0, k_scale=k_scale, v_scale=v_scale)
                  for i in range(layers)]
    return fb, layer_objs, pool, req_to_token
