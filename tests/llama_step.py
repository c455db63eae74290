"""A Llama-3.2-1B-shaped decode step for config 5 (test infrastructure).

16 decoder layers, hidden 2048, 32 q heads / 8 kv heads of 64 dims, SwiGLU MLP 8192,
RMSNorm, Llama-3 rotary frequencies (theta 500000, factor 32), tied embeddings over a
128256-token vocabulary; random weights N(0, 0.02^2) from a seed (no checkpoint is
available offline). One decode step for a batch whose sequences already hold ctx - 1
tokens of synthetic bf16 K/V history in a paged cache (page_size 16).

Two runs of the same step:
  * `gpu_step()`: bf16 on the GPU; the new token is written with paging.append_kv (RoPE
    fused) and attention is attention.decode_attention; optionally every layer's attention
    output is also checked against the oracle on the same inputs;
  * `cpu_step()`: everything in fp32 on the CPU with the oracle (oracle/append.py,
    oracle/reference.py).
With `kv_scale` set, the caches are fp8 (E4M3) with that scale for K and V: the history is
quantised once, the GPU step writes the new token with the quantising append, and the CPU
step quantises it the same way (oracle append_kv_fp8) and attends over the dequantised
cache.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

import attention
import paging
from helpers import to_np
from oracle import append as oapp
from oracle import reference as ref

PAGE = 16


@dataclass
class Cfg:
    layers: int = 16
    hidden: int = 2048
    hq: int = 32
    hkv: int = 8
    d: int = 64
    ffn: int = 8192
    vocab: int = 128256
    batch: int = 32
    ctx: int = 2048
    eps: float = 1e-5


def llama3_inv_freq(cfg: Cfg) -> np.ndarray:
    """Llama 3.2's rotary frequencies, from transformers' own rope initialisation."""
    from transformers import LlamaConfig
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS
    c = LlamaConfig(hidden_size=cfg.hidden, num_attention_heads=cfg.hq,
                    num_key_value_heads=cfg.hkv, head_dim=cfg.d, rope_theta=500000.0,
                    max_position_embeddings=131072,
                    rope_scaling={"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
                                  "high_freq_factor": 4.0,
                                  "original_max_position_embeddings": 8192})
    inv, _ = ROPE_INIT_FUNCTIONS["llama3"](c, "cpu")
    return inv.float().numpy()


def make_model(cfg: Cfg, seed: int = 0, device="cuda"):
    """bf16 weights on the device, N(0, 0.02^2); norm weights 1 (Llama's init)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    w = lambda *s: (torch.randn(*s, generator=g, device=device) * 0.02).to(torch.bfloat16)  # noqa: E731
    layers = []
    for _ in range(cfg.layers):
        layers.append(dict(wq=w(cfg.hq * cfg.d, cfg.hidden), wk=w(cfg.hkv * cfg.d, cfg.hidden),
                           wv=w(cfg.hkv * cfg.d, cfg.hidden), wo=w(cfg.hidden, cfg.hq * cfg.d),
                           wg=w(cfg.ffn, cfg.hidden), wu=w(cfg.ffn, cfg.hidden),
                           wd=w(cfg.hidden, cfg.ffn)))
    return dict(embed=w(cfg.vocab, cfg.hidden), layers=layers)


def make_cache(cfg: Cfg, seed: int = 1, device="cuda", kv_scale=None):
    """Per-layer combined caches (pages, 2, 16, Hkv, D) bf16 (or fp8 E4M3 codes of
    value / kv_scale) holding ctx - 1 history tokens per sequence on a permuted page pool,
    and the page table already grown by the new token's slot (position ctx - 1)."""
    pages_per_seq = math.ceil(cfg.ctx / PAGE)
    n_pages = cfg.batch * pages_per_seq
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    perm = torch.randperm(n_pages, generator=gen).to(torch.int32)
    indptr = torch.arange(0, n_pages + 1, pages_per_seq, dtype=torch.int32)
    last = torch.full((cfg.batch,), cfg.ctx - (pages_per_seq - 1) * PAGE, dtype=torch.int32)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    caches = [torch.randn(n_pages, 2, PAGE, cfg.hkv, cfg.d, generator=g,
                          device=device).to(torch.bfloat16) for _ in range(cfg.layers)]
    if kv_scale is not None:
        caches = [(c.float() / kv_scale).clamp(-448, 448).to(torch.float8_e4m3fn)
                  for c in caches]
    return caches, indptr.to(device), perm.to(device), last.to(device)


def _cache_np(cache, kv_scale):
    """float32 values of a cache (dequantised when it is fp8)."""
    if cache.dtype == torch.float8_e4m3fn:
        from oracle import fp8
        return fp8.dequantize(cache.view(torch.uint8).cpu().numpy(), kv_scale)
    return to_np(cache)


def _rms(x, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)


def gpu_step(cfg, model, caches, indptr, ids, last, tokens, inv_freq, check_rows=None,
             kv_scale=None):
    """Logits (batch, vocab) fp32 of the bf16 decode step on the device, and, for the
    sequences in check_rows, each layer's max-abs error of the HIP attention against the
    oracle on the same inputs."""
    hint = attention.plan_hint(indptr.cpu())
    inv = torch.as_tensor(inv_freq, device=tokens.device)
    sc = {} if kv_scale is None else dict(k_scale=kv_scale, v_scale=kv_scale)
    h = model["embed"][tokens].float()
    errs = []
    for li, L in enumerate(model["layers"]):
        x = _rms(h, cfg.eps).to(torch.bfloat16)
        q = (x @ L["wq"].T).view(-1, cfg.hq, cfg.d)
        k = (x @ L["wk"].T).view(-1, cfg.hkv, cfg.d)
        v = (x @ L["wv"].T).view(-1, cfg.hkv, cfg.d)
        paging.append_kv(q, k, v, caches[li], indptr, ids, last, inv_freq=inv, **sc)
        o = attention.decode_attention(q, caches[li], indptr, ids, last, split_kv=0,
                                       max_pages_per_seq=hint, **sc)
        if check_rows is not None:
            want = ref.reference_attention_paged(to_np(q), _cache_np(caches[li], kv_scale),
                                                 to_np(indptr),
                                                 to_np(ids), to_np(last),
                                                 batch_subset=check_rows)
            got = to_np(o)[list(check_rows)].astype(np.float64)
            errs.append(float(np.abs(got - want[list(check_rows)]).max()))
        h = h + (o.reshape(-1, cfg.hq * cfg.d) @ L["wo"].T).float()
        x = _rms(h, cfg.eps).to(torch.bfloat16)
        mlp = (torch.nn.functional.silu(x @ L["wg"].T) * (x @ L["wu"].T)) @ L["wd"].T
        h = h + mlp.float()
    logits = (_rms(h, cfg.eps).to(torch.bfloat16) @ model["embed"].T).float()
    return logits, errs


def cpu_step(cfg, model, caches, indptr, ids, last, tokens, inv_freq, kv_scale=None):
    """Logits (batch, vocab) of the same step in fp32 on the CPU with the oracle."""
    ip, ix, ll = to_np(indptr), to_np(ids), to_np(last)
    f = lambda t: t.float().cpu()  # noqa: E731
    h = f(model["embed"][tokens])
    for li, L in enumerate(model["layers"]):
        x = _rms(h, cfg.eps)
        q = (x @ f(L["wq"]).T).view(-1, cfg.hq, cfg.d).numpy()
        k = (x @ f(L["wk"]).T).view(-1, cfg.hkv, cfg.d).numpy()
        v = (x @ f(L["wv"]).T).view(-1, cfg.hkv, cfg.d).numpy()
        if kv_scale is None:
            kv_np, q_np = oapp.append_kv(to_np(caches[li]), q, k, v, ip, ix, ll,
                                         inv_freq=inv_freq)
        else:
            from oracle import fp8
            codes, q_np = oapp.append_kv_fp8(caches[li].view(torch.uint8).cpu().numpy(), q, k,
                                             v, ip, ix, ll, kv_scale, kv_scale,
                                             inv_freq=inv_freq)
            kv_np = fp8.dequantize(codes, kv_scale)
        o = ref.reference_attention_paged(q_np.astype(np.float32), kv_np.astype(np.float32),
                                          ip, ix, ll)
        h = h + torch.from_numpy(np.ascontiguousarray(o, np.float32)).reshape(-1, cfg.hq * cfg.d) @ f(L["wo"]).T
        x = _rms(h, cfg.eps)
        h = h + (torch.nn.functional.silu(x @ f(L["wg"]).T) * (x @ f(L["wu"]).T)) @ f(L["wd"]).T
    return _rms(h, cfg.eps) @ f(model["embed"]).T


def top5_agreement(a: torch.Tensor, b: torch.Tensor):
    """(mean |top5(a) & top5(b)| / 5, fraction of rows whose top-1 agree)."""
    ta, tb = a.topk(5, dim=-1).indices.cpu(), b.topk(5, dim=-1).indices.cpu()
    overlap = [len(set(x.tolist()) & set(y.tolist())) / 5 for x, y in zip(ta, tb)]
    return float(np.mean(overlap)), float((ta[:, 0] == tb[:, 0]).float().mean())
