"""SGLang attention backend on the MI355X split-KV decode kernel.

Counterpart of the reference adapter (integration/sglang_backend.py:50-137): decode steps
go to the HIP kernel through `decode_attention`; prefill (extend) stays outside this path.
Two entry styles are provided:

* SGLang's backend API — `init_forward_metadata(forward_batch)` once per batch, then
  `forward_decode(q, k, v, layer, forward_batch, save_kv_cache=True)` per layer — reading
  the token pool SGLang owns: per-layer K and V buffers of shape (slots, kv_heads,
  head_dim) with pages of 16 tokens or a multiple of 16 (server `page_size`), the
  request-to-token map and the batch's sequence lengths. The page table is built on the device once per batch
  (paging.build_page_table) and shared by every layer; the pool is read in place as a
  (k_cache, v_cache) pair of (pages, 16, kv_heads, head_dim) views.
* The reference shim's `forward(q, kv_data, kv_indptr, kv_indices, kv_last_page_len,
  is_prefill=False)` (integration/sglang_backend.py:85-101), for callers that already
  hold FlashInfer page tables.

An fp8_e4m3 KV cache (SGLang stores it as uint8 and hands out float8_e4m3fn views) is
read with the layer's k_scale / v_scale, which the pool also divides by when it writes.

Registration (the reference's entry points, integration/sglang_backend.py:112-137):
`register_backend()` adds the class under BACKEND_NAME to SGLang's attention-backend table:
through `register_attention_backend` where SGLang exports it (its decorator form,
`register_attention_backend(name)(factory)` with a factory called with the model runner,
or a `(name, cls)` function), else into the module's `ATTENTION_BACKENDS` or
`_BACKEND_REGISTRY` dict; importing this module with SGLANG_ATTENTION_BACKEND=split_kv_hip
does it once. SGLang is looked up lazily; without it the backend class has a plain base,
so the module imports (and is tested) anywhere.
"""
from __future__ import annotations

import importlib
import logging
import math
import os
from dataclasses import dataclass
from typing import Optional

import torch

import attention
import paging
from attention import decode_attention

BACKEND_NAME = "split_kv_hip"
PAGE_SIZE = 16
# split_kv for decode: 0 = automatic (balanced / one pass, chosen per batch); the
# reference's SPLIT_KV variable (integration/sglang_backend.py:32) is honoured.
DEFAULT_SPLIT_KV = int(os.environ.get("SPLIT_KV", "0"))


_log = logging.getLogger(__name__)

# Where SGLang keeps its attention-backend base class and its backend table, newest
# layout first (the class moved into base_attn_backend, the table into
# attention_registry, in later releases).
_SGLANG_BASE_MODULES = ("sglang.srt.layers.attention.base_attn_backend",
                        "sglang.srt.layers.attention")
_SGLANG_REGISTRY_MODULES = ("sglang.srt.layers.attention.attention_registry",
                            "sglang.srt.layers.attention")
# backend tables by name, newest first
_REGISTRY_TABLES = ("ATTENTION_BACKENDS", "_BACKEND_REGISTRY")
# forward()'s is_prefill when the caller leaves it out (None is a value a caller may pass)
_UNSET = object()


def _optional_module(path: str):
    """The module at `path`, or None when it (or SGLang itself) cannot be imported."""
    try:
        return importlib.import_module(path)
    except ImportError:
        return None


def _backend_base() -> type:
    """SGLang's AttentionBackend when SGLang is importable, else `object`: the adapter
    defines every method it is called through, so it needs nothing from the base."""
    for path in _SGLANG_BASE_MODULES:
        base = getattr(_optional_module(path), "AttentionBackend", None)
        if isinstance(base, type):
            return base
    return object


@dataclass
class DecodeMetadata:
    """Per-batch state shared by every layer's decode call."""
    kv_indptr: torch.Tensor
    kv_indices: torch.Tensor
    kv_last_page_len: torch.Tensor
    max_pages_per_seq: int          # plan hint (0 = unknown)


class SplitKVHipBackend(_backend_base()):
    """Decode attention on the HIP split-KV kernel; prefill on PyTorch SDPA."""

    def __init__(self, model_runner=None, split_kv: Optional[int] = None):
        self.model_runner = model_runner
        self.split_kv = DEFAULT_SPLIT_KV if split_kv is None else split_kv
        self.forward_metadata: Optional[DecodeMetadata] = None
        self._workspace: Optional[torch.Tensor] = None
        self._scales: dict = {}           # layer_id -> (k_scale, v_scale) of an fp8 pool
        self._sink_cache: dict = {}       # (layer_id, tensor) -> fp32 attention sinks
        self._graph_tables = None         # persistent page tables for HIP graph replay
        self._graph_max_bs = 0
        self._graph_workspace: Optional[torch.Tensor] = None   # captured calls' scratch
        self._retired_graph_workspaces: list = []   # outgrown, still read by old graphs
        self.page_size = _server_page_size(model_runner)
        # A server page of a multiple of 16 slots holds whole, aligned 16-slot blocks, so
        # a request's tokens 16p .. 16p+15 sit in slots 16 * id .. 16 * id + 15 with
        # id = slot(16p) // 16: the kernel's 16-token page. Smaller pages (SGLang's
        # default, 1) scatter them.
        if self.page_size is not None and (self.page_size <= 0 or
                                           self.page_size % PAGE_SIZE != 0):
            raise ValueError(
                f"{BACKEND_NAME} reads the token pool as 16-token pages (page id = slot // "
                f"16), so SGLang must run with a page_size that is a multiple of 16; this "
                f"server has page_size {self.page_size} (start it with --page-size 16)")

    @classmethod
    def name(cls) -> str:
        return BACKEND_NAME

    # ---------------------------------------------------------------- SGLang API
    def init_forward_metadata(self, forward_batch) -> None:
        """Build the batch's page table on the device (no host sync)."""
        req_to_token = forward_batch.req_to_token_pool.req_to_token
        seq_lens = forward_batch.seq_lens
        batch = int(seq_lens.shape[0])
        seq_lens_sum = getattr(forward_batch, "seq_lens_sum", None)
        lens_cpu = getattr(forward_batch, "seq_lens_cpu", None)
        if seq_lens_sum is None:
            # last resort: one device read (SGLang always provides seq_lens_sum)
            seq_lens_sum = int(seq_lens.sum().item())
        indptr, indices, last = paging.build_page_table(
            req_to_token, forward_batch.req_pool_indices, seq_lens,
            capacity=paging.page_capacity(seq_lens_sum, batch))
        hint = 0
        if lens_cpu is not None and batch:
            hint = (int(torch.as_tensor(lens_cpu).max()) + PAGE_SIZE - 1) // PAGE_SIZE
        self.forward_metadata = DecodeMetadata(indptr, indices, last, hint)

    def forward_decode(self, q, k, v, layer, forward_batch, save_kv_cache: bool = True,
                       **kwargs):
        """One layer's decode attention; returns (batch, q_heads * head_dim)."""
        sinks = self._sinks(kwargs.pop("sinks", None), layer)
        _refuse_extras("forward_decode", kwargs)
        pool = forward_batch.token_to_kv_pool
        if k is not None and save_kv_cache:
            self._save(pool, layer, forward_batch.out_cache_loc, k, v)
        md = self.forward_metadata
        if md is None:
            raise RuntimeError("init_forward_metadata must run before forward_decode")
        hq, d = layer.tp_q_head_num, layer.head_dim
        kc, vc = self._paged_views(pool, layer.layer_id)
        qv = q.reshape(-1, hq, d)
        scales = {}
        if kc.dtype == torch.float8_e4m3fn:      # SGLang's fp8_e4m3 KV cache
            scales = dict(zip(("k_scale", "v_scale"), self._kv_scales(layer)))
        out = decode_attention(
            qv, (kc, vc), md.kv_indptr, md.kv_indices, md.kv_last_page_len,
            split_kv=self.split_kv, workspace=self._workspace_for(qv, kc.shape[2]),
            max_pages_per_seq=md.max_pages_per_seq, sm_scale=_scale(layer, d),
            logit_cap=_logit_cap(layer), window=_window(layer), sinks=sinks, **scales)
        return out.view(-1, hq * d)

    @staticmethod
    def _save(pool, layer, loc, k, v):
        """The pool's own write (SGLang quantises to an fp8 pool with the layer's scales)."""
        ks, vs = getattr(layer, "k_scale", None), getattr(layer, "v_scale", None)
        if ks is None and vs is None:
            pool.set_kv_buffer(layer, loc, k, v)
        else:
            pool.set_kv_buffer(layer, loc, k, v, ks, vs)

    def _sinks(self, sinks, layer):
        """A layer's attention sinks as decode_attention takes them (contiguous float32,
        one per q head), converted once per layer and source tensor; None stays None."""
        if sinks is None:
            return None
        key = (getattr(layer, "layer_id", id(layer)), sinks.data_ptr(), sinks.dtype)
        got = self._sink_cache.get(key)
        if got is None:
            got = self._sink_cache[key] = sinks.detach().reshape(-1).to(torch.float32).contiguous()
        return got

    def _kv_scales(self, layer):
        """(k_scale, v_scale) floats of a layer (1.0 when unset), read once per layer:
        `k_scale_float` when the model loader set it, else `k_scale` (float or tensor)."""
        key = getattr(layer, "layer_id", id(layer))
        if key not in self._scales:
            vals = []
            for name in ("k_scale", "v_scale"):
                x = getattr(layer, name + "_float", None)
                if x is None:
                    x = getattr(layer, name, None)
                if isinstance(x, torch.Tensor):
                    x = float(x.detach().float().reshape(-1)[0].item())
                vals.append(1.0 if x is None else float(x))
            self._scales[key] = tuple(vals)
        return self._scales[key]

    def forward_extend(self, q, k, v, layer, forward_batch, save_kv_cache: bool = True,
                       **kwargs):
        """Prefill / extend: causal attention of the new tokens over each request's cached
        prefix and themselves, with PyTorch SDPA per request (outside the decode path)."""
        sinks = self._sinks(kwargs.pop("sinks", None), layer)
        _refuse_extras("forward_extend", kwargs)
        pool = forward_batch.token_to_kv_pool
        if k is not None and save_kv_cache:
            self._save(pool, layer, forward_batch.out_cache_loc, k, v)
        hq, hkv, d = layer.tp_q_head_num, layer.tp_k_head_num, layer.head_dim
        kb, vb = pool.get_key_buffer(layer.layer_id), pool.get_value_buffer(layer.layer_id)
        ks, vs = self._kv_scales(layer) if kb.dtype == torch.float8_e4m3fn else (1.0, 1.0)
        req_to_token = forward_batch.req_to_token_pool.req_to_token
        qv = q.reshape(-1, hq, d)
        out = torch.empty_like(qv)
        ext = forward_batch.extend_seq_lens_cpu
        lens = forward_batch.seq_lens_cpu
        rows = forward_batch.req_pool_indices.tolist()
        start = 0
        for row, n_new, n_all in zip(rows, list(ext), list(lens)):
            n_new, n_all = int(n_new), int(n_all)
            slots = req_to_token[row, :n_all].long()
            kk = kb[slots].float().transpose(0, 1) * ks      # (hkv, n_all, d)
            vv = vb[slots].float().transpose(0, 1) * vs
            qq = qv[start:start + n_new].float().transpose(0, 1)   # (hq, n_new, d)
            g = hq // hkv
            kk = kk.repeat_interleave(g, dim=0)
            vv = vv.repeat_interleave(g, dim=0)
            # new token i sits at position n_all - n_new + i and sees positions <= it
            pos_q = torch.arange(n_all - n_new, n_all, device=q.device)[:, None]
            kpos = torch.arange(n_all, device=q.device)[None, :]
            mask = kpos <= pos_q
            win = _window(layer)
            if win:                                   # sliding window: the last `win` keys
                mask &= kpos > pos_q - win
            scale = _scale(layer, d) or 1.0 / math.sqrt(d)
            cap = _logit_cap(layer)
            if cap or sinks is not None:
                # soft-capped scores or attention sinks: SDPA has neither, so attend
                # explicitly (a sink is one more logit per head, with no value)
                s_ = torch.matmul(qq, kk.transpose(1, 2)) * scale
                if cap:
                    s_ = torch.tanh(s_ / cap) * cap
                s_ = s_.masked_fill(~mask, float("-inf"))
                if sinks is not None:
                    col = sinks.view(hq, 1, 1).expand(hq, s_.shape[1], 1)
                    p_ = torch.softmax(torch.cat([s_, col], dim=-1), -1)[..., :-1]
                else:
                    p_ = torch.softmax(s_, -1)
                o = torch.matmul(p_, vv)
            else:
                o = torch.nn.functional.scaled_dot_product_attention(
                    qq, kk, vv, attn_mask=mask, scale=scale)
            out[start:start + n_new] = o.transpose(0, 1).to(out.dtype)
            start += n_new
        return out.view(-1, hq * d)

    def forward_sglang(self, q, k, v, layer, forward_batch, save_kv_cache: bool = True,
                       **kwargs):
        """SGLang's dispatch by forward mode."""
        if forward_batch.forward_mode.is_decode():
            return self.forward_decode(q, k, v, layer, forward_batch, save_kv_cache, **kwargs)
        return self.forward_extend(q, k, v, layer, forward_batch, save_kv_cache, **kwargs)

    # ---------------------------------------------------------------- HIP graphs
    # SGLang captures decode steps in graphs (its "CUDA graph" runner; HIP graphs here).
    # The page table then lives in persistent buffers the graph reads, refilled in place
    # before each replay by one kernel; the captured decode call uses the balanced
    # schedule (no plan hint), which is valid for any sequence lengths at replay.

    def get_cuda_graph_seq_len_fill_value(self) -> int:
        return 1

    def init_cuda_graph_state(self, max_bs: int, max_num_tokens: Optional[int] = None,
                              max_context_len: Optional[int] = None, device=None):
        """Persistent page-table buffers for batches of up to max_bs requests."""
        mr = self.model_runner
        if max_context_len is None:
            max_context_len = int(mr.model_config.context_len)
        if device is None:
            device = mr.device if mr is not None and hasattr(mr, "device") else "cuda"
        pages = max_bs * ((int(max_context_len) + PAGE_SIZE - 1) // PAGE_SIZE + 1)
        self._graph_tables = (torch.zeros(max_bs + 1, dtype=torch.int32, device=device),
                              torch.zeros(pages, dtype=torch.int32, device=device),
                              torch.ones(max_bs, dtype=torch.int32, device=device))
        self._graph_max_bs = max_bs

    def _fill_graph_tables(self, bs, req_pool_indices, seq_lens, req_to_token=None):
        if getattr(self, "_graph_tables", None) is None:
            raise RuntimeError("init_cuda_graph_state must run before graph capture")
        if bs > self._graph_max_bs:
            raise ValueError(f"batch {bs} exceeds the graph state's {self._graph_max_bs}")
        if req_to_token is None:
            req_to_token = self.model_runner.req_to_token_pool.req_to_token
        indptr, indices, last = paging.build_page_table(
            req_to_token, req_pool_indices[:bs], seq_lens[:bs], out=self._graph_tables)
        self.forward_metadata = DecodeMetadata(indptr, indices, last, 0)

    def init_forward_metadata_capture_cuda_graph(self, bs, num_tokens, req_pool_indices,
                                                 seq_lens, encoder_lens=None, forward_mode=None,
                                                 spec_info=None, req_to_token=None):
        self._fill_graph_tables(bs, req_pool_indices, seq_lens, req_to_token)

    def init_forward_metadata_replay_cuda_graph(self, bs, req_pool_indices, seq_lens,
                                                seq_lens_sum=None, encoder_lens=None,
                                                forward_mode=None, spec_info=None,
                                                seq_lens_cpu=None, req_to_token=None):
        self._fill_graph_tables(bs, req_pool_indices, seq_lens, req_to_token)

    # ---------------------------------------------------------------- reference shim API
    def forward(self, q, kv_data=None, kv_indptr=None, kv_indices=None, kv_last_page_len=None,
                is_prefill=_UNSET, **kwargs):
        """The reference adapter's entry (integration/sglang_backend.py:85-101): page
        tables given by the caller; decode runs the HIP kernel. Called with SGLang's
        (q, k, v, layer, forward_batch[, save_kv_cache]) it dispatches like SGLang's own
        backends."""
        fb = kwargs.pop("forward_batch", None)
        if fb is None and hasattr(kv_last_page_len, "forward_mode"):
            fb = kv_last_page_len
        if fb is not None:
            # SGLang's signature: forward(q, k, v, layer, forward_batch, save_kv_cache=True);
            # RadixAttention passes save_kv_cache by position, i.e. in is_prefill's slot
            layer = kwargs.pop("layer", kv_indices)
            k = kwargs.pop("k", kv_data)
            v = kwargs.pop("v", kv_indptr)
            save = kwargs.pop("save_kv_cache", True if is_prefill is _UNSET else is_prefill)
            return self.forward_sglang(q, k, v, layer, fb, bool(save), **kwargs)
        if is_prefill is not _UNSET and is_prefill:
            raise NotImplementedError(
                "prefill is not on the decode path; use forward_extend with SGLang's batch")
        return decode_attention(q, kv_data, kv_indptr, kv_indices, kv_last_page_len,
                                split_kv=self.split_kv)

    # ---------------------------------------------------------------- helpers
    @staticmethod
    def _paged_views(pool, layer_id):
        kb, vb = pool.get_key_buffer(layer_id), pool.get_value_buffer(layer_id)
        pages = kb.shape[0] // PAGE_SIZE
        shape = (pages, PAGE_SIZE) + tuple(kb.shape[1:])
        return kb[:pages * PAGE_SIZE].view(shape), vb[:pages * PAGE_SIZE].view(shape)

    def _workspace_for(self, q, hkv):
        """Scratch for one decode call (None when the call needs none). Eager calls share
        one buffer that grows with the batch. A call under graph capture gets the graph
        workspace instead: its address is baked into the graph and every replay writes
        there, so it is sized once for the graph state's largest batch, never handed to
        eager calls, and never freed while the backend lives (one outgrown by a later
        capture is kept too)."""
        split = attention.resolve_split(self.split_kv)
        bs, hq, d = q.shape
        need = attention.dk_lib.workspace_bytes(bs, hq, hkv, d, split)
        if need == 0:
            return None
        if torch.cuda.is_current_stream_capturing():
            ws = self._graph_workspace
            if ws is None or ws.numel() < need or ws.device != q.device:
                if ws is not None:
                    self._retired_graph_workspaces.append(ws)
                most = attention.dk_lib.workspace_bytes(max(bs, self._graph_max_bs), hq, hkv,
                                                        d, split)
                ws = self._graph_workspace = torch.empty(max(need, most), dtype=torch.uint8,
                                                         device=q.device)
            return ws
        ws = self._workspace
        if ws is None or ws.numel() < need or ws.device != q.device:
            ws = self._workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
        return ws


def _refuse_extras(where: str, kwargs: dict) -> None:
    """Newer SGLang releases pass optional per-call inputs by keyword (separate rope parts
    of q and k for MLA, ...); attention sinks are taken before this check. The others are
    not supported here: a call that sets one is refused rather than attended without it;
    unset (None) ones pass."""
    extras = sorted(k for k, v in kwargs.items() if v is not None)
    if extras:
        raise NotImplementedError(f"{BACKEND_NAME}.{where}: unsupported inputs {extras}")


def _server_page_size(model_runner) -> Optional[int]:
    """Token-pool page size of the SGLang server (ModelRunner.page_size, else its
    server_args.page_size); None when the runner does not say."""
    if model_runner is None:
        return None
    ps = getattr(model_runner, "page_size", None)
    if ps is None:
        ps = getattr(getattr(model_runner, "server_args", None), "page_size", None)
    return None if ps is None else int(ps)


def _window(layer) -> Optional[int]:
    """RadixAttention.sliding_window_size (FlashInfer's window_left: the new token attends
    to itself and that many before it; -1 or None = no window) as a token count."""
    w = getattr(layer, "sliding_window_size", None)
    return int(w) + 1 if w is not None and int(w) >= 0 else None


def _logit_cap(layer) -> Optional[float]:
    """RadixAttention.logit_cap (Gemma 2's soft-capping), None when off."""
    cap = getattr(layer, "logit_cap", None)
    return float(cap) if cap not in (None, 0, 0.0) else None


def _scale(layer, d) -> Optional[float]:
    s = getattr(layer, "scaling", None)
    if s is None or abs(s * math.sqrt(d) - 1.0) < 1e-7:
        return None
    return float(s)


def _registry_module():
    """The first of SGLang's modules that holds an attention-backend table (a
    registration hook or a table dict), else the first that imports, else None."""
    first = None
    for path in _SGLANG_REGISTRY_MODULES:
        mod = _optional_module(path)
        if mod is None:
            continue
        first = first or mod
        if callable(getattr(mod, "register_attention_backend", None)) or any(
                isinstance(getattr(mod, t, None), dict) for t in _REGISTRY_TABLES):
            return mod
    return first


def _register_through_hook(hook) -> str:
    """Call SGLang's register_attention_backend. Its decorator form takes the name and
    returns a decorator for a factory called with the model runner (the class is such a
    factory: SplitKVHipBackend(model_runner)); other versions take (name, cls). Returns
    the form used; raises what the hook raises."""
    try:
        deco = hook(BACKEND_NAME)
    except TypeError:
        hook(BACKEND_NAME, SplitKVHipBackend)
        return "register_attention_backend(name, cls)"
    if not callable(deco):
        raise TypeError("register_attention_backend(name) returned no decorator")
    deco(SplitKVHipBackend)
    return "register_attention_backend(name)(factory)"


def register_backend(registry=None) -> bool:
    """Make SplitKVHipBackend selectable under BACKEND_NAME (the reference's
    register_backend, integration/sglang_backend.py:112-137). `registry` is the module
    holding SGLang's backend table (default: sglang.srt.layers.attention.attention_registry,
    else sglang.srt.layers.attention). Uses its `register_attention_backend` when present
    (see _register_through_hook), else sets the entry of its `ATTENTION_BACKENDS` or
    `_BACKEND_REGISTRY` dict. Returns whether the backend is now registered; never raises
    for a missing or unfamiliar SGLang (the outcome is logged)."""
    if registry is None:
        registry = _registry_module()
    if registry is None:
        _log.warning("%s: SGLang is not importable, so there is no backend table to add "
                     "the decode backend to", BACKEND_NAME)
        return False
    name = getattr(registry, "__name__", type(registry).__name__)
    hook = getattr(registry, "register_attention_backend", None)
    table_name = next((t for t in _REGISTRY_TABLES
                       if isinstance(getattr(registry, t, None), dict)), None)
    try:
        if callable(hook):
            how = _register_through_hook(hook)
        elif table_name is not None:
            getattr(registry, table_name)[BACKEND_NAME] = SplitKVHipBackend
            how = table_name
        else:
            _log.warning("%s: %s has neither register_attention_backend nor a backend "
                         "table (%s); not registered", BACKEND_NAME, name,
                         " / ".join(_REGISTRY_TABLES))
            return False
    except Exception as exc:  # noqa: BLE001 - SGLang's own checks: log them, do not fail import
        _log.warning("%s: %s refused the backend: %s", BACKEND_NAME, name, exc)
        return False
    _log.info("%s: added to %s through %s", BACKEND_NAME, name, how)
    return True


def _register_if_selected() -> None:
    """SGLANG_ATTENTION_BACKEND=split_kv_hip at import selects this backend (the
    reference's environment switch)."""
    if os.environ.get("SGLANG_ATTENTION_BACKEND", "").strip() == BACKEND_NAME:
        register_backend()


_register_if_selected()
