"""The SGLang backend adapter, the device page-table builder and the (k_cache, v_cache)
and sm_scale paths it uses.

CPU tests: the adapter imports and registers without SGLang (as the reference's does,
integration/sglang_backend.py:37-47,112-137). GPU tests: a decode step through the
adapter on an SGLang-shaped token pool against the oracle, the page table against
oracle/page_table.py (bit-exact), split caches and custom scales against the oracle.
"""
import math

import numpy as np
import pytest
import torch

import attention
import layout
import paging
import sglang_backend
from helpers import err_stats, to_np
from oracle import page_table as ptab
from oracle import reference as ref
from sglang_fakes import make_batch

DEV = "cuda"


# ---------------------------------------------------------------- CPU

def test_backend_imports_and_names_without_sglang():
    b = sglang_backend.SplitKVHipBackend(split_kv=4)
    assert b.name() == "split_kv_hip" and b.split_kv == 4
    assert sglang_backend.SplitKVHipBackend().split_kv == sglang_backend.DEFAULT_SPLIT_KV


def test_register_backend_reports_missing_sglang(caplog):
    with caplog.at_level("WARNING"):
        assert sglang_backend.register_backend() is False
    assert "SGLang is not importable" in caplog.text


def test_register_backend_uses_the_registration_hook():
    from types import SimpleNamespace
    seen = {}
    mod = SimpleNamespace(__name__="fake_attention",
                          register_attention_backend=lambda n, c: seen.update({n: c}),
                          _BACKEND_REGISTRY={})
    assert sglang_backend.register_backend(mod) is True
    assert seen == {"split_kv_hip": sglang_backend.SplitKVHipBackend}
    assert mod._BACKEND_REGISTRY == {}          # the hook wins over the dict


def test_register_backend_falls_back_to_the_registry_dict():
    from types import SimpleNamespace
    mod = SimpleNamespace(__name__="fake_attention", _BACKEND_REGISTRY={"fa3": object})
    assert sglang_backend.register_backend(mod) is True
    assert mod._BACKEND_REGISTRY["split_kv_hip"] is sglang_backend.SplitKVHipBackend
    assert sglang_backend.register_backend(SimpleNamespace(__name__="bare")) is False

    def refuse(name, cls):
        raise KeyError(name)
    assert sglang_backend.register_backend(
        SimpleNamespace(__name__="strict", register_attention_backend=refuse)) is False


def test_register_backend_through_the_decorator_hook():
    """SGLang's attention_registry form: register_attention_backend(name) returns a
    decorator that stores a factory called with the model runner."""
    from types import SimpleNamespace
    table = {}

    def register_attention_backend(name):
        def deco(fn):
            table[name] = fn
            return fn
        return deco
    mod = SimpleNamespace(__name__="fake_registry", ATTENTION_BACKENDS=table,
                          register_attention_backend=register_attention_backend)
    assert sglang_backend.register_backend(mod) is True
    factory = table["split_kv_hip"]
    backend = factory(SimpleNamespace(page_size=16))      # how SGLang builds a backend
    assert isinstance(backend, sglang_backend.SplitKVHipBackend) and backend.page_size == 16
    # a table without a hook: ATTENTION_BACKENDS before the legacy dict
    mod = SimpleNamespace(__name__="tables", ATTENTION_BACKENDS={}, _BACKEND_REGISTRY={})
    assert sglang_backend.register_backend(mod) is True
    assert "split_kv_hip" in mod.ATTENTION_BACKENDS and mod._BACKEND_REGISTRY == {}


@pytest.mark.parametrize("args,kwargs,save", [
    ((), {}, True),                                  # save_kv_cache left out
    ((False,), {}, False),                           # RadixAttention: by position
    ((True,), {}, True),
    ((), {"save_kv_cache": False}, False),           # by keyword
])
def test_sglang_forward_passes_save_kv_cache(monkeypatch, args, kwargs, save):
    """forward(q, k, v, layer, forward_batch, save_kv_cache) reaches forward_sglang with
    the caller's save_kv_cache, whether given by position (the reference shim's is_prefill
    slot) or by keyword."""
    from types import SimpleNamespace
    seen = {}

    def record(self, q, k, v, layer, fb, save_kv_cache=True):
        seen.update(q=q, k=k, v=v, layer=layer, fb=fb, save=save_kv_cache)
        return "out"
    monkeypatch.setattr(sglang_backend.SplitKVHipBackend, "forward_sglang", record)
    fb = SimpleNamespace(forward_mode=object())
    b = sglang_backend.SplitKVHipBackend()
    assert b.forward("q", "k", "v", "layer", fb, *args, **kwargs) == "out"
    assert seen == dict(q="q", k="k", v="v", layer="layer", fb=fb, save=save)


def test_unsupported_sglang_inputs_are_refused():
    """Keyword inputs of newer SGLang calls that the backend does not support (MLA rope
    parts) are refused when set, before anything is written or launched."""
    from types import SimpleNamespace
    b = sglang_backend.SplitKVHipBackend()
    fb = SimpleNamespace(forward_mode=SimpleNamespace(is_decode=lambda: True))
    with pytest.raises(NotImplementedError, match="k_rope"):
        b.forward_decode(None, None, None, None, fb, True, k_rope=object(), sinks=None)
    with pytest.raises(NotImplementedError, match="q_rope"):
        b.forward("q", "k", "v", "layer", fb, True, q_rope=object())
    fb.forward_mode = SimpleNamespace(is_decode=lambda: False)
    with pytest.raises(NotImplementedError, match="q_rope"):
        b.forward("q", "k", "v", "layer", fb, q_rope=object())


def test_reference_shim_prefill_is_refused():
    b = sglang_backend.SplitKVHipBackend()
    with pytest.raises(NotImplementedError):
        b.forward(None, None, None, None, None, True)
    with pytest.raises(NotImplementedError):
        b.forward(None, None, None, None, None, is_prefill=True)


@pytest.mark.parametrize("runner,ok", [
    (dict(page_size=16), True), (dict(page_size=1), False), (dict(page_size=32), True),
    (dict(page_size=64), True), (dict(page_size=8), False), (dict(page_size=24), False),
    (dict(page_size=0), False),
    (dict(server_args=dict(page_size=16)), True), (dict(server_args=dict(page_size=1)), False),
    (dict(), True)])
def test_backend_requires_pages_of_a_multiple_of_sixteen_tokens(runner, ok):
    from types import SimpleNamespace
    if "server_args" in runner:
        runner = dict(server_args=SimpleNamespace(**runner["server_args"]))
    mr = SimpleNamespace(**runner)
    if ok:
        assert sglang_backend.SplitKVHipBackend(mr).split_kv == sglang_backend.DEFAULT_SPLIT_KV
    else:
        with pytest.raises(ValueError, match="multiple of 16"):
            sglang_backend.SplitKVHipBackend(mr)


def test_page_capacity_bounds_the_page_count():
    rng = np.random.default_rng(0)
    for _ in range(100):
        lens = rng.integers(0, 300, size=rng.integers(1, 20))
        pages = sum(-(-int(n) // 16) for n in lens)
        assert pages <= paging.page_capacity(int(lens.sum()), len(lens))


def test_decode_without_metadata_is_an_error():
    fb = type("FB", (), {"token_to_kv_pool": None, "out_cache_loc": None})()
    layer = type("L", (), {"logit_cap": 0.0})()
    with pytest.raises(RuntimeError, match="init_forward_metadata"):
        sglang_backend.SplitKVHipBackend().forward_decode(None, None, None, layer, fb)


# ---------------------------------------------------------------- GPU

def _pool_as_combined(pool, layer_id):
    """(pages, 2, 16, Hkv, D) numpy copy of one layer's pool, the reference layout."""
    kb, vb = pool.get_key_buffer(layer_id), pool.get_value_buffer(layer_id)
    pages = kb.shape[0] // 16
    k = to_np(kb[:pages * 16].reshape(pages, 16, *kb.shape[1:]))
    v = to_np(vb[:pages * 16].reshape(pages, 16, *vb.shape[1:]))
    return np.stack([k, v], axis=1)


def _want_by_slots(q, pool, layer_id, r2t, rows, lens):
    """Attention of each request's q over its tokens gathered slot by slot from the
    request-to-token map (no page table), in float64: independent of how the pool is
    paged."""
    kb = to_np(pool.get_key_buffer(layer_id)).astype(np.float64)
    vb = to_np(pool.get_value_buffer(layer_id)).astype(np.float64)
    qn = to_np(q).astype(np.float64)
    hq, d = qn.shape[1], qn.shape[2]
    g = hq // kb.shape[1]
    out = np.zeros_like(qn)
    for b, (r, n) in enumerate(zip(rows, lens)):
        slots = np.asarray(r2t[r, :n], dtype=np.int64)
        for h in range(hq):
            s_ = kb[slots, h // g] @ qn[b, h] / math.sqrt(d)
            w = np.exp(s_ - s_.max())
            out[b, h] = (w / w.sum()) @ vb[slots, h // g]
    return out


def _want(q, pool, layer_id, r2t, rows, lens, scale_mult=1.0):
    indptr, indices, last = ptab.build_page_table(r2t, rows, lens)
    qn = to_np(q) * np.float32(scale_mult)
    return ref.reference_attention_paged(qn, _pool_as_combined(pool, layer_id), indptr,
                                         indices, last)


@pytest.mark.gpu
@pytest.mark.parametrize("lens,server_page", [
    ([1, 17, 300, 16, 1000, 33], 16), ([2048] * 12, 16), ([5], 16),
    ([1, 17, 300, 16, 1000, 33], 32), ([2048, 7, 64] * 3, 64)])
def test_device_page_table_matches_oracle(lens, server_page):
    fb, _, _, r2t = make_batch(lens, layers=1, seed=len(lens), server_page=server_page)
    rows = fb.req_pool_indices.tolist()
    print(f"[case] page table lens={lens[:4]}... server page {server_page}", flush=True)
    indptr, indices, last = paging.build_page_table(
        fb.req_to_token_pool.req_to_token, fb.req_pool_indices, fb.seq_lens,
        seq_lens_sum=fb.seq_lens_sum)
    torch.cuda.synchronize()
    wi, wx, wl = ptab.build_page_table(r2t.numpy(), rows, lens)
    assert indptr.cpu().tolist() == wi.tolist()
    assert last.cpu().tolist() == wl.tolist()
    assert indices[:int(wi[-1])].cpu().tolist() == wx.tolist()


@pytest.mark.gpu
def test_device_page_table_empty_requests_and_capacity_clamp():
    fb, _, _, r2t = make_batch([0, 40, 0, 16], layers=1, seed=9)
    rows = fb.req_pool_indices.tolist()
    indptr, indices, last = paging.build_page_table(
        fb.req_to_token_pool.req_to_token, fb.req_pool_indices, fb.seq_lens, capacity=2)
    torch.cuda.synchronize()
    wi, wx, wl = ptab.build_page_table(r2t.numpy(), rows, [0, 40, 0, 16])
    assert indptr.cpu().tolist() == wi.tolist() and last.cpu().tolist() == wl.tolist()
    assert indices.cpu().tolist() == wx[:2].tolist()     # writes past capacity are dropped


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,split_kv,server_page", [
    (dt, s, 16) for dt in (torch.float16, torch.bfloat16) for s in (0, 1, 4)] + [
    (torch.float16, 0, 32), (torch.bfloat16, 0, 64), (torch.float16, 4, 64)])
def test_decode_step_through_the_adapter(dtype, split_kv, server_page):
    """A decode step through SGLang's API; the server's pages hold 16 tokens or a
    multiple of 16 (each then read as aligned 16-token pages)."""
    lens = [1, 17, 300, 16, 1000, 33, 129]
    fb, layers, pool, r2t = make_batch(lens, dtype=dtype, seed=3, server_page=server_page)
    rows = fb.req_pool_indices.tolist()
    backend = sglang_backend.SplitKVHipBackend(split_kv=split_kv)
    backend.init_forward_metadata(fb)
    g = torch.Generator(device=DEV)
    g.manual_seed(5)
    for layer in layers:
        print(f"[case] adapter {dtype} split={split_kv} server page={server_page} "
              f"layer={layer.layer_id}", flush=True)
        q = torch.randn(len(lens), 32 * 128, generator=g, device=DEV).to(dtype)
        k = torch.randn(len(lens), 8 * 128, generator=g, device=DEV).to(dtype)
        v = torch.randn(len(lens), 8 * 128, generator=g, device=DEV).to(dtype)
        out = backend.forward(q, k, v, layer, fb)          # SGLang's positional call
        torch.cuda.synchronize()
        assert out.shape == (len(lens), 32 * 128)
        # the new token's K/V landed in the pool at out_cache_loc
        kb = pool.get_key_buffer(layer.layer_id)
        assert torch.equal(kb[fb.out_cache_loc.long()].reshape(len(lens), -1), k)
        want = _want(q.view(-1, 32, 128), pool, layer.layer_id, r2t.numpy(), rows, lens)
        mx, mean = err_stats(out.view(-1, 32, 128), want)
        assert mx <= 1e-2 and mean <= 1e-3, (mx, mean)
        if server_page != 16 or split_kv == 0:
            want = _want_by_slots(q.view(-1, 32, 128), pool, layer.layer_id, r2t.numpy(),
                                  rows, lens)
            mx, mean = err_stats(out.view(-1, 32, 128), want)
            assert mx <= 1e-2 and mean <= 1e-3, ("by slots", mx, mean)


@pytest.mark.gpu
def test_adapter_custom_scaling_and_reference_shim():
    lens = [64, 500, 3]
    fb, layers, pool, r2t = make_batch(lens, layers=1, seed=4)
    rows = fb.req_pool_indices.tolist()
    layer = layers[0]
    layer.scaling = 0.05                           # not 1/sqrt(128)
    backend = sglang_backend.SplitKVHipBackend()
    backend.init_forward_metadata(fb)
    q = torch.randn(3, 32 * 128, device=DEV).half()
    out = backend.forward_decode(q, None, None, layer, fb)
    torch.cuda.synchronize()
    # softmax(0.05 q.k) = softmax((0.05 sqrt(128) q).k / sqrt(128))
    want = _want(q.view(-1, 32, 128), pool, 0, r2t.numpy(), rows, lens,
                 scale_mult=0.05 * math.sqrt(128))
    mx, mean = err_stats(out.view(-1, 32, 128), want)
    assert mx <= 1e-2 and mean <= 1e-3, (mx, mean)
    # the reference shim's forward(q, kv_data, indptr, indices, last) on the same pool
    kv = torch.from_numpy(_pool_as_combined(pool, 0)).to(DEV).half()
    md = backend.forward_metadata
    o2 = backend.forward(q.view(-1, 32, 128), kv, md.kv_indptr, md.kv_indices,
                         md.kv_last_page_len)
    torch.cuda.synchronize()
    mx2, _ = err_stats(o2, _want(q.view(-1, 32, 128), pool, 0, r2t.numpy(), rows, lens))
    assert mx2 <= 1e-2


@pytest.mark.gpu
@pytest.mark.parametrize("split_kv", [1, 3, 0])
def test_split_caches_equal_combined_cache(split_kv):
    # the (k_cache, v_cache) form (separate buffers; V allocated first, so its offset from
    # K may be negative) gives the same result as the combined cache holding the same data
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        5, [100, 1, 4000, 0, 333], 32, 8, 128, device=DEV, page_table="permuted", seed=8)
    v_cache = kv[:, 1].clone()
    k_cache = kv[:, 0].clone()
    a = attention.decode_attention(q, kv, indptr, ids, last, split_kv=split_kv)
    b = attention.decode_attention(q, (k_cache, v_cache), indptr, ids, last, split_kv=split_kv)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.gpu
@pytest.mark.parametrize("scale", [0.02, 0.3])
def test_sm_scale_matches_prescaled_q(scale):
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        4, [700, 20, 1, 64], 32, 8, 64, device=DEV, page_table="permuted", seed=12)
    out = attention.decode_attention(q, kv, indptr, ids, last, split_kv=0, sm_scale=scale)
    torch.cuda.synchronize()
    want = ref.reference_attention_paged(to_np(q) * np.float32(scale * 8.0), to_np(kv),
                                         to_np(indptr), to_np(ids), to_np(last))
    mx, mean = err_stats(out, want)
    assert mx <= 1e-2 and mean <= 1e-3, (mx, mean)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fp8_pool_decode_step_through_the_adapter(dtype):
    # SGLang's fp8_e4m3 KV cache: the pool quantises k / k_scale and v / v_scale on write;
    # the adapter attends with the same scales
    from oracle import fp8
    lens = [1, 17, 300, 16, 1000, 33]
    ks, vs = 0.5, 0.25
    fb, layers, pool, r2t = make_batch(lens, dtype=dtype, seed=4, kv_dtype=torch.float8_e4m3fn,
                                       k_scale=ks, v_scale=vs)
    rows = fb.req_pool_indices.tolist()
    backend = sglang_backend.SplitKVHipBackend(split_kv=0)
    backend.init_forward_metadata(fb)
    g = torch.Generator(device=DEV)
    g.manual_seed(6)
    for layer in layers:
        print(f"[case] adapter fp8 pool {dtype} layer={layer.layer_id}", flush=True)
        q = torch.randn(len(lens), 32 * 128, generator=g, device=DEV).to(dtype)
        k = torch.randn(len(lens), 8 * 128, generator=g, device=DEV).to(dtype)
        v = torch.randn(len(lens), 8 * 128, generator=g, device=DEV).to(dtype)
        out = backend.forward_decode(q, k, v, layer, fb)
        torch.cuda.synchronize()
        kb = pool.get_key_buffer(layer.layer_id)
        assert kb.dtype == torch.float8_e4m3fn
        codes = np.stack([pool.k_buffer[layer.layer_id].cpu().numpy(),
                          pool.v_buffer[layer.layer_id].cpu().numpy()], axis=1)   # (slots, 2, ..)
        pages = codes.shape[0] // 16
        codes = codes[:pages * 16].reshape(pages, 16, 2, 8, 128).transpose(0, 2, 1, 3, 4)
        deq = np.stack([fp8.dequantize(codes[:, 0], ks), fp8.dequantize(codes[:, 1], vs)], 1)
        indptr, indices, last = ptab.build_page_table(r2t.numpy(), rows, lens)
        want = ref.reference_attention_paged(to_np(q.view(-1, 32, 128)).astype(np.float32),
                                             deq, indptr, indices, last)
        mx, mean = err_stats(out.view(-1, 32, 128), want)
        assert mx <= 1e-2 and mean <= 1e-3, (mx, mean)


@pytest.mark.gpu
@pytest.mark.parametrize("cap,win", [(None, None), (2.0, None), (None, 9), (2.0, 20)])
def test_softcap_layer_decode_and_extend(cap, win):
    # a Gemma-2-like layer (own softmax scale, logit soft-capping, sliding window) through
    # both entry points: decode on the HIP kernel, extend on the explicit PyTorch path
    lens = [5, 40, 17]
    n_new = [5, 3, 1]
    fb, layers, pool, r2t = make_batch(lens, layers=1, seed=7, decode=False)
    layer = layers[0]
    layer.scaling = 0.11
    layer.logit_cap = cap
    layer.sliding_window_size = -1 if win is None else win - 1     # SGLang's window_left
    rows = fb.req_pool_indices.tolist()
    g = torch.Generator(device=DEV)
    g.manual_seed(8)
    # extend: the last n_new tokens of each request are new
    locs = torch.cat([r2t[r, n - m:n] for r, n, m in zip(rows, lens, n_new)]).long()
    fb.out_cache_loc = locs.to(DEV)
    fb.extend_seq_lens_cpu = torch.tensor(n_new)
    T = sum(n_new)
    q = (torch.randn(T, 32 * 128, generator=g, device=DEV) * 2).half()
    k = torch.randn(T, 8 * 128, generator=g, device=DEV).half()
    v = torch.randn(T, 8 * 128, generator=g, device=DEV).half()
    backend = sglang_backend.SplitKVHipBackend()
    print(f"[case] softcap layer extend cap={cap} window={win}", flush=True)
    out = backend.forward_extend(q, k, v, layer, fb)
    torch.cuda.synchronize()
    kb, vb = to_np(pool.get_key_buffer(0)), to_np(pool.get_value_buffer(0))
    start = 0
    for r, n, m in zip(rows, lens, n_new):
        for i in range(m):
            p = n - m + i
            slots = r2t[r, :p + 1].long().numpy()[-(win or p + 1):]
            want = ref.reference_attention(to_np(q[start + i].view(1, 32, 128)),
                                           kb[slots][None], vb[slots][None],
                                           sm_scale=0.11, logit_cap=cap)
            mx, _ = err_stats(out[start + i].view(1, 32, 128), want)
            assert mx <= 1e-2, (r, i, mx)
        start += m
    # decode: one more step for every request through the kernel
    print(f"[case] softcap layer decode cap={cap} window={win}", flush=True)
    fb.forward_mode = type(fb.forward_mode)(True)
    backend.init_forward_metadata(fb)
    qd = (torch.randn(len(lens), 32 * 128, generator=g, device=DEV) * 2).half()
    o = backend.forward_decode(qd, None, None, layer, fb)
    torch.cuda.synchronize()
    indptr, indices, last = ptab.build_page_table(r2t.numpy(), rows, lens)
    want = ref.reference_attention_paged(to_np(qd.view(-1, 32, 128)), _pool_as_combined(pool, 0),
                                         indptr, indices, last, sm_scale=0.11, logit_cap=cap,
                                         window=win)
    mx, mean = err_stats(o.view(-1, 32, 128), want)
    assert mx <= 1e-2 and mean <= 1e-3, (mx, mean)


@pytest.mark.gpu
def test_hip_graph_capture_and_replay():
    # SGLang's graph runner: persistent page tables, the decode step captured once (two
    # layers, K/V writes included) and replayed for growing sequences; every replay is
    # checked against the oracle, with eager work and synchronisations between replays
    from types import SimpleNamespace
    full = [40, 17, 300, 5]
    fb, layers, pool, r2t = make_batch(full, seed=9)
    rows = fb.req_pool_indices
    mr = SimpleNamespace(req_to_token_pool=fb.req_to_token_pool, device=DEV,
                         model_config=SimpleNamespace(context_len=512))
    backend = sglang_backend.SplitKVHipBackend(mr)
    backend.init_cuda_graph_state(max_bs=8)
    bs = len(full)
    seq_lens = torch.tensor([n - 3 for n in full], dtype=torch.int64, device=DEV)   # static
    fb.seq_lens = seq_lens
    loc = torch.empty(bs, dtype=torch.int64, device=DEV)
    fb.out_cache_loc = loc
    q = torch.empty(bs, 32 * 128, dtype=torch.float16, device=DEV)
    k = torch.empty(bs, 8 * 128, dtype=torch.float16, device=DEV)
    v = torch.empty_like(k)

    def set_step(lens, seed):
        g = torch.Generator(device=DEV)
        g.manual_seed(seed)
        seq_lens.copy_(torch.tensor(lens, device=DEV))
        loc.copy_(torch.tensor([int(r2t[r, n - 1]) for r, n in zip(rows.tolist(), lens)],
                               device=DEV))
        q.copy_(torch.randn(q.shape, generator=g, device=DEV))
        k.copy_(torch.randn(k.shape, generator=g, device=DEV))
        v.copy_(torch.randn(v.shape, generator=g, device=DEV))

    set_step([n - 3 for n in full], 1)
    backend.init_forward_metadata_capture_cuda_graph(bs, bs, rows, seq_lens)
    for layer in layers:                        # warm-up outside the graph (allocations)
        backend.forward_decode(q, k, v, layer, fb)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = [backend.forward_decode(q, k, v, layer, fb) for layer in layers]
    for step, back in enumerate((2, 1, 0)):
        lens = [n - back for n in full]
        set_step(lens, 10 + step)
        backend.init_forward_metadata_replay_cuda_graph(bs, rows, seq_lens)
        print(f"[case] graph replay {step} lens={lens}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        for layer, o in zip(layers, outs):
            want = _want(q.view(-1, 32, 128), pool, layer.layer_id, r2t.numpy(), rows.tolist(),
                         lens)
            mx, mean = err_stats(o.view(-1, 32, 128), want)
            assert mx <= 1e-2 and mean <= 1e-3, (step, layer.layer_id, mx, mean)
            # the replay wrote this step's K into the pool
            kb = pool.get_key_buffer(layer.layer_id)
            assert torch.equal(kb[loc].reshape(bs, -1), k)
        # eager work between replays: an uncaptured decode of the same step agrees
        backend.init_forward_metadata(fb)
        eager = backend.forward_decode(q, None, None, layers[0], fb)
        torch.cuda.synchronize()
        assert float((eager.float() - outs[0].float()).abs().max()) <= 2e-3
        # ... and an eager batch larger than any captured one, whose workspace is larger:
        # the graph's workspace must stay the graph's (the next replay writes there while
        # these tensors are alive), and this batch's result must survive that replay
        big_fb, big_layers, big_pool, big_r2t = make_batch([700 + 13 * i for i in range(24)],
                                                           seed=20 + step)
        backend.init_forward_metadata(big_fb)
        qb = torch.randn(24, 32 * 128, generator=torch.Generator(device=DEV).manual_seed(step),
                         device=DEV).half()
        big = backend.forward_decode(qb, None, None, big_layers[0], big_fb)
        torch.cuda.synchronize()
        big_keep = big.clone()
        want_big = _want(qb.view(-1, 32, 128), big_pool, 0, big_r2t.numpy(),
                         big_fb.req_pool_indices.tolist(), [700 + 13 * i for i in range(24)])
        mx, mean = err_stats(big.view(-1, 32, 128), want_big)
        assert mx <= 1e-2 and mean <= 1e-3, ("large eager batch", mx, mean)
        backend.init_forward_metadata_replay_cuda_graph(bs, rows, seq_lens)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(big, big_keep), "a graph replay wrote into an eager tensor"
        del big_fb, big_layers, big_pool, big, big_keep


@pytest.mark.gpu
def test_sinks_layer_decode_and_extend():
    """gpt-oss-style attention sinks passed by SGLang's keyword: the decode step (HIP
    kernel) and the extend path (explicit attention) against the oracle's sink form."""
    lens = [5, 130, 700]
    fb, layers, pool, r2t = make_batch(lens, hq=16, hkv=4, d=64, layers=1, seed=8)
    rows = fb.req_pool_indices.tolist()
    layer = layers[0]
    sinks = (torch.randn(16) * 2).to(DEV).to(torch.bfloat16)    # the model's dtype
    backend = sglang_backend.SplitKVHipBackend()
    backend.init_forward_metadata(fb)
    q = torch.randn(len(lens), 16 * 64, device=DEV).half()
    print("[case] adapter sinks decode", flush=True)
    out = backend.forward(q, None, None, layer, fb, True, sinks=sinks)
    torch.cuda.synchronize()
    indptr, indices, last = ptab.build_page_table(r2t.numpy(), rows, lens)
    s32 = sinks.float().cpu().numpy()
    want = ref.reference_attention_paged(to_np(q.view(-1, 16, 64)).astype(np.float32),
                                         _pool_as_combined(pool, 0), indptr, indices, last,
                                         sinks=s32)
    mx, mean = err_stats(out.view(-1, 16, 64), want)
    assert mx <= 1e-2 and mean <= 1e-3, ("decode", mx, mean)
    # extend: the last 3 tokens of each request are new; each sees its prefix and itself
    print("[case] adapter sinks extend", flush=True)
    ext = [3, 3, 3]
    fb.forward_mode = type(fb.forward_mode)(False)
    fb.extend_seq_lens_cpu = ext
    qe = torch.randn(sum(ext), 16 * 64, device=DEV).half()
    oe = backend.forward_extend(qe, None, None, layer, fb, sinks=sinks).view(-1, 16, 64)
    torch.cuda.synchronize()
    kb, vb = pool.get_key_buffer(0).float().cpu(), pool.get_value_buffer(0).float().cpu()
    start = 0
    for r, n, e in zip(rows, lens, ext):
        for i in range(e):
            upto = n - e + i + 1                              # tokens this query sees
            slots = r2t[r, :upto].long()
            k, v = kb[slots].numpy(), vb[slots].numpy()      # (upto, Hkv, D)
            qi = to_np(qe[start + i].view(1, 16, 64)).astype(np.float32)
            w = ref.reference_attention(qi, k[None], v[None], sinks=s32)[0]
            got = oe[start + i].float().cpu().numpy()
            assert np.abs(got - w).max() <= 1e-2, (r, i)
        start += e
