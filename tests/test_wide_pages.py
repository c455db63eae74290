"""Caches with pages of a multiple of 16 tokens (FlashInfer allows any page size; the
reference checks page_size == 16, src/cuda_/attention_ext.cu:508,551): the page table is
rewritten over 16-token sub-pages (dk_expand_page_table) and decode_attention reads the
same memory as 16-token pages.

CPU: the oracle's expansion (oracle/page_table.expand_page_table) is pinned by a
hand-worked table and by token order -- the sub-page table over the 16-token view must
gather exactly the token rows the original table gathers from the original cache -- with a
planted mistake that this check catches; the C ABI rejects bad arguments before any device
call. GPU: the kernel's table equals the oracle's bit for bit, and decode_attention over
pages of 32 / 64 / 128 tokens (combined cache and K/V pair, fp16 / bf16 / fp8, automatic
and explicit splits) matches the fp32 oracle run on the original layout.
"""
import ctypes

import numpy as np
import pytest
import torch

import attention
import dk_lib
import paging
from helpers import err_stats, to_np
from oracle import fp8
from oracle import page_table as ptab
from oracle import reference as ref

DEV = "cuda"
INVALID = 2**31 - 1


def _random_table(rng, batch, page_size, num_pages, bad_ids=False):
    """Ragged CSR table over a pool of num_pages pages: some empty sequences, last-page
    lengths over [0, page_size] (0 included: the sequence ends at the page before)."""
    n = [int(x) if rng.random() > 0.2 else 0 for x in rng.integers(1, 9, size=batch)]
    indptr = np.concatenate([[0], np.cumsum(n)]).astype(np.int32)
    ids = rng.permutation(num_pages)[:indptr[-1]].astype(np.int32) if indptr[-1] <= num_pages \
        else rng.integers(0, num_pages, size=indptr[-1]).astype(np.int32)
    if bad_ids and len(ids):
        ids[rng.integers(0, len(ids), size=max(1, len(ids) // 8))] = num_pages + 3
    last = rng.integers(0, page_size + 1, size=batch).astype(np.int32)
    last[rng.random(batch) < 0.3] = page_size
    return indptr, ids, last


def _view16(kv, page_size):
    """numpy counterpart of decode_attention's 16-token view of a contiguous combined
    cache (N, 2, P, Hkv, D): page stride 16 rows, K/V stride unchanged."""
    n = kv.shape[0]
    s = page_size // 16
    row = kv.strides[2]
    mult = kv.strides[0] // (16 * row)
    shape = ((n - 1) * mult + s, 2, 16) + kv.shape[3:]
    strides = (16 * row,) + kv.strides[1:]
    return np.lib.stride_tricks.as_strided(kv, shape=shape, strides=strides), mult


# ---------------------------------------------------------------- CPU: the oracle

def test_expand_known_answer():
    # P = 32 (two sub-pages per page), combined cache: sub-page j of page p is 4 p + j
    indptr, indices, last = ptab.expand_page_table(
        [0, 2, 2, 4, 5], [5, 1, 7, 9, 3], [17, 5, 32, 0], 32, 4, 8)
    assert indptr.tolist() == [0, 4, 4, 8, 8]
    assert indices.tolist() == [20, 21, 4, 5, 28, 29, INVALID, INVALID]   # page 9 is past the pool
    assert last.tolist() == [1, 0, 16, 0]   # 17 = 16 + 1; empty; 32 = two full; last 0, one page


def test_expand_overlapping_indptr_saturates_at_capacity():
    # kv_indptr [0, 4, 0, 4] is clamped entry by entry: sequence 1 is empty and sequence 2
    # covers all four pages again, 16 sub-pages for a table of capacity 4 * 2 = 8
    indptr, indices, last = ptab.expand_page_table([0, 4, 0, 4], [3, 0, 2, 1], [32, 5, 32],
                                                   32, 2, 4)
    assert indptr.tolist() == [0, 8, 8, 8]
    assert indices.tolist() == [6, 7, 0, 1, 4, 5, 2, 3]     # sequence 0's, then full
    assert last.tolist() == [16, 0, 16]


@pytest.mark.parametrize("page_size", [32, 64, 128])
@pytest.mark.parametrize("seed", range(4))
def test_expansion_gathers_the_same_tokens(page_size, seed):
    """Token order pins the expansion: over the 16-token view, the expanded table gathers
    the same rows, in the same order and number, as the original table over the cache."""
    rng = np.random.default_rng(seed)
    num_pages = 40
    kv = rng.standard_normal((num_pages, 2, page_size, 2, 3)).astype(np.float32)
    indptr, ids, last = _random_table(rng, 9, page_size, num_pages)
    view, mult = _view16(kv, page_size)
    e_ptr, e_ids, e_last = ptab.expand_page_table(indptr, ids, last, page_size, mult, num_pages)
    assert (ref.seq_lens_of(e_ptr, e_last, 16) == ref.seq_lens_of(indptr, last, page_size)).all()
    k0, v0 = ref.gather_paged_to_dense(kv, indptr, ids, last)
    k1, v1 = ref.gather_paged_to_dense(view, e_ptr, e_ids, e_last)
    assert np.array_equal(k0, k1) and np.array_equal(v0, v1)
    # a planted mistake fails the same check: the last sub-page's tokens as last % 16
    bad_last = np.where(e_last == 16, 0, e_last)
    if (bad_last != e_last).any():
        assert not (ref.seq_lens_of(e_ptr, bad_last, 16) ==
                    ref.seq_lens_of(indptr, last, page_size)).all()


def test_expansion_of_separate_caches_uses_their_page_stride():
    """K / V caches of (N, P, Hkv, D): a page is s sub-pages, so ids are p * s + j."""
    rng = np.random.default_rng(7)
    P, N = 64, 12
    k = rng.standard_normal((N, P, 1, 2)).astype(np.float32)
    v = rng.standard_normal((N, P, 1, 2)).astype(np.float32)
    indptr, ids, last = _random_table(rng, 5, P, N)
    e_ptr, e_ids, e_last = ptab.expand_page_table(indptr, ids, last, P, P // 16, N)
    comb = np.stack([k, v], axis=1)                                    # (N, 2, P, 1, 2)
    k16, v16 = k.reshape(N * P // 16, 16, 1, 2), v.reshape(N * P // 16, 16, 1, 2)
    comb16 = np.stack([k16, v16], axis=1)
    a = ref.gather_paged_to_dense(comb, indptr, ids, last)
    b = ref.gather_paged_to_dense(comb16, e_ptr, e_ids, e_last)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))


# ---------------------------------------------------------------- CPU: the C ABI

@pytest.mark.parametrize("kw,needle", [
    (dict(page_size=24), "multiple of 16"),
    (dict(page_size=0), "multiple of 16"),
    (dict(pages_mult=1), "pages_mult"),
    (dict(batch=-1), "negative"),
    (dict(capacity=-1), "negative"),
    (dict(num_pages=2**30, pages_mult=4), "2^31"),
    (dict(num_indices=2**30, page_size=64, pages_mult=8), "sub-pages exceed"),
    (dict(num_pages=2**62, pages_mult=4), "num_pages must be < 2^31"),   # no wrapped product
])
def test_expand_rejects_bad_arguments_before_launch(kw, needle):
    lib = dk_lib.load()
    a = dict(batch=2, page_size=32, pages_mult=4, num_pages=8, num_indices=4, capacity=8)
    a.update(kw)
    fake = ctypes.c_void_p(16)      # never dereferenced: the checks come first
    rc = lib.dk_expand_page_table(fake, fake, fake, a["batch"], a["page_size"],
                                  a["pages_mult"], a["num_pages"], a["num_indices"], fake,
                                  fake, a["capacity"], fake, None)
    assert rc == dk_lib.DK_EINVAL
    assert needle in lib.dk_last_error().decode()
    # batch 0 is a no-op that touches nothing
    assert lib.dk_expand_page_table(None, None, None, 0, 32, 4, 8, 0, None, None, 0, None,
                                    None) == 0


def test_wide_page_tables_are_checked_before_the_expansion():
    """The expansion kernel reads the three tables on the GPU: host tables and a
    kv_last_page_len shorter than the batch are refused on the host, before any launch."""
    t5, t4, t3 = (torch.zeros(n, dtype=torch.int32) for n in (5, 4, 3))
    with pytest.raises(dk_lib.DecodeArgumentError, match="one entry per sequence"):
        paging.expand_page_table(t5, t4, t3, 32, 2, 4)
    with pytest.raises(dk_lib.DecodeArgumentError, match="on one GPU"):
        paging.expand_page_table(t5, t4, t4, 32, 2, 4)
    q = torch.zeros(4, 8, 64, dtype=torch.float16)
    kv = torch.zeros(4, 2, 32, 2, 64, dtype=torch.float16)
    for fn in (attention.decode_attention, attention.DecodePlan):
        with pytest.raises(dk_lib.DecodeArgumentError, match="CUDA"):
            fn(q, kv, t5, t4, t4)


def test_page_sizes_not_a_multiple_of_sixteen_are_refused():
    q = torch.zeros(1, 4, 64, dtype=torch.float16)
    kv = torch.zeros(2, 2, 24, 1, 64, dtype=torch.float16)
    t = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(dk_lib.DecodeArgumentError, match="page_size"):
        attention.decode_attention(q, kv, t, t[:1], t[:1])


# ---------------------------------------------------------------- GPU

@pytest.mark.gpu
@pytest.mark.parametrize("page_size,mult", [(32, 4), (64, 8), (128, 16), (64, 4)])
@pytest.mark.parametrize("seed", range(3))
def test_device_expansion_matches_oracle(page_size, mult, seed):
    rng = np.random.default_rng(100 + seed)
    num_pages = 50
    indptr, ids, last = _random_table(rng, 300, page_size, num_pages, bad_ids=True)
    print(f"[case] expand P={page_size} mult={mult} seed={seed}", flush=True)
    to = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    d_ptr, d_ids, d_last = paging.expand_page_table(to(indptr), to(ids), to(last), page_size,
                                                    mult, num_pages)
    torch.cuda.synchronize()
    w_ptr, w_ids, w_last = ptab.expand_page_table(indptr, ids, last, page_size, mult, num_pages)
    assert d_ptr.cpu().numpy().tolist() == w_ptr.tolist()
    assert d_last.cpu().numpy().tolist() == w_last.tolist()
    assert d_ids[:int(w_ptr[-1])].cpu().numpy().tolist() == w_ids.tolist()


@pytest.mark.gpu
def test_device_expansion_of_overlapping_ranges_stays_in_its_table():
    """kv_indptr whose clamped ranges overlap (each of 40 sequences covering the whole
    index range): the offsets saturate at the capacity and nothing is written past it,
    as the oracle states."""
    rng = np.random.default_rng(5)
    n, batch, num_pages = 64, 40, 80
    indptr = np.array([0, n] * (batch // 2) + [0], np.int32)
    ids = rng.permutation(num_pages)[:n].astype(np.int32)
    last = rng.integers(1, 65, size=batch).astype(np.int32)
    print("[case] expand overlapping kv_indptr", flush=True)
    to = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    d_ptr, d_ids, d_last = paging.expand_page_table(to(indptr), to(ids), to(last), 64, 4,
                                                    num_pages)
    torch.cuda.synchronize()
    w_ptr, w_ids, w_last = ptab.expand_page_table(indptr, ids, last, 64, 4, num_pages)
    assert int(w_ptr[-1]) == n * 4 == d_ids.shape[0]
    assert d_ptr.cpu().numpy().tolist() == w_ptr.tolist()
    assert d_last.cpu().numpy().tolist() == w_last.tolist()
    assert d_ids.cpu().numpy().tolist() == w_ids.tolist()


@pytest.mark.gpu
def test_wide_pages_refuse_host_tables_and_short_last_page_len():
    """A 32-token cache on the GPU with a host kv_indices, or a kv_last_page_len shorter
    than the batch: decode_attention and DecodePlan raise before the expansion launches."""
    lens = [40, 70, 33]
    q, kv, indptr, ids, last = _wide_inputs(len(lens), lens, 32, 16, 4, 64, torch.float16,
                                            seed=2)
    qd, kd, ipd, idd, lad = (t.to(DEV) for t in (q, kv, indptr, ids, last))
    print("[case] wide pages bad tables", flush=True)
    for fn in (attention.decode_attention, attention.DecodePlan):
        with pytest.raises(dk_lib.DecodeArgumentError, match="kv_indices must be on"):
            fn(qd, kd, ipd, ids, lad)
        with pytest.raises(dk_lib.DecodeArgumentError, match="one entry per sequence"):
            fn(qd, kd, ipd, idd, lad[:2])
    plan = attention.DecodePlan(qd, kd, ipd, idd, lad)
    with pytest.raises(dk_lib.DecodeArgumentError):
        plan.run(qd, kd, ipd, idd.cpu(), lad)
    with pytest.raises(dk_lib.DecodeArgumentError):
        plan.run(qd, kd, ipd, idd, lad[:2])
    torch.cuda.synchronize()


def _wide_inputs(batch, lens, page_size, hq, hkv, d, dtype, seed):
    """q and a combined cache of `page_size`-token pages (random page order), with the
    page table; lens in tokens."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    npg = [-(-n // page_size) for n in lens]
    pool = sum(npg) + 5
    kv = torch.randn(pool, 2, page_size, hkv, d, generator=g).to(dtype)
    q = (torch.randn(batch, hq, d, generator=g) * d ** -0.5 * 4).to(dtype)
    perm = torch.randperm(pool, generator=g)[:sum(npg)].to(torch.int32)
    indptr = torch.tensor([0] + np.cumsum(npg).tolist(), dtype=torch.int32)
    last = torch.tensor([n - (p - 1) * page_size if p else 0 for n, p in zip(lens, npg)],
                        dtype=torch.int32)
    return q, kv, indptr, perm, last


@pytest.mark.gpu
@pytest.mark.parametrize("page_size", [32, 64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("split", [0, 1, 3])
def test_decode_over_wide_pages_matches_oracle(page_size, dtype, split):
    lens = [1, 15, 16, 17, 31, 32, 33, 100, 1000, 2048, 0, 513]
    b = len(lens)
    q, kv, indptr, ids, last = _wide_inputs(b, lens, page_size, 32, 8, 128, dtype,
                                            seed=page_size + split)
    print(f"[case] wide pages P={page_size} {dtype} split={split}", flush=True)
    want = ref.reference_attention_paged(to_np(q).astype(np.float32),
                                         to_np(kv).astype(np.float32), indptr.numpy(),
                                         ids.numpy(), last.numpy())
    hint = int((indptr[1:] - indptr[:-1]).max())
    out = attention.decode_attention(q.to(DEV), kv.to(DEV), indptr.to(DEV), ids.to(DEV),
                                     last.to(DEV), split_kv=split,
                                     max_pages_per_seq=hint if split == 0 else 0)
    torch.cuda.synchronize()
    rows = [i for i, n in enumerate(lens) if n > 0]
    mx, mean = err_stats(out[rows], want[rows])
    assert mx <= 1e-2 and mean <= 1e-3, (mx, mean)
    assert torch.count_nonzero(out[[i for i, n in enumerate(lens) if n == 0]]).item() == 0


@pytest.mark.gpu
@pytest.mark.parametrize("page_size", [32, 64])
def test_decode_over_wide_pages_kv_pair_and_fp8(page_size):
    """(k_cache, v_cache) of (N, P, Hkv, D), and an fp8 combined cache, over wide pages;
    D = 64 and a GQA group of 4."""
    lens = [70, 3, 400, 129, 64]
    q, kv, indptr, ids, last = _wide_inputs(len(lens), lens, page_size, 16, 4, 64,
                                            torch.float16, seed=3)
    want = ref.reference_attention_paged(to_np(q).astype(np.float32),
                                         to_np(kv).astype(np.float32), indptr.numpy(),
                                         ids.numpy(), last.numpy())
    qd, kd = q.to(DEV), kv.to(DEV)
    tabs = (indptr.to(DEV), ids.to(DEV), last.to(DEV))
    print(f"[case] wide pages pair P={page_size}", flush=True)
    kc, vc = kd[:, 0].contiguous(), kd[:, 1].contiguous()
    out = attention.decode_attention(qd, (kc, vc), *tabs, split_kv=0)
    torch.cuda.synchronize()
    mx, mean = err_stats(out, want)
    assert mx <= 1e-2 and mean <= 1e-3, ("pair", mx, mean)
    # fp8 E4M3 combined cache with scales, against the oracle on the dequantised values
    print(f"[case] wide pages fp8 P={page_size}", flush=True)
    ks, vs = 0.5, 0.25
    x = kv.float().numpy()
    codes = np.empty(x.shape, np.uint8)
    codes[:, 0] = fp8.encode(np.clip(x[:, 0] / ks, -448, 448))
    codes[:, 1] = fp8.encode(np.clip(x[:, 1] / vs, -448, 448))
    vals = np.empty(x.shape, np.float32)
    vals[:, 0] = fp8.dequantize(codes[:, 0], ks)
    vals[:, 1] = fp8.dequantize(codes[:, 1], vs)
    want8 = ref.reference_attention_paged(to_np(q).astype(np.float32), vals, indptr.numpy(),
                                          ids.numpy(), last.numpy())
    k8 = torch.from_numpy(codes).to(DEV).view(torch.float8_e4m3fn)
    out8 = attention.decode_attention(qd, k8, *tabs, split_kv=2, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    mx, mean = err_stats(out8, want8)
    assert mx <= 1e-2 and mean <= 1e-3, ("fp8", mx, mean)


@pytest.mark.gpu
def test_sixteen_token_pages_once_for_many_layers():
    """The table rewritten once (sixteen_token_pages) and reused by every layer's call on
    its own cache view gives what decode_attention gives on the wide pages directly."""
    lens = [300, 65, 1000]
    q, kv, indptr, ids, last = _wide_inputs(len(lens), lens, 64, 32, 8, 128, torch.float16,
                                            seed=11)
    qd, tabs = q.to(DEV), (indptr.to(DEV), ids.to(DEV), last.to(DEV))
    layers = [kv.to(DEV), (kv * 0.5).to(DEV)]
    print("[case] sixteen_token_pages reuse", flush=True)
    _, e_ptr, e_ids, e_last = attention.sixteen_token_pages(layers[0], *tabs)
    for layer_kv in layers:
        view, _, _, _ = attention.sixteen_token_pages(layer_kv)
        assert view.data_ptr() == layer_kv.data_ptr() and view.shape[2] == 16
        a = attention.decode_attention(qd, view, e_ptr, e_ids, e_last, split_kv=0)
        b = attention.decode_attention(qd, layer_kv, *tabs, split_kv=0)
        torch.cuda.synchronize()
        assert torch.equal(a, b)


@pytest.mark.gpu
def test_decode_plan_over_wide_pages():
    """DecodePlan over 64-token pages (planned over the 16-token view, the table rewritten
    by each run) gives decode_attention's output, layer after layer."""
    lens = [300, 65, 1000, 16]
    q, kv, indptr, ids, last = _wide_inputs(len(lens), lens, 64, 32, 8, 128, torch.bfloat16,
                                            seed=13)
    qd, tabs = q.to(DEV), (indptr.to(DEV), ids.to(DEV), last.to(DEV))
    layers = [kv.to(DEV), (kv * 0.5).to(DEV)]
    hint = int((indptr[1:] - indptr[:-1]).max())
    print("[case] DecodePlan over 64-token pages", flush=True)
    plan = attention.DecodePlan(qd, layers[0], *tabs, split_kv=0, max_pages_per_seq=hint)
    # the table rewritten once for all layers, each run over a layer's 16-token view
    _, *tabs16 = attention.sixteen_token_pages(layers[0], *tabs)
    for layer_kv in layers:
        got = plan.run(qd, layer_kv, *tabs)
        view, *_ = attention.sixteen_token_pages(layer_kv)
        got16 = plan.run(qd, view, *tabs16)
        want = attention.decode_attention(qd, layer_kv, *tabs, split_kv=0,
                                          max_pages_per_seq=hint)
        torch.cuda.synchronize()
        assert torch.equal(got, want) and torch.equal(got16, want)
