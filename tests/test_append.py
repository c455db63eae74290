"""GPU tests of the cache write before a decode step (dk_append_kv) against the oracle
(oracle/append.py): the new token's K (rotated) and V land in the slot the page table
names, q is rotated in place, nothing else in the cache changes."""
import numpy as np
import pytest
import torch

import layout
import paging
from helpers import to_np
from oracle import append as oapp

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(dtype, lens, hq=8, hkv=2, d=64, seed=0):
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        len(lens), lens, hq, hkv, d, dtype=dtype, device=DEV, page_table="permuted", seed=seed)
    g = torch.Generator(device=DEV)
    g.manual_seed(seed + 100)
    k_new = torch.randn(len(lens), hkv, d, generator=g, device=DEV).to(dtype)
    v_new = torch.randn(len(lens), hkv, d, generator=g, device=DEV).to(dtype)
    return q, kv, indptr, ids, last, k_new, v_new


def _close(got, want, dtype):
    rtol = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10   # one rounding of the result
    np.testing.assert_allclose(to_np(got), want, rtol=rtol, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("style", [0, 1])
@pytest.mark.parametrize("split_cache", [False, True])
def test_append_with_rope_matches_oracle(dtype, style, split_cache):
    lens = [1, 16, 17, 0, 300, 2047]
    q, kv, indptr, ids, last, k_new, v_new = _inputs(dtype, lens, seed=style + 2 * split_cache)
    print(f"[case] append {dtype} style={style} split={split_cache}", flush=True)
    inv = paging.rope_inv_freq(64, theta=500000.0)
    kv_before, q_before = to_np(kv), to_np(q)
    if split_cache:
        k_cache, v_cache = kv[:, 0].clone(), kv[:, 1].clone()
        paging.append_kv(q, k_new, v_new, (k_cache, v_cache), indptr, ids, last,
                         inv_freq=inv, rope_style=style)
        got = torch.stack([k_cache, v_cache], dim=1)
    else:
        paging.append_kv(q, k_new, v_new, kv, indptr, ids, last, inv_freq=inv, rope_style=style)
        got = kv
    torch.cuda.synchronize()
    want_kv, want_q = oapp.append_kv(kv_before, q_before, to_np(k_new), to_np(v_new),
                                     to_np(indptr), to_np(ids), to_np(last),
                                     inv_freq=to_np(inv), style=style)
    _close(got, want_kv, dtype)
    _close(q, want_q, dtype)
    # V rows are copied bit for bit; untouched slots keep their bits
    got_np, before = to_np(got), kv_before
    changed = np.any(got_np != before, axis=(1, 3, 4))          # (pages, 16)
    ip, ix, ll = to_np(indptr), to_np(ids), to_np(last)
    expect = np.zeros_like(changed)
    for b in range(len(lens)):
        if ip[b + 1] > ip[b]:
            expect[ix[ip[b + 1] - 1], ll[b] - 1] = True
            assert np.array_equal(got_np[ix[ip[b + 1] - 1], 1, ll[b] - 1], to_np(v_new[b]))
    assert np.array_equal(changed & ~expect, np.zeros_like(changed))


def test_append_without_rope_copies_and_explicit_positions():
    lens = [5, 40]
    q, kv, indptr, ids, last, k_new, v_new = _inputs(torch.float16, lens, seed=7)
    q0 = q.clone()
    paging.append_kv(q, k_new, v_new, kv, indptr, ids, last)           # no rotation
    torch.cuda.synchronize()
    assert torch.equal(q, q0)
    ip, ix, ll = to_np(indptr), to_np(ids), to_np(last)
    for b in range(2):
        assert torch.equal(kv[ix[ip[b + 1] - 1], 0, ll[b] - 1], k_new[b])
    # explicit positions override the in-sequence index
    q, kv, indptr, ids, last, k_new, v_new = _inputs(torch.float16, lens, seed=8)
    inv = paging.rope_inv_freq(64)
    pos = torch.tensor([1000, 3], dtype=torch.int32, device=DEV)
    kv_before, q_before = to_np(kv), to_np(q)
    paging.append_kv(q, k_new, v_new, kv, indptr, ids, last, inv_freq=inv, positions=pos)
    torch.cuda.synchronize()
    want_kv, want_q = oapp.append_kv(kv_before, q_before, to_np(k_new), to_np(v_new),
                                     to_np(indptr), to_np(ids), to_np(last),
                                     inv_freq=to_np(inv), positions=[1000, 3])
    _close(kv, want_kv, torch.float16)
    _close(q, want_q, torch.float16)
