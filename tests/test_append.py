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


# ---- fp8 (OCP E4M3) cache: dk_append_kv_fp8 against oracle/append.py append_kv_fp8

def _fp8_cache(kv):
    """An fp8 cache of random finite codes with kv's shape (and the uint8 view)."""
    g = torch.Generator(device=DEV)
    g.manual_seed(5)
    codes = torch.randint(0, 0x7F, kv.shape, generator=g, device=DEV, dtype=torch.int32)
    codes = codes.to(torch.uint8) | (torch.randint(0, 2, kv.shape, generator=g, device=DEV,
                                                   dtype=torch.int32) * 0x80).to(torch.uint8)
    return codes.view(torch.float8_e4m3fn), codes


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fp8_append_rounds_every_value_and_tie_like_the_oracle(dtype):
    # V rows (no rotation, v_scale 1) hold every finite E4M3 value, every midpoint between
    # neighbours (ties: round to even), values beyond +-448 (clamped) and NaN
    from oracle import fp8
    vals = np.unique(fp8.decode(np.arange(0x7F)))
    mids = (vals[1:] + vals[:-1]) / 2
    pool = np.concatenate([vals, -vals, mids, -mids, [470.0, -1000.0, 60000.0, np.nan]])
    if dtype == torch.bfloat16:     # bf16 keeps only the values it represents exactly
        pool = pool[torch.from_numpy(pool).to(dtype).double().numpy() == pool]
    batch, hkv, d = 8, 1, 64
    lens = [1 + 16 * b for b in range(batch)]
    q, kv, indptr, ids, last, _, _ = _inputs(dtype, lens, hkv=hkv, d=d, seed=11)
    flat = np.resize(pool, batch * hkv * d).reshape(batch, hkv, d)
    v_new = torch.from_numpy(flat).to(dtype).to(DEV)
    k_new = torch.zeros_like(v_new)
    cache, codes = _fp8_cache(kv)
    before = codes.cpu().numpy()
    print(f"[case] fp8 append rounding {dtype}", flush=True)
    paging.append_kv(None, k_new, v_new, cache, indptr, ids, last, k_scale=1.0, v_scale=1.0)
    torch.cuda.synchronize()
    want, _ = oapp.append_kv_fp8(before, None, to_np(k_new), to_np(v_new), to_np(indptr),
                                 to_np(ids), to_np(last), 1.0, 1.0)
    got = codes.cpu().numpy()
    nan_w = np.isnan(fp8.decode(want))
    assert np.array_equal(np.isnan(fp8.decode(got)), nan_w)
    assert np.array_equal(got[~nan_w], want[~nan_w])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("split_cache", [False, True])
def test_fp8_append_with_rope_and_scales(dtype, split_cache):
    from oracle import fp8
    lens = [1, 16, 17, 0, 300, 2047]
    q, kv, indptr, ids, last, k_new, v_new = _inputs(dtype, lens, seed=13 + split_cache)
    k_new = k_new * 40                                    # some values beyond 448 * k_scale
    inv = paging.rope_inv_freq(64, theta=500000.0)
    cache, codes = _fp8_cache(kv)
    before, q_before = codes.cpu().numpy(), to_np(q)
    ks, vs = 0.0625, 0.37
    print(f"[case] fp8 append rope {dtype} split={split_cache}", flush=True)
    if split_cache:
        kc, vc = cache[:, 0].clone(), cache[:, 1].clone()
        paging.append_kv(q, k_new, v_new, (kc, vc), indptr, ids, last, inv_freq=inv,
                         k_scale=ks, v_scale=vs)
        got = torch.stack([kc.view(torch.uint8), vc.view(torch.uint8)], dim=1).cpu().numpy()
    else:
        paging.append_kv(q, k_new, v_new, cache, indptr, ids, last, inv_freq=inv,
                         k_scale=ks, v_scale=vs)
        got = codes.cpu().numpy()
    torch.cuda.synchronize()
    want, want_q = oapp.append_kv_fp8(before, q_before, to_np(k_new), to_np(v_new),
                                      to_np(indptr), to_np(ids), to_np(last), ks, vs,
                                      inv_freq=to_np(inv))
    _close(q, want_q, dtype)
    # V is not rotated: exact. K: the rotation runs in fp32 with sincosf on the device and
    # in float64 in the oracle, so a value next to a rounding boundary may land on the
    # neighbouring code; never further.
    np.testing.assert_array_equal(got[:, 1], want[:, 1])
    step = np.abs(fp8.signed_rank(got[:, 0]) - fp8.signed_rank(want[:, 0]))
    assert step.max() <= 1 and (step > 0).mean() < 0.01
    assert not np.isnan(fp8.decode(got)).any()          # values beyond 448 are clamped


def test_fp8_append_then_decode_matches_oracle():
    from oracle import fp8
    from oracle import reference as ref
    import attention
    lens = [33, 700, 5]
    q, kv, indptr, ids, last, k_new, v_new = _inputs(torch.float16, lens, hq=32, hkv=8, d=128,
                                                     seed=21)
    cache, codes = _fp8_cache(kv)
    cache.view(torch.uint8).copy_(torch.from_numpy(fp8.encode_saturating(
        to_np(kv).astype(np.float32) / np.float32(0.5))).to(DEV))
    inv = paging.rope_inv_freq(128)
    print("[case] fp8 append then decode", flush=True)
    paging.append_kv(q, k_new, v_new, cache, indptr, ids, last, inv_freq=inv, k_scale=0.5,
                     v_scale=0.5)
    out = attention.decode_attention(q, cache, indptr, ids, last, split_kv=0, k_scale=0.5,
                                     v_scale=0.5)
    torch.cuda.synchronize()
    deq = fp8.dequantize(codes.cpu().numpy(), 0.5)
    want = ref.reference_attention_paged(to_np(q).astype(np.float32), deq, to_np(indptr),
                                         to_np(ids), to_np(last))
    err = np.abs(out.float().cpu().numpy() - want).max()
    assert err <= 1e-2, err
