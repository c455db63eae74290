"""Attention sinks (gpt-oss style; dk_options.sinks / decode_attention(sinks=...)): each q
head's softmax has one more logit, with no value. The HIP path against the fp32 oracle
(whose sink form is pinned against transformers' gpt-oss eager attention in
tests/test_oracle.py) on every place that normalises an output: one pass (one and several
wavefronts per workgroup, VALU and MFMA q.k head layouts, D = 64, 128 and 256), explicit
splits (merge kernel), the balanced schedule (direct writes and merges), an fp8 cache, a
sliding window, soft-capped scores (logit_cap) together with sinks, empty and one-token
sequences, and a sink that dominates every score.
"""
import numpy as np
import pytest
import torch

import attention
import layout
from helpers import err_stats, to_np
from oracle import fp8
from oracle import reference as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(lens, hq, hkv, d, dtype, seed):
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        len(lens), lens, hq, hkv, d, dtype=dtype, device=DEV, page_table="freelist",
        pool_pages=sum((n + 15) // 16 for n in lens) + 5, seed=seed, q_scale=d ** -0.5 * 4)
    return q, kv, indptr, ids, last


def _check(out, want, lens, dtype, label):
    rows = [b for b, n in enumerate(lens) if n > 0]
    half_ulp = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    d = np.abs(out[rows].float().cpu().numpy().astype(np.float64) - want[rows])
    mx, mean = err_stats(out[rows], want[rows])
    assert (d <= 1e-2 + half_ulp * np.abs(want[rows])).all() and mean <= 1e-3, (label, mx, mean)
    empty = [b for b, n in enumerate(lens) if n == 0]
    if empty:
        assert torch.count_nonzero(out[empty]).item() == 0, label


CASES = [
    # (label, hq, hkv, d, split, extra decode_attention options)
    ("one pass NW=2", 32, 8, 128, 1, {}),
    ("one pass NW=1", 32, 8, 128, 1, dict(waves_per_group=1)),
    ("one pass NW=4 D=64", 32, 8, 64, 1, {}),
    ("one pass MFMA q.k 64/8", 64, 8, 128, 1, {}),
    ("split 3", 32, 8, 128, 3, {}),
    ("split 5 MFMA q.k", 64, 8, 128, 5, {}),
    ("balanced", 32, 8, 128, 0, {}),
    ("balanced D=64 grouped", 32, 8, 64, 0, {}),
    ("automatic with hint", 32, 8, 128, 0, dict(hint=True)),
    ("window 100", 32, 8, 128, 0, dict(window=100)),
    ("one pass D=256", 16, 4, 256, 1, {}),
    ("balanced D=256", 16, 4, 256, 0, {}),
    ("one pass logit_cap", 32, 8, 128, 1, dict(logit_cap=20.0)),
    ("balanced logit_cap", 32, 8, 128, 0, dict(logit_cap=20.0)),
    ("split 3 D=256 logit_cap", 16, 4, 256, 3, dict(logit_cap=15.0)),
    ("balanced MFMA q.k logit_cap", 64, 8, 128, 0, dict(logit_cap=20.0)),
]


@pytest.mark.parametrize("label,hq,hkv,d,split,extra", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_sinks_match_oracle(label, hq, hkv, d, split, extra, dtype):
    lens = [1, 40, 300, 0, 1000, 17, 512, 2]
    q, kv, indptr, ids, last = _inputs(lens, hq, hkv, d, dtype, seed=hq + d + split)
    g = torch.Generator(device="cpu")
    g.manual_seed(7)
    sinks = torch.randn(hq, generator=g) * 2
    sinks[3] = 30.0                                  # a head whose sink outweighs every score
    print(f"[case] sinks {label} {dtype}", flush=True)
    extra = dict(extra)
    hint = attention.plan_hint(indptr.cpu()) if extra.pop("hint", False) else 0
    out = attention.decode_attention(q, kv, indptr, ids, last, split_kv=split,
                                     sinks=sinks.to(DEV), max_pages_per_seq=hint, **extra)
    torch.cuda.synchronize()
    want = ref.reference_attention_paged(to_np(q).astype(np.float32),
                                         to_np(kv).astype(np.float32), to_np(indptr),
                                         to_np(ids), to_np(last), sinks=sinks.numpy(),
                                         window=extra.get("window"),
                                         logit_cap=extra.get("logit_cap"))
    _check(out, want, lens, dtype, label)
    assert out[:, 3].abs().max().item() < 1e-6      # the dominant sink leaves ~nothing


def test_sinks_over_fp8_cache_and_pass1_only_partials_stay_plain():
    lens = [64, 333, 5]
    q, kv, indptr, ids, last = _inputs(lens, 32, 8, 128, torch.float16, seed=9)
    x = kv.float().cpu().numpy()
    codes = fp8.encode(np.clip(x, -448, 448))
    vals = fp8.dequantize(codes, 1.0)
    k8 = torch.from_numpy(codes).to(DEV).view(torch.float8_e4m3fn)
    sinks = torch.linspace(-2, 3, 32)
    print("[case] sinks fp8", flush=True)
    out = attention.decode_attention(q, k8, indptr, ids, last, split_kv=0,
                                     sinks=sinks.to(DEV))
    torch.cuda.synchronize()
    want = ref.reference_attention_paged(to_np(q).astype(np.float32), vals, to_np(indptr),
                                         to_np(ids), to_np(last), sinks=sinks.numpy())
    _check(out, want, lens, torch.float16, "fp8")
    # decode_partials has no sinks option: its partials are the plain split's
    po, pm, pl = attention.decode_partials(q, kv, indptr, ids, last, 2)
    plain = attention.merge_partials(po, pm, pl, torch.float16)
    ref_plain = attention.decode_attention(q, kv, indptr, ids, last, split_kv=2)
    torch.cuda.synchronize()
    assert torch.equal(plain, ref_plain)


def test_decode_plan_takes_each_layers_sinks():
    lens = [200, 31, 777]
    q, kv, indptr, ids, last = _inputs(lens, 32, 8, 128, torch.bfloat16, seed=4)
    s1, s2 = torch.randn(32).to(DEV), (torch.randn(32) - 1).to(DEV)
    plan = attention.DecodePlan(q, kv, indptr, ids, last, split_kv=0, sinks=s1)
    print("[case] sinks DecodePlan", flush=True)
    for s in (s1, s2, s1):
        got = plan.run(q, kv, indptr, ids, last, sinks=s)
        want = attention.decode_attention(q, kv, indptr, ids, last, split_kv=0, sinks=s)
        torch.cuda.synchronize()
        assert torch.equal(got, want)
    with pytest.raises(Exception, match="sinks"):
        plan.run(q, kv, indptr, ids, last)
