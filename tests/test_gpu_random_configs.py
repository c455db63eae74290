"""Seeded random configurations against the CPU oracle, so that the library's automatic
choices meet in combinations the targeted tests do not spell out.

Each case draws head_dim, kv heads, group size, batch and ragged lengths (some empty),
q dtype, cache type (fp8 E4M3 in a fifth of the cases), split_kv (automatic, one pass,
explicit), the plan hint (none, or exact), the q.k path, the wave count, and sometimes
soft-capping or a sliding window; the automatic schedule then picks one pass or the
balanced schedule, head chunks, grouped kv heads, the small-problem and short-sequence
wave counts by itself. A few cases use many short sequences, where the plan hint selects
one wavefront per balanced workgroup, and a few are uniform batches (equal lengths, 64 to
512 (sequence, kv head) pairs), where it selects the one-pass rules for uniform batches.
Bar: max-abs 1e-2 and mean-abs 1e-3 against the fp32 oracle on the values the kernel reads
(the dequantised cache for fp8), with half an ulp of the output's type added to the
max-abs bound (short sequences give large outputs).
"""

import os

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


def _case(i: int):
    r = np.random.default_rng(1000 + i)
    many_short = i % 12 == 11
    d = int(r.choice([64, 128, 256]))
    hkv = int(r.choice([1, 2, 3, 4, 8]))
    group = int(r.choice([1, 2, 3, 4, 5, 7, 8, 12, 16, 17]))
    if hkv * group > 64:
        group = max(1, 64 // hkv)
    if many_short:
        hkv = int(r.choice([4, 8]))
        group = min(group, 64 // hkv)
        batch = 512
        lens = [int(x) for x in r.integers(1, 64, size=batch)]
    else:
        batch = int(r.integers(1, 9))
        lens = [int(x) if r.random() > 0.15 else 0 for x in r.integers(1, 700, size=batch)]
    kv8 = bool(r.random() < 0.2)
    c = dict(
        d=d, hkv=hkv, hq=hkv * group, batch=batch, lens=lens,
        dtype=torch.bfloat16 if r.random() < 0.4 else torch.float16,
        kv8=kv8, scales=(float(r.choice([1.0, 0.5])), float(r.choice([1.0, 0.25]))),
        split=[0, 0, 1, 2, 3, 5][int(r.integers(0, 6))],
        hint=bool(r.random() < 0.6),
        qk_path=int(r.choice([0, 0, 0, 1, 2])),
        waves=int(r.choice([0, 0, 0, 1, 2, 4])),
        cap=float(r.choice([20.0, 50.0])) if r.random() < 0.1 else None,
        window=int(r.integers(1, 400)) if r.random() < 0.1 else None,
        seed=i)
    if many_short:   # the automatic schedule with the plan hint: its short-sequence rule
        c.update(split=0, hint=True, waves=0, window=None)
    if i % 12 == 5:
        # a uniform batch (every sequence the same length) of 64 to 512 (sequence, kv
        # head) pairs, automatic schedule with the plan hint: the one-pass rules for
        # uniform batches of short sequences (16-bit D=128, fp8 D=128, D=64) and the
        # one-pass-or-balanced choice by pairs per CU
        hkv = int(r.choice([4, 8]))
        batch = int(r.choice([8, 16, 32, 64]))
        n = int(r.choice([16, 100, 256, 500, 512, 1024]))
        c.update(hkv=hkv, hq=hkv * min(group, 64 // hkv), batch=batch, lens=[n] * batch,
                 split=0, hint=True, waves=0, window=None, qk_path=0)
    return c


# 96 cases by default; DK_RANDOM_CASES=N runs the first N seeds of the same generator,
# DK_RANDOM_START=K starts at seed K
_START = int(os.environ.get("DK_RANDOM_START", "0"))
CASES = {i: _case(i) for i in range(_START, _START + int(os.environ.get("DK_RANDOM_CASES", "96")))}


@pytest.mark.parametrize("i", sorted(CASES))
def test_random_configuration_matches_oracle(i):
    c = CASES[i]
    label = (f"random case {i}: B={c['batch']} {c['hq']}/{c['hkv']}/{c['d']} {c['dtype']} "
             f"kv8={c['kv8']} split={c['split']} hint={c['hint']} qk={c['qk_path']} "
             f"waves={c['waves']} cap={c['cap']} window={c['window']}")
    print(f"[case] {label}", flush=True)
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        c["batch"], c["lens"], c["hq"], c["hkv"], c["d"], dtype=c["dtype"], device=DEV,
        page_table="freelist", pool_pages=sum((n + 15) // 16 for n in c["lens"]) + 7,
        seed=c["seed"], q_scale=c["d"] ** -0.5 * 4)
    kw = {}
    if c["kv8"]:
        ks, vs = c["scales"]
        x = kv.float().cpu().numpy()
        codes = np.empty(x.shape, np.uint8)
        codes[:, 0] = fp8.encode(np.clip(x[:, 0] / ks, -448, 448))
        codes[:, 1] = fp8.encode(np.clip(x[:, 1] / vs, -448, 448))
        kv_vals = np.empty(x.shape, np.float32)
        kv_vals[:, 0] = fp8.dequantize(codes[:, 0], ks)
        kv_vals[:, 1] = fp8.dequantize(codes[:, 1], vs)
        kv = torch.from_numpy(codes).to(DEV).view(torch.float8_e4m3fn)
        kw.update(k_scale=ks, v_scale=vs)
    else:
        kv_vals = to_np(kv).astype(np.float32)
    want = ref.reference_attention_paged(to_np(q).astype(np.float32), kv_vals, to_np(indptr),
                                         to_np(ids), to_np(last), logit_cap=c["cap"],
                                         window=c["window"])
    hint = attention.plan_hint(indptr.cpu()) if c["hint"] else 0
    out = attention.decode_attention(q, kv, indptr, ids, last, split_kv=c["split"],
                                     max_pages_per_seq=hint, qk_path=c["qk_path"],
                                     waves_per_group=c["waves"], logit_cap=c["cap"],
                                     window=c["window"], **kw)
    torch.cuda.synchronize()
    rows = [b for b, n in enumerate(c["lens"]) if n > 0]
    mx, mean = err_stats(out[rows], want[rows])
    # 1e-2, plus the rounding of the output itself to q's type (half an ulp: 2^-8 |x| for
    # bf16, 2^-11 |x| for fp16): one- and two-token sequences with large V give outputs of
    # magnitude ~4-5, where a bf16 output's rounding alone reaches 0.016
    half_ulp = 2.0 ** -8 if c["dtype"] == torch.bfloat16 else 2.0 ** -11
    d = np.abs(out[rows].float().cpu().numpy().astype(np.float64) - want[rows])
    bound = 1e-2 + half_ulp * np.abs(want[rows])
    assert (d <= bound).all() and mean <= 1e-3, (label, mx, mean)
    # sequences without pages: zeros (the reference's empty-split merge gives 0)
    empty = [b for b, n in enumerate(c["lens"]) if n == 0]
    if empty:
        assert torch.count_nonzero(out[empty]).item() == 0, label
