"""Size-independent properties at the benchmark's full size (B=32, ctx 8192, Hq 32 / Hkv 8,
D 128, fp16, 1 GiB page pool), where the CPU oracle covers only sampled sequences:

* relabelling the physical pages (permuting the pool, remapping kv_indices) changes no bit;
* scaling V by 2 scales every output by 2 to within one output ulp (binary scaling is
  exact in the kernel's fp32 arithmetic and in the final rounding, except that the
  matrix cores may treat fp16 subnormal V elements as zero while their doubles are
  normal);
* adding 1 to every V adds 1 to every output (attention weights sum to one), up to the
  output rounding;
* every schedule (one pass, balanced, explicit splits) agrees with every other, and
  repeated calls are bitwise identical;
plus a large-batch, short-context ragged mix (B=2048, many empty and one-token sequences)
against the oracle.
"""
import numpy as np
import pytest
import torch

import attention
import layout
from helpers import err_stats, to_np
from oracle import reference as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _announce(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def metric_inputs():
    return layout.synthesize_paged(32, 8192, 32, 8, 128, device=DEV, page_table="permuted",
                                   seed=7)


def _schedules(q, kv, indptr, ids, last):
    hint = attention.plan_hint(indptr.cpu())
    return {
        "one pass (hint)": attention.decode_attention(q, kv, indptr, ids, last, split_kv=0,
                                                      max_pages_per_seq=hint),
        "balanced": attention.decode_attention(q, kv, indptr, ids, last, split_kv=0,
                                               schedule=1),
        "split 1": attention.decode_attention(q, kv, indptr, ids, last, split_kv=1),
        "split 8": attention.decode_attention(q, kv, indptr, ids, last, split_kv=8),
    }


def test_page_relabelling_changes_no_bit(metric_inputs):
    q, kv, indptr, ids, last, _ = metric_inputs
    g = torch.Generator(device="cpu")
    g.manual_seed(3)
    perm = torch.randperm(kv.shape[0], generator=g).to(DEV)
    kv2 = torch.empty_like(kv)
    kv2[perm] = kv                                   # physical page p moves to perm[p]
    ids2 = perm[ids.long()].to(torch.int32)
    a, b = _schedules(q, kv, indptr, ids, last), _schedules(q, kv2, indptr, ids2, last)
    torch.cuda.synchronize()
    for name in a:
        _announce(f"relabel {name}")
        assert torch.equal(a[name], b[name]), name


def test_v_scaling_and_shift(metric_inputs):
    q, kv, indptr, ids, last, _ = metric_inputs
    base = _schedules(q, kv, indptr, ids, last)
    kv2 = kv.clone()
    kv2[:, 1] *= 2
    doubled = _schedules(q, kv2, indptr, ids, last)
    kv2[:, 1] = kv[:, 1] + 1
    shifted = _schedules(q, kv2, indptr, ids, last)
    torch.cuda.synchronize()
    for name in base:
        _announce(f"V scaling / shift {name}")
        two = base[name].float() * 2
        diff = (doubled[name].float() - two).abs()
        assert bool((diff <= two.abs() * 2.0 ** -10 + 2.0 ** -24).all()), name
        d = (shifted[name].float() - 1) - base[name].float()
        # V + 1 is itself rounded to fp16 (spacing up to 2^-8 for |V + 1| < 8, so each
        # value moves by <= 2^-9), plus one output rounding on each side (<= 2^-11 for
        # |out + 1| < 2, 2^-12 for |out| < 1): a bound of 2^-9 + 2^-11 + 2^-12
        assert float(d.abs().max()) <= 2.0 ** -9 + 2.0 ** -11 + 2.0 ** -12, name


def test_schedules_agree_and_repeat_bitwise(metric_inputs):
    q, kv, indptr, ids, last, _ = metric_inputs
    a = _schedules(q, kv, indptr, ids, last)
    b = _schedules(q, kv, indptr, ids, last)
    torch.cuda.synchronize()
    ref_out = a["split 1"].float()
    for name in a:
        _announce(f"schedules {name}")
        assert torch.equal(a[name], b[name]), name
        assert float((a[name].float() - ref_out).abs().max()) <= 2e-3, name


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_large_batch_short_ragged(dtype):
    # 2048 sequences of 0..100 tokens (every tenth empty), in a pool with spare pages
    rng = np.random.default_rng(5)
    lens = [0 if i % 10 == 0 else int(rng.integers(1, 101)) for i in range(2048)]
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        2048, lens, 32, 8, 128, dtype=dtype, device=DEV, page_table="freelist",
        pool_pages=sum(-(-n // 16) for n in lens) + 500, seed=6)
    subset = list(range(0, 2048, 37)) + [2047]
    want = ref.reference_attention_paged(to_np(q), to_np(kv), to_np(indptr), to_np(ids),
                                         to_np(last), batch_subset=subset)
    hint = attention.plan_hint(indptr.cpu())
    for split, sched, h in ((0, 0, 0), (0, 0, hint), (1, 0, 0), (3, 0, 0), (0, 1, 0)):
        _announce(f"large batch {dtype} split={split} schedule={sched} hint={h}")
        out = attention.decode_attention(q, kv, indptr, ids, last, split_kv=split,
                                         schedule=sched, max_pages_per_seq=h)
        torch.cuda.synchronize()
        mx, mean = err_stats(out[subset], want[subset])
        assert mx <= 1e-2 and mean <= 1e-3, (split, sched, mx, mean)
        empty = [i for i in range(2048) if lens[i] == 0]
        assert torch.count_nonzero(out[empty]) == 0
