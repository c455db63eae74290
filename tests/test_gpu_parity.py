"""GPU parity tests: the HIP decode path (through libdk_decode.so's C ABI) against the
CPU oracle and the brute-force golden fixtures.

Tolerance (north star): max-abs error <= 1e-2 vs the fp32 reference for fp16 / bf16
outputs; the reference's own gates add mean-abs <= 1e-3 (notebook.ipynb:203-204).
Results must be bitwise identical on re-runs (notebook.ipynb:258).
"""
import math

import numpy as np
import pytest
import torch

import attention
import layout
from attention import decode_attention, decode_partials, merge_partials
from helpers import check_partials as _check_partials
from helpers import err_stats, golden_to_torch, load_golden, to_np
from oracle import reference as ref
from oracle import split_kv as skv

pytestmark = pytest.mark.gpu
DEV = "cuda"
MAX_ERR = 1e-2
MEAN_ERR = 1e-3


def _oracle(q, kv, indptr, ids, last, batch_subset=None):
    return ref.reference_attention_paged(to_np(q), to_np(kv), to_np(indptr), to_np(ids),
                                         to_np(last), batch_subset=batch_subset)


def _check(out, want, rows=None, max_err=MAX_ERR, mean_err=MEAN_ERR, label=""):
    if rows is not None:
        out, want = out[rows], want[rows]
    assert torch.isfinite(out).all(), f"{label}: non-finite output"
    mx, mean = err_stats(out, want)
    assert mx <= max_err and mean <= mean_err, f"{label}: max {mx:.3e} mean {mean:.3e}"
    return mx


def _announce(msg):
    print(f"[case] {msg}", flush=True)


# ---------------------------------------------------------------- golden fixtures

@pytest.mark.parametrize("name", ["gqa4_d64_f16", "gqa8_d128_bf16", "mha_d128_f16"])
@pytest.mark.parametrize("split", [1, 2, 3, 8, 0])
@pytest.mark.parametrize("qk_path", [1, 2])
def test_golden_outputs(name, split, qk_path):
    _announce(f"golden {name} split={split} qk_path={qk_path}")
    z, dtype = load_golden(name)
    q, kv, indptr, ids, last = golden_to_torch(z, dtype, DEV)
    out = decode_attention(q, kv, indptr, ids, last, split_kv=split, qk_path=qk_path)
    torch.cuda.synchronize()
    # output rounding dominates: half an ulp at |out| < 4 is <= 2e-3 (fp16), 8e-3 (bf16)
    tol = 4e-3 if dtype == "f16" else 1e-2
    _check(out, z["out"], max_err=tol, label=name)


@pytest.mark.parametrize("name", ["gqa4_d64_f16", "gqa8_d128_bf16", "mha_d128_f16"])
def test_golden_partials(name):
    z, dtype = load_golden(name)
    q, kv, indptr, ids, last = golden_to_torch(z, dtype, DEV)
    for key in [k for k in z if k.startswith("partial_m_s")]:
        S = int(key[len("partial_m_s"):])
        _announce(f"golden partials {name} S={S}")
        po, pm, pl = decode_partials(q, kv, indptr, ids, last, S)
        torch.cuda.synchronize()
        m_want, l_want, o_want = z[f"partial_m_s{S}"], z[f"partial_l_s{S}"], z[f"partial_o_s{S}"]
        _check_partials(po, pm, pl, o_want, m_want, l_want, q.dtype)
        # pass 2 alone on the golden partials
        merged = merge_partials(torch.tensor(o_want, dtype=torch.float32, device=DEV),
                                torch.tensor(m_want, dtype=torch.float32, device=DEV),
                                torch.tensor(l_want, dtype=torch.float32, device=DEV),
                                dtype=q.dtype)
        torch.cuda.synchronize()
        _check(merged, z["out"], max_err=1e-2, label=f"merge {name} S={S}")


def test_primer_known_answer_on_gpu():
    # writeup/cuda_primer.md:31-43 embedded in head_dim 64: the four tokens sit on one
    # page (kv_last_page_len 4) and q = [4,4,0,...] so that q.k / sqrt(64) equals the
    # primer's q.k / sqrt(4). Every score is 0.5 and all V = 0.5, so out = 0.5 exactly;
    # the single split has m = 0.5, l = 4 and O = 2 in every dim.
    K = [[1, 0, 1, 0], [0, 1, 0, 1], [1, 0, 0, 1], [0, 1, 1, 0]]
    kv = torch.zeros(1, 2, 16, 1, 64, dtype=torch.float16)
    for t, k in enumerate(K):
        kv[0, 0, t, 0, :4] = torch.tensor(k, dtype=torch.float16)
    kv[:, 1] = 0.5
    q = torch.zeros(1, 1, 64, dtype=torch.float16)
    q[0, 0, :2] = 4.0
    args = [t.to(DEV) for t in (q, kv, torch.tensor([0, 1], dtype=torch.int32),
                                torch.tensor([0], dtype=torch.int32),
                                torch.tensor([4], dtype=torch.int32))]
    for path in (1, 2):
        out = decode_attention(*args, split_kv=1, qk_path=path)
        po, pm, pl = decode_partials(*args, 1, qk_path=path)
        torch.cuda.synchronize()
        assert torch.equal(out.cpu(), torch.full((1, 1, 64), 0.5, dtype=torch.float16))
        assert abs(float(pm[0, 0, 0]) - 0.5) < 1e-6 and abs(float(pl[0, 0, 0]) - 4.0) < 1e-5
        assert torch.allclose(po[0, 0, 0], torch.full((64,), 2.0, device=DEV), atol=1e-5)


# ---------------------------------------------------------------- configs

def test_config1_small_decode():
    # B=2, ctx=512, 32/8/128, fp16, contiguous pages, split 4
    _announce("config1")
    q, kv, indptr, ids, last, _ = layout.synthesize(2, 512, 32, 8, 128, device=DEV, seed=0)
    out = decode_attention(q, kv, indptr, ids, last, split_kv=4)
    torch.cuda.synchronize()
    _check(out, _oracle(q, kv, indptr, ids, last), label="config1")


@pytest.mark.parametrize("ctx", [128, 512, 2048])
@pytest.mark.parametrize("batch", [1, 4])
def test_gate2_sweep(ctx, batch):
    # notebook Gate 2: Hq=8, Hkv=2, D=64, fp16, split in {1,2,4,8}
    q, kv, indptr, ids, last, _ = layout.synthesize(batch, ctx, 8, 2, 64, device=DEV)
    want = _oracle(q, kv, indptr, ids, last)
    for s in (1, 2, 4, 8):
        _announce(f"gate2 ctx={ctx} batch={batch} split={s}")
        out = decode_attention(q, kv, indptr, ids, last, split_kv=s)
        torch.cuda.synchronize()
        _check(out, want, label=f"ctx={ctx} B={batch} S={s}")


@pytest.mark.parametrize("label,ctx,batch,hq,hkv,split", [
    ("ctx=1", 1, 1, 8, 2, 4),
    ("ctx not divisible by page_size (17)", 17, 1, 8, 2, 4),
    ("ctx not divisible by split (30)", 30, 1, 8, 2, 4),
    ("batch=1", 128, 1, 8, 2, 4),
    ("MHA (group 1)", 128, 1, 4, 4, 4),
    ("MQA (group 8)", 128, 1, 8, 1, 4),
])
def test_gate3_edges_and_determinism(label, ctx, batch, hq, hkv, split):
    _announce(f"gate3 {label}")
    q, kv, indptr, ids, last, _ = layout.synthesize(batch, ctx, hq, hkv, 64, device=DEV)
    out = decode_attention(q, kv, indptr, ids, last, split_kv=split)
    out2 = decode_attention(q, kv, indptr, ids, last, split_kv=split)
    torch.cuda.synchronize()
    assert torch.equal(out, out2), f"{label}: not deterministic"
    _check(out, _oracle(q, kv, indptr, ids, last), label=label)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 4), (32, 8), (16, 2), (32, 2)])
def test_dtypes_head_dims_and_groups(dtype, d, hq, hkv):
    _announce(f"shape dtype={dtype} d={d} hq={hq} hkv={hkv}")
    lens = [1, 16, 77, 300]
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        4, lens, hq, hkv, d, dtype=dtype, device=DEV, page_table="permuted", pool_pages=40,
        seed=d + hq)
    want = _oracle(q, kv, indptr, ids, last)
    for s in (1, 3, 0):
        for path in (1, 2):
            out = decode_attention(q, kv, indptr, ids, last, split_kv=s, qk_path=path)
            torch.cuda.synchronize()
            _check(out, want, label=f"{dtype} d={d} {hq}/{hkv} S={s} path={path}")


@pytest.mark.parametrize("waves", [1, 2, 4])
def test_waves_per_group(waves):
    _announce(f"waves={waves}")
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        3, [5, 200, 1000], 32, 8, 128, device=DEV, page_table="permuted", seed=9)
    want = _oracle(q, kv, indptr, ids, last)
    for s in (1, 4):
        out = decode_attention(q, kv, indptr, ids, last, split_kv=s, waves_per_group=waves)
        torch.cuda.synchronize()
        _check(out, want, label=f"waves={waves} S={s}")


def test_nan_poison_outside_valid_tokens_does_not_leak():
    # Rows past kv_last_page_len on the last page and pages no sequence uses are NaN/Inf;
    # the output must be finite and equal to the clean run (select, never 0 * NaN).
    _announce("nan poison")
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        3, [17, 33, 250], 32, 8, 128, device=DEV, page_table="permuted", pool_pages=40, seed=4)
    clean = {s: decode_attention(q, kv, indptr, ids, last, split_kv=s) for s in (1, 2, 5)}
    poisoned = kv.clone()
    used = set(ids.tolist())
    for p in range(kv.shape[0]):
        if p not in used:
            poisoned[p] = float("nan")
    ip, lp, idl = indptr.tolist(), last.tolist(), ids.tolist()
    for b in range(3):
        lastpage = idl[ip[b + 1] - 1]
        poisoned[lastpage, :, lp[b]:] = float("inf") if b % 2 else float("nan")
    for s, ref_out in clean.items():
        out = decode_attention(q, poisoned, indptr, ids, last, split_kv=s)
        torch.cuda.synchronize()
        assert torch.isfinite(out).all()
        assert torch.equal(out, ref_out), f"split {s}"


@pytest.mark.parametrize("split", [1, 2, 7, 16, 64, 128])
def test_split_invariance_long_sequence(split):
    _announce(f"split invariance {split}")
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        2, [4096, 3001], 32, 8, 128, device=DEV, page_table="permuted", seed=21)
    want = _oracle(q, kv, indptr, ids, last)
    out = decode_attention(q, kv, indptr, ids, last, split_kv=split)
    torch.cuda.synchronize()
    _check(out, want, label=f"S={split}")


def test_empty_sequences_and_more_splits_than_pages():
    _announce("empty sequences")
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        4, [0, 3, 0, 40], 8, 2, 64, device=DEV, page_table="permuted", pool_pages=8, seed=2)
    want = _oracle(q, kv, indptr, ids, last)
    for s in (1, 4, 32):
        out = decode_attention(q, kv, indptr, ids, last, split_kv=s)
        torch.cuda.synchronize()
        _check(out, want, label=f"S={s}")
        assert torch.count_nonzero(out[0]) == 0 and torch.count_nonzero(out[2]) == 0


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_partials_match_oracle_two_pass(dtype):
    _announce(f"partials vs oracle {dtype}")
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        2, [500, 61], 8, 2, 128, dtype=dtype, device=DEV, page_table="permuted", seed=3)
    for S in (1, 3, 8, 40):
        po, pm, pl = decode_partials(q, kv, indptr, ids, last, S)
        torch.cuda.synchronize()
        O, m, l = skv.split_partials(to_np(q), to_np(kv), to_np(indptr), to_np(ids),
                                     to_np(last), S)
        _check_partials(po, pm, pl, O, m, l, q.dtype)


def test_strided_q_out_and_side_stream():
    _announce("strided q/out, side stream")
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        2, [100, 260], 32, 8, 128, device=DEV, page_table="permuted", seed=8)
    big = torch.randn(2, 64, 128, dtype=torch.float16, device=DEV)
    big[:, ::2] = q
    qv = big[:, ::2]                       # q_h stride 256, non-contiguous
    out_big = torch.zeros(2, 32, 256, dtype=torch.float16, device=DEV)
    outv = out_big[:, :, :128]
    want = _oracle(q, kv, indptr, ids, last)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        decode_attention(qv, kv, indptr, ids, last, split_kv=4, out=outv)
    s.synchronize()
    _check(outv, want, label="strided")
    assert torch.count_nonzero(out_big[:, :, 128:]) == 0


def test_reference_extension_surface():
    ext = attention.get_hip_ext()
    q, kv, indptr, ids, last, _ = layout.synthesize(2, 64, 8, 2, 64, device=DEV)
    want = _oracle(q, kv, indptr, ids, last)
    _check(ext.decode_attention_naive(q, kv, indptr, ids, last), want)
    _check(ext.decode_attention_split_kv(q, kv, indptr, ids, last), want)
    torch.cuda.synchronize()


# ---------------------------------------------------------------- benchmark configs

@pytest.mark.parametrize("batch", [1, 4, 16, 32, 64])
def test_config2_batch_sweep(batch):
    # ctx=4096, 32/8/128 fp16, pool of batch*256 pages in seeded random order
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        batch, 4096, 32, 8, 128, device=DEV, page_table="permuted", seed=batch)
    subset = list(range(batch)) if batch <= 16 else [0, batch // 2, batch - 1]
    want = _oracle(q, kv, indptr, ids, last, batch_subset=subset)
    for s in (1, 2, 4, 8, 16):
        _announce(f"config2 B={batch} S={s}")
        out = decode_attention(q, kv, indptr, ids, last, split_kv=s)
        torch.cuda.synchronize()
        _check(out, want, rows=subset, label=f"B={batch} S={s}")


@pytest.mark.parametrize("batch,ctx", [(1, 32768), (4, 32768), (1, 131072), (4, 131072)])
def test_config3_long_context_bf16(batch, ctx):
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        batch, ctx, 32, 8, 128, dtype=torch.bfloat16, device=DEV, page_table="permuted",
        seed=ctx + batch)
    subset = [0] if batch == 1 else [0, batch - 1]
    want = _oracle(q, kv, indptr, ids, last, batch_subset=subset)
    for s in (16, 32, 64, 128):
        _announce(f"config3 B={batch} ctx={ctx} S={s}")
        out = decode_attention(q, kv, indptr, ids, last, split_kv=s)
        torch.cuda.synchronize()
        _check(out, want, rows=subset, label=f"B={batch} ctx={ctx} S={s}")


def test_config4_ragged_freelist():
    # B=128, ctx ~ U[128, 8192], q scaled by 1/sqrt(d), pages drawn without replacement
    # from a shuffled free list of 65536 pages (a 4 GiB pool: byte offsets above 2^32)
    lens = layout.ragged_lengths(128, 128, 8192, seed=4)
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        128, lens, 32, 8, 128, device=DEV, page_table="freelist", pool_pages=65536,
        q_scale=1 / math.sqrt(128), seed=4)
    assert int(ids.max()) > 60000
    subset = list(range(0, 128, 8)) + [int(np.argmax(lens)), int(np.argmin(lens))]
    want = _oracle(q, kv, indptr, ids, last, batch_subset=subset)
    for s in (1, 4, 0):
        _announce(f"config4 S={s}")
        out = decode_attention(q, kv, indptr, ids, last, split_kv=s)
        torch.cuda.synchronize()
        _check(out, want, rows=subset, label=f"ragged S={s}")


def test_metric_config_every_sequence():
    # B=32, ctx=8192, 32/8/128 fp16, random page permutation (bench.py's metric workload):
    # the oracle on all 32 sequences, for the reference's split values, the automatic
    # schedule without and with the plan hint (one pass, what bench.py times)
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        32, 8192, 32, 8, 128, device=DEV, page_table="permuted", seed=1)
    want = _oracle(q, kv, indptr, ids, last)
    hint = attention.plan_hint(indptr.cpu())
    for s, h in ((1, 0), (3, 0), (8, 0), (0, 0), (0, hint)):
        _announce(f"metric S={s} hint={h}")
        out = decode_attention(q, kv, indptr, ids, last, split_kv=s, max_pages_per_seq=h)
        torch.cuda.synchronize()
        _check(out, want, label=f"metric S={s} hint={h}")


# ---------------------------------------------------------------- balanced mode

@pytest.mark.parametrize("waves_per_cu", [1, 2, 5, 16])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_balanced_ragged_with_empty_sequences(waves_per_cu, dtype):
    # lengths chosen so that wavefront ranges start and end inside pairs, on pair
    # boundaries, and span several short sequences; two sequences have no pages
    lens = [0, 1, 17, 16, 4000, 0, 33, 2, 900, 1023, 1024, 1025, 5]
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        len(lens), lens, 32, 8, 128, dtype=dtype, device=DEV, page_table="permuted",
        pool_pages=1200, seed=waves_per_cu)
    want = _oracle(q, kv, indptr, ids, last)
    for path in (0, 1):
        for wpg in (1, 4):
            _announce(f"balanced wpc={waves_per_cu} {dtype} path={path} wpg={wpg}")
            out = decode_attention(q, kv, indptr, ids, last, split_kv=0, qk_path=path,
                                   waves_per_group=wpg, waves_per_cu=waves_per_cu, schedule=1)
            out2 = decode_attention(q, kv, indptr, ids, last, split_kv=0, qk_path=path,
                                    waves_per_group=wpg, waves_per_cu=waves_per_cu, schedule=1)
            torch.cuda.synchronize()
            assert torch.equal(out, out2)
            _check(out, want, label=f"wpc={waves_per_cu} path={path} wpg={wpg}")
            assert torch.count_nonzero(out[0]) == 0 and torch.count_nonzero(out[5]) == 0


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d,hq,hkv", [(128, 32, 8), (128, 8, 8), (64, 32, 8), (128, 64, 8)])
def test_balanced_many_short_sequences_one_wave(dtype, d, hq, hkv):
    # one wavefront per workgroup: the page ring runs on from one sequence to the next
    # inside a workgroup's range, so segments of 1-7 pages (every remainder of the ring's
    # groups of three, with and without steady-state rounds), a 0-page sequence between
    # two others, and ranges cut inside sequences must all come out right
    rng = np.random.default_rng(d + hq)
    lens = [int(x) for x in rng.integers(1, 7 * 16 + 1, size=150)]
    lens[10] = 0
    lens[11] = 16 * 3
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        len(lens), lens, hq, hkv, d, dtype=dtype, device=DEV, page_table="permuted",
        seed=d + hq + hkv)
    want = _oracle(q, kv, indptr, ids, last)
    for wpc in (1, 2, 3):
        _announce(f"short sequences one wave {dtype} d={d} {hq}/{hkv} wpc={wpc}")
        out = decode_attention(q, kv, indptr, ids, last, split_kv=0, waves_per_group=1,
                               waves_per_cu=wpc, schedule=1)
        torch.cuda.synchronize()
        _check(out, want, label=f"wpc={wpc}")
        assert torch.count_nonzero(out[10]) == 0


@pytest.mark.parametrize("d,hq,hkv", [(64, 32, 8), (64, 8, 1), (128, 64, 4), (256, 16, 4),
                                      (128, 6, 2)])
def test_balanced_head_layouts(d, hq, hkv):
    # group 8 and 16 (head chunks), group 3 (1 head per wavefront), head_dim 64 / 256
    lens = [300, 7, 129]
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        3, lens, hq, hkv, d, device=DEV, page_table="permuted", pool_pages=60, seed=d + hq)
    want = _oracle(q, kv, indptr, ids, last)
    for wpc in (1, 8):
        _announce(f"balanced heads d={d} {hq}/{hkv} wpc={wpc}")
        out = decode_attention(q, kv, indptr, ids, last, split_kv=0, waves_per_cu=wpc,
                               schedule=1)
        torch.cuda.synchronize()
        _check(out, want, label=f"d={d} {hq}/{hkv} wpc={wpc}")


# GQA groups that are not a power of two, or exceed one chunk: the group is processed in
# the fewest chunks of at most 8 q heads (4 at D=256) on the VALU q.k path or 16 on the
# MFMA path (the default beyond 4 q heads per kv head), each by a wavefront sized to
# the next power of two with the surplus heads masked (no q read, no output or partial
# write)
PADDED_GROUPS = [(128, 3, 1), (128, 10, 2), (64, 12, 2), (128, 14, 2), (128, 20, 2),
                 (64, 24, 2), (128, 48, 2), (256, 5, 1), (256, 12, 2), (128, 32, 1),
                 (64, 40, 1), (256, 17, 1),
                 # narrow rows with several head chunks: the balanced schedule's grouped kv
                 # heads (2 and 4 per workgroup) with the chunks of a unit 8 ids apart
                 (64, 64, 2), (64, 96, 4),
                 # kv-head counts that are not a power of two: 3 groups of 2 (6 kv heads)
                 # and 3 groups of 4 (12 kv heads) per sequence
                 (64, 24, 6), (64, 36, 12)]


@pytest.mark.parametrize("d,hq,hkv", PADDED_GROUPS)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_padded_head_chunks(d, hq, hkv, dtype):
    lens = [1, 300, 17, 129]
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        4, lens, hq, hkv, d, dtype=dtype, device=DEV, page_table="permuted", pool_pages=60,
        seed=d + hq)
    want = _oracle(q, kv, indptr, ids, last)
    hint = attention.plan_hint(indptr.cpu())
    for split, sched, h in ((1, 0, 0), (3, 0, 0), (0, 1, 0), (0, 0, hint)):
        for path in (0, 1, 2):
            for waves in (0, 1, 4):
                label = (f"padded {dtype} d={d} {hq}/{hkv} S={split} sched={sched} "
                         f"path={path} waves={waves}")
                _announce(label)
                out = decode_attention(q, kv, indptr, ids, last, split_kv=split, schedule=sched,
                                       max_pages_per_seq=h, qk_path=path,
                                       waves_per_group=waves)
                torch.cuda.synchronize()
                _check(out, want, label=label)


def test_padded_head_chunks_partials_and_neighbours():
    # partials of a 5-head group (one chunk of 8, 3 masked) equal the oracle's, and no
    # masked head's write reaches a neighbouring group's rows: q heads of kv head 1 come
    # out right although kv head 0's chunk has masked heads right before them
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        2, [500, 61], 10, 2, 128, device=DEV, page_table="permuted", seed=4)
    for S in (1, 3, 8):
        _announce(f"padded partials S={S}")
        po, pm, pl = decode_partials(q, kv, indptr, ids, last, S)
        torch.cuda.synchronize()
        O, m, l = skv.split_partials(to_np(q), to_np(kv), to_np(indptr), to_np(ids),
                                     to_np(last), S)
        _check_partials(po, pm, pl, O, m, l, q.dtype)
    out = torch.full_like(q, float("nan"))
    decode_attention(q, kv, indptr, ids, last, split_kv=0, out=out)
    torch.cuda.synchronize()
    _check(out, _oracle(q, kv, indptr, ids, last), label="padded out= over NaN")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_hnd_cache_as_a_strided_view(dtype):
    # FlashInfer's HND layout (pages, 2, kv_heads, 16, head_dim) is the NHD call on the
    # permuted view: the strides carry the layout, no copy
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        3, [700, 16, 129], 32, 8, 128, dtype=dtype, device=DEV, page_table="permuted", seed=8)
    want = _oracle(q, kv, indptr, ids, last)
    hnd = kv.permute(0, 1, 3, 2, 4).contiguous()        # the HND storage of the same values
    view = hnd.permute(0, 1, 3, 2, 4)                    # seen as NHD
    assert view.data_ptr() == hnd.data_ptr() and not view.is_contiguous()
    for split, path in ((1, 0), (0, 0), (4, 1), (0, 2)):
        _announce(f"HND view {dtype} S={split} path={path}")
        out = decode_attention(q, view, indptr, ids, last, split_kv=split, qk_path=path)
        torch.cuda.synchronize()
        _check(out, want, label=f"HND S={split} path={path}")


# logit soft-capping (Gemma 2: cap 50 on the scaled scores; smaller caps make it bite on
# these inputs) with the model's own softmax scale
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d,hq,hkv,cap,sm", [(256, 16, 8, 1.5, 256 ** -0.5),
                                             (128, 32, 16, 2.0, 144 ** -0.5),
                                             (128, 32, 8, 50.0, 0.3), (64, 40, 4, 1.0, None)])
def test_logit_softcap(dtype, d, hq, hkv, cap, sm):
    lens = [1, 300, 17, 129]
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        4, lens, hq, hkv, d, dtype=dtype, device=DEV, page_table="permuted", pool_pages=60,
        seed=d + hq + 1)
    q = (q.float() * 2).to(dtype)                           # scores large enough to cap
    args = (to_np(q), to_np(kv), to_np(indptr), to_np(ids), to_np(last))
    want = ref.reference_attention_paged(*args, sm_scale=sm, logit_cap=cap)
    plain = ref.reference_attention_paged(*args, sm_scale=sm)
    if cap < 10:
        assert np.abs(want - plain).max() > 2e-2            # the cap changes the result
    hint = attention.plan_hint(indptr.cpu())
    for split, sched, h in ((1, 0, 0), (3, 0, 0), (0, 1, 0), (0, 0, hint)):
        for path in (0, 1, 2):
            label = f"softcap {dtype} d={d} {hq}/{hkv} cap={cap} S={split} sched={sched} path={path}"
            _announce(label)
            out = decode_attention(q, kv, indptr, ids, last, split_kv=split, schedule=sched,
                                   max_pages_per_seq=h, qk_path=path, sm_scale=sm,
                                   logit_cap=cap)
            torch.cuda.synchronize()
            _check(out, want, label=label)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("window", [1, 5, 16, 17, 100, 4096, 100000])
def test_sliding_window(dtype, window):
    lens = [1, 16, 17, 300, 2047, 0, 5000]
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        7, lens, 32, 8, 128, dtype=dtype, device=DEV, page_table="freelist", pool_pages=600,
        seed=window % 97)
    args = (to_np(q), to_np(kv), to_np(indptr), to_np(ids), to_np(last))
    want = ref.reference_attention_paged(*args, window=window)
    want[5] = 0                                        # the empty sequence
    hint = attention.plan_hint(indptr.cpu())
    for split, path in ((1, 0), (3, 0), (0, 0), (0, 1), (8, 2)):
        label = f"window={window} {dtype} S={split} path={path}"
        _announce(label)
        out = decode_attention(q, kv, indptr, ids, last, split_kv=split, qk_path=path,
                               max_pages_per_seq=hint, window=window)
        torch.cuda.synchronize()
        _check(out, want, label=label)


def test_sliding_window_with_softcap_and_partials():
    lens = [700, 33, 160]
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        3, lens, 16, 8, 256, device=DEV, page_table="permuted", seed=31)
    q = (q.float() * 2).half()
    args = (to_np(q), to_np(kv), to_np(indptr), to_np(ids), to_np(last))
    want = ref.reference_attention_paged(*args, window=129, logit_cap=2.0, sm_scale=0.05)
    _announce("window + softcap")
    out = decode_attention(q, kv, indptr, ids, last, split_kv=0, window=129, logit_cap=2.0,
                           sm_scale=0.05)
    torch.cuda.synchronize()
    _check(out, want, label="window + softcap")
    # pass 1 alone over the window's pages, merged by pass 2, equals the full call
    po, pm, pl = decode_partials(q, kv, indptr, ids, last, 4, window=129, logit_cap=2.0)
    merged = merge_partials(po, pm, pl, dtype=q.dtype)
    full = decode_attention(q, kv, indptr, ids, last, split_kv=4, window=129, logit_cap=2.0)
    torch.cuda.synchronize()
    assert torch.equal(merged, full)


def test_balanced_pass1_alone_runs():
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        4, 1000, 32, 8, 128, device=DEV, page_table="permuted", seed=5)
    import ctypes
    import dk_lib
    lib = dk_lib.load()
    ws = torch.empty(dk_lib.workspace_bytes(4, 32, 8, 128, 0), dtype=torch.uint8, device=DEV)
    st = attention._strides(q, kv, None)
    rc = lib.dk_decode_partials(q.data_ptr(), kv.data_ptr(), indptr.data_ptr(), ids.data_ptr(),
                                last.data_ptr(), ws.data_ptr(), ws.numel(), 4, 32, 8, 128, 16,
                                kv.shape[0], ids.shape[0], 0, ctypes.byref(st), 0, None,
                                torch.cuda.current_stream().cuda_stream)
    dk_lib.check(rc, "partials")
    torch.cuda.synchronize()


# ---------------------------------------------------------------- schedules

@pytest.mark.parametrize("batch", [5, 40])
def test_schedules_agree_and_reuse_a_dirty_workspace(batch):
    # split_kv=0: the automatic choice, the balanced schedule (at two grid sizes, so the
    # same sequence is covered by one workgroup in one call and several in another) and
    # the one-pass kernel all match the oracle; the workspace is reused across calls and
    # first filled with junk, which no schedule may read
    import dk_lib
    base = [3000, 17, 0, 800, 1]
    lens = (base * (batch // len(base) + 1))[:batch]
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        batch, lens, 32, 8, 128, device=DEV, page_table="permuted", seed=batch + 11)
    want = _oracle(q, kv, indptr, ids, last)
    ws = torch.randint(0, 256, (dk_lib.workspace_bytes(batch, 32, 8, 128, 0),),
                       dtype=torch.uint8, device=DEV)
    # plan hints: none, the true longest sequence, and one far too small (speed only)
    hint = attention.plan_hint(indptr.cpu())
    outs = []
    for sched, wpc, h in ((0, 0, 0), (1, 1, 0), (1, 8, 0), (2, 0, 0), (0, 0, hint), (0, 0, 1),
                          (0, 16, hint), (0, 0, 0)):
        _announce(f"schedule={sched} wpc={wpc} hint={h} batch={batch}")
        out = decode_attention(q, kv, indptr, ids, last, split_kv=0, workspace=ws,
                               schedule=sched, waves_per_cu=wpc, max_pages_per_seq=h)
        torch.cuda.synchronize()
        _check(out, want, label=f"schedule={sched} wpc={wpc} hint={h}")
        outs.append(out.clone())
    for o in outs[1:]:
        assert torch.allclose(o.float(), outs[0].float(), atol=2e-3)


@pytest.mark.parametrize("kv8,d,hq,hkv,batch,pages,want", [
    (True, 128, 32, 8, 32, 512, 0), (True, 128, 32, 8, 32, 353, 0),
    (True, 128, 32, 8, 32, 352, 1), (True, 128, 32, 8, 32, 256, 1),
    (True, 128, 8, 8, 32, 512, 0), (True, 128, 32, 32, 8, 512, 0),
    (True, 128, 8, 2, 128, 512, 0), (True, 128, 32, 8, 32, 2048, 0),
    (True, 128, 64, 8, 32, 512, 1), (True, 128, 12, 3, 85, 512, 1),
    (False, 64, 32, 8, 32, 512, 0), (False, 64, 32, 8, 32, 352, 1),
    (False, 64, 64, 8, 32, 512, 0), (False, 64, 32, 32, 8, 1024, 0),
    (False, 64, 12, 3, 85, 512, 1), (False, 128, 32, 8, 32, 512, 1)])
def test_narrow_rows_long_uniform_plans_balanced(kv8, d, hq, hkv, batch, pages, want):
    # about one (sequence, kv head) pair per CU of the MI355X's 256, uniform lengths: one
    # pass fits, and it is what the automatic schedule runs over 256-byte rows (16-bit
    # D=128); over 128-byte rows (fp8 D=128 with up to 4 q heads per kv head, 16-bit D=64
    # with up to 8) with an even kv-head count, sequences longer than 352 pages take the
    # balanced schedule with grouped kv heads (0); fp8 with 8 q heads per kv head, an odd
    # kv-head count and shorter sequences keep one pass (1)
    import dk_lib
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if cus != 256:
        pytest.skip(f"the cases are sized for 256 CUs, not {cus}")
    code = attention._DTYPE_CODE[torch.float16]
    opts = dk_lib.options(max_pages_per_seq=pages,
                          kv_dtype=dk_lib.DK_KV_FP8_E4M3 if kv8 else dk_lib.DK_KV_SAME)
    got = dk_lib.plan_schedule(batch, hq, hkv, d, batch * pages, code, 0, opts)
    _announce(f"plan {'fp8' if kv8 else 'fp16'} D={d} {hq}/{hkv} B={batch} pages={pages}: "
              f"{got}")
    assert got == want


@pytest.mark.parametrize("batch,pages,dtype,want", [
    (16, 4096, torch.float16, 2), (4, 8192, torch.bfloat16, 8), (16, 2048, torch.float16, 2),
    (8, 4096, torch.float16, 4), (16, 1024, torch.float16, 0), (1, 8192, torch.bfloat16, 0),
    (2, 4096, torch.float16, 0)])
def test_long_uniform_plans_explicit_split(batch, pages, dtype, want):
    # 16-bit D=128, uniform lengths: when the (sequence, kv head) pairs divide the balanced
    # grid of the MI355X's 256 CUs into S >= 2 ranges of at least 1024 pages, split_kv 0
    # runs the explicit split S (the plan names it); shorter ranges stay balanced (0)
    import dk_lib
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if cus != 256:
        pytest.skip(f"the cases are sized for 256 CUs, not {cus}")
    code = attention._DTYPE_CODE[dtype]
    got = dk_lib.plan_schedule(batch, 32, 8, 128, batch * pages, code, 0,
                               dk_lib.options(max_pages_per_seq=pages))
    _announce(f"plan B={batch} pages={pages} {dtype}: {got}")
    assert got == want
    # an fp8 cache, or a ragged batch, of the same size stays balanced
    assert dk_lib.plan_schedule(batch, 32, 8, 128, batch * pages, code, 0,
                                dk_lib.options(max_pages_per_seq=pages,
                                               kv_dtype=dk_lib.DK_KV_FP8_E4M3)) == 0
    if batch > 1:
        assert dk_lib.plan_schedule(batch, 32, 8, 128, batch * pages // 2, code, 0,
                                    dk_lib.options(max_pages_per_seq=pages)) == 0


def test_long_uniform_split_fill_matches_oracle():
    # B=16 uniform sequences of 2048 pages with the plan hint: split_kv 0 runs the explicit
    # split 2 (on 256 CUs); checked against the oracle on three sequences and against the
    # forced balanced schedule on all of them
    import dk_lib
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        16, 2048 * 16 - 7, 32, 8, 128, dtype=torch.float16, device=DEV,
        page_table="permuted", seed=41)
    hint = attention.plan_hint(indptr.cpu())
    code = attention._DTYPE_CODE[torch.float16]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    s = dk_lib.plan_schedule(16, 32, 8, 128, ids.shape[0], code, 0,
                             dk_lib.options(max_pages_per_seq=hint))
    _announce(f"split fill B=16 pages=2048: plan {s}")
    if cus == 256:
        assert s == 2
    rows = [0, 7, 15]
    want = _oracle(q, kv, indptr, ids, last, batch_subset=rows)
    a = decode_attention(q, kv, indptr, ids, last, split_kv=0, max_pages_per_seq=hint)
    b = decode_attention(q, kv, indptr, ids, last, split_kv=0, schedule=1)
    c = decode_attention(q, kv, indptr, ids, last, split_kv=2)
    torch.cuda.synchronize()
    _check(a, want, rows=rows, label="split fill")
    assert torch.allclose(a.float(), b.float(), atol=2e-3)
    if s == 2:
        assert torch.equal(a, c)   # the same kernel and partition as split_kv=2


def test_d64_long_uniform_balanced_matches_oracle():
    # 16-bit D=64, uniform B=32 sequences of 400 pages with the plan hint: the automatic
    # schedule is the balanced one with grouped kv heads; checked against the oracle and
    # against the forced one pass
    import dk_lib
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        32, 400 * 16 - 5, 32, 8, 64, dtype=torch.bfloat16, device=DEV, page_table="permuted",
        seed=33)
    hint = attention.plan_hint(indptr.cpu())
    code = attention._DTYPE_CODE[torch.bfloat16]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if cus == 256:
        assert dk_lib.plan_schedule(32, 32, 8, 64, ids.shape[0], code, 0,
                                    dk_lib.options(max_pages_per_seq=hint)) == 0
    rows = [0, 13, 31]
    want = _oracle(q, kv, indptr, ids, last, batch_subset=rows)
    a = decode_attention(q, kv, indptr, ids, last, split_kv=0, max_pages_per_seq=hint)
    b = decode_attention(q, kv, indptr, ids, last, split_kv=0, schedule=2)
    torch.cuda.synchronize()
    _check(a, want, rows=rows, label="balanced D=64")
    assert torch.allclose(a.float(), b.float(), atol=2e-3)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_plan_hint_one_pass_on_uniform_batch(dtype):
    # uniform batch that fills the balanced grid: with the hint the automatic schedule is
    # the one pass (no merge); results agree with the balanced schedule and the oracle
    import dk_lib
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        32, 1000, 32, 8, 128, dtype=dtype, device=DEV, page_table="permuted", seed=21)
    hint = attention.plan_hint(indptr.cpu())
    code = attention._DTYPE_CODE[dtype]
    assert dk_lib.plan_schedule(32, 32, 8, 128, ids.shape[0], code, 0,
                                dk_lib.options(max_pages_per_seq=hint)) == 1
    assert dk_lib.plan_schedule(32, 32, 8, 128, ids.shape[0], code, 0) == 0
    want = _oracle(q, kv, indptr, ids, last, batch_subset=range(0, 32, 5))
    a = decode_attention(q, kv, indptr, ids, last, split_kv=0, max_pages_per_seq=hint)
    b = decode_attention(q, kv, indptr, ids, last, split_kv=0)
    torch.cuda.synchronize()
    _check(a, want, rows=list(range(0, 32, 5)), label="hinted")
    assert torch.allclose(a.float(), b.float(), atol=2e-3)


@pytest.mark.parametrize("hq", [32, 64])
def test_plan_hint_one_pass_one_wave_on_twice_the_pairs(hq):
    # a uniform batch of twice the pairs the two-wavefront grid holds: with the hint the
    # automatic schedule is the one pass at one wavefront per workgroup (no merge); a batch
    # whose pairs do not fill the CUs evenly stays balanced; results agree with the oracle
    # and with the balanced schedule
    import dk_lib
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    batch = 2 * cus // 8                      # 2 * CUs (sequence, kv head) pairs
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        batch, 1000, hq, 8, 128, device=DEV, page_table="permuted", seed=hq)
    hint = attention.plan_hint(indptr.cpu())
    code = attention._DTYPE_CODE[torch.float16]
    opts = dk_lib.options(max_pages_per_seq=hint)
    assert dk_lib.plan_schedule(batch, hq, 8, 128, ids.shape[0], code, 0, opts) == 1
    # user-set wave counts, or three quarters of the batch: the balanced schedule
    assert dk_lib.plan_schedule(batch, hq, 8, 128, ids.shape[0], code, 0,
                                dk_lib.options(waves_per_cu=2, max_pages_per_seq=hint)) == 0
    b3 = batch * 3 // 4
    assert dk_lib.plan_schedule(b3, hq, 8, 128, b3 * 63, code, 0, opts) == 0
    rows = list(range(0, batch, 7))
    want = _oracle(q, kv, indptr, ids, last, batch_subset=rows)
    _announce(f"one pass one wave hq={hq} batch={batch}")
    a = decode_attention(q, kv, indptr, ids, last, split_kv=0, max_pages_per_seq=hint)
    b = decode_attention(q, kv, indptr, ids, last, split_kv=0, schedule=1)
    torch.cuda.synchronize()
    _check(a, want, rows=rows, label="one pass, one wave")
    assert torch.allclose(a.float(), b.float(), atol=2e-3)


@pytest.mark.parametrize("batch,ctx,dtype,hq", [(16, 500, torch.float16, 32),
                                                 (8, 256, torch.bfloat16, 32),
                                                 (32, 300, torch.float16, 16),
                                                 (16, 512, torch.float16, 64)])
def test_plan_hint_one_pass_four_waves_short_uniform(batch, ctx, dtype, hq):
    # a uniform batch of sequences of at most 32 pages with CUs/4 to CUs (sequence, kv
    # head) pairs: with the hint the automatic schedule is one pass (4 wavefronts per
    # workgroup, no merge); longer sequences or fewer pairs stay balanced; results agree
    # with the oracle and with the balanced schedule (64 q heads: the MFMA q.k path)
    import dk_lib
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        batch, ctx, hq, 8, 128, dtype=dtype, device=DEV, page_table="permuted", seed=batch)
    hint = attention.plan_hint(indptr.cpu())
    code = attention._DTYPE_CODE[dtype]
    n = ids.shape[0]
    assert 4 * batch * 8 >= cus and batch * 8 <= cus
    assert dk_lib.plan_schedule(batch, hq, 8, 128, n, code, 0,
                                dk_lib.options(max_pages_per_seq=hint)) == 1
    # sequences of 33 pages or more (fewer pairs than CUs), or a quarter of the pairs:
    # balanced
    if batch * 8 < cus:
        assert dk_lib.plan_schedule(batch, hq, 8, 128, batch * 64, code, 0,
                                    dk_lib.options(max_pages_per_seq=64)) == 0
    b2 = max(cus // 64, 1)
    assert dk_lib.plan_schedule(b2, hq, 8, 128, b2 * 32, code, 0,
                                dk_lib.options(max_pages_per_seq=32)) == 0
    rows = list(range(batch))
    want = _oracle(q, kv, indptr, ids, last, batch_subset=rows)
    _announce(f"one pass four waves short uniform batch={batch} ctx={ctx} hq={hq}")
    a = decode_attention(q, kv, indptr, ids, last, split_kv=0, max_pages_per_seq=hint)
    b = decode_attention(q, kv, indptr, ids, last, split_kv=0, schedule=1)
    torch.cuda.synchronize()
    _check(a, want, rows=rows, label="one pass, four waves")
    assert torch.allclose(a.float(), b.float(), atol=2e-3)


@pytest.mark.parametrize("batch,ctx,dtype", [(16, 500, torch.float16),
                                             (64, 256, torch.bfloat16)])
def test_plan_hint_one_pass_short_uniform_d64(batch, ctx, dtype):
    # D=64 (128-byte rows): a uniform batch of sequences of at most 32 pages with CUs/4 to
    # 2 * CUs pairs runs one pass at 4 wavefronts per workgroup instead of the balanced
    # schedule; four times the pairs stays balanced; checked against the oracle and the
    # balanced schedule
    import dk_lib
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        batch, ctx, 32, 8, 64, dtype=dtype, device=DEV, page_table="permuted", seed=batch)
    hint = attention.plan_hint(indptr.cpu())
    code = attention._DTYPE_CODE[dtype]
    if 4 * batch * 8 >= cus and batch * 8 <= 2 * cus:
        assert dk_lib.plan_schedule(batch, 32, 8, 64, ids.shape[0], code, 0,
                                    dk_lib.options(max_pages_per_seq=hint)) == 1
    b8 = cus                                   # 8 pairs per CU
    assert dk_lib.plan_schedule(b8, 32, 8, 64, b8 * 32, code, 0,
                                dk_lib.options(max_pages_per_seq=32)) == 0
    rows = list(range(0, batch, 3)) + [batch - 1]
    want = _oracle(q, kv, indptr, ids, last, batch_subset=rows)
    _announce(f"one pass short uniform D=64 batch={batch} ctx={ctx}")
    a = decode_attention(q, kv, indptr, ids, last, split_kv=0, max_pages_per_seq=hint)
    b = decode_attention(q, kv, indptr, ids, last, split_kv=0, schedule=1)
    torch.cuda.synchronize()
    _check(a, want, rows=rows, label="one pass D=64, four waves")
    assert torch.allclose(a.float(), b.float(), atol=2e-3)


@pytest.mark.parametrize("per_cu,ctx,dtype", [(4, 1000, torch.float16),
                                              (8, 500, torch.bfloat16),
                                              (12, 300, torch.float16)])
def test_plan_hint_one_pass_uniform_whole_multiple_of_pairs_per_cu(per_cu, ctx, dtype):
    # a uniform batch whose (sequence, kv head) pairs are a whole multiple of 4 per CU:
    # with the hint the automatic schedule is one pass (two wavefronts per workgroup at 4
    # per CU, one above); 5 per CU, or the same batch made ragged, stays balanced; results
    # agree with the oracle and with the balanced schedule
    import dk_lib
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    batch = per_cu * cus // 8
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        batch, ctx, 32, 8, 128, dtype=dtype, device=DEV, page_table="permuted", seed=per_cu)
    hint = attention.plan_hint(indptr.cpu())
    code = attention._DTYPE_CODE[dtype]
    opts = dk_lib.options(max_pages_per_seq=hint)
    n = ids.shape[0]
    assert dk_lib.plan_schedule(batch, 32, 8, 128, n, code, 0, opts) == 1
    b5 = 5 * cus // 8
    assert dk_lib.plan_schedule(b5, 32, 8, 128, b5 * hint, code, 0, opts) == 0
    # the longest sequence more than 1/32 above the mean: not uniform
    assert dk_lib.plan_schedule(batch, 32, 8, 128, n, code, 0,
                                dk_lib.options(max_pages_per_seq=hint + hint // 16 + 1)) == 0
    rows = list(range(0, batch, 11)) + [batch - 1]
    want = _oracle(q, kv, indptr, ids, last, batch_subset=rows)
    _announce(f"one pass uniform per_cu={per_cu} batch={batch} ctx={ctx}")
    a = decode_attention(q, kv, indptr, ids, last, split_kv=0, max_pages_per_seq=hint)
    b = decode_attention(q, kv, indptr, ids, last, split_kv=0, schedule=1)
    torch.cuda.synchronize()
    _check(a, want, rows=rows, label=f"one pass, {per_cu} pairs per CU")
    assert torch.allclose(a.float(), b.float(), atol=2e-3)


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("batch", [5, 63, 64, 65, 300, 5000])
def test_balanced_ragged_split_charges_sequence_starts(batch, d):
    # a ragged batch with the plan hint: the balanced schedule charges each sequence start
    # in its range split (pass 1 searches kv_indptr for its range, one to three search
    # steps for these batch sizes, and the merge finds each sequence's ranges with the same
    # formula); empty sequences and ranges that begin in the charge of a sequence start
    # included; D=64 rows also with grouped kv heads (several per workgroup). Checked
    # against the oracle and against the equal-page split (no hint)
    rng = np.random.default_rng(batch)
    hi = 60 if batch >= 300 else 3000
    lens = [int(x) for x in rng.integers(0, hi, size=batch)]
    lens[batch // 2] = 0
    lens[-1] = hi * 3                      # one long sequence: the hint shows a ragged mix
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        batch, lens, 32, 8, d, device=DEV, page_table="permuted", seed=batch)
    hint = attention.plan_hint(indptr.cpu())
    rows = list(range(batch)) if batch <= 65 else \
        sorted(set(range(0, batch, max(batch // 40, 1))) | {batch // 2, batch - 1})
    want = _oracle(q, kv, indptr, ids, last, batch_subset=rows)
    for wpg in (0, 1, 2, 4):
        _announce(f"ragged cost split batch={batch} d={d} wpg={wpg}")
        out = decode_attention(q, kv, indptr, ids, last, split_kv=0, waves_per_group=wpg,
                               schedule=1, max_pages_per_seq=hint)
        ref = decode_attention(q, kv, indptr, ids, last, split_kv=0, waves_per_group=wpg,
                               schedule=1)
        torch.cuda.synchronize()
        _check(out, want, rows=rows, label=f"hint wpg={wpg}")
        assert torch.count_nonzero(out[batch // 2]) == 0
        assert torch.allclose(out.float(), ref.float(), atol=2e-3), wpg


@pytest.mark.parametrize("batch,window", [(2, 128), (32, 128), (32, 4096), (256, 64)])
def test_plan_schedule_names_the_window_split_that_runs(batch, window):
    """With a window, split_kv 0 runs explicit splits of the window's pages: the count
    dk_plan_schedule reports (for the default workspace) is the one that runs, shown by a
    bit-identical output from that explicit split_kv."""
    import dk_lib
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        batch, 2048, 32, 8, 128, device=DEV, page_table="permuted", seed=batch + window)
    code = attention._DTYPE_CODE[q.dtype]
    opts = dk_lib.options(window=window)
    s = dk_lib.plan_schedule(batch, 32, 8, 128, ids.shape[0], code, 0, opts)
    assert s >= 1
    _announce(f"plan_schedule window={window} B={batch}: split {s}")
    auto = decode_attention(q, kv, indptr, ids, last, split_kv=0, window=window)
    explicit = decode_attention(q, kv, indptr, ids, last, split_kv=s, window=window)
    torch.cuda.synchronize()
    assert torch.equal(auto, explicit)
