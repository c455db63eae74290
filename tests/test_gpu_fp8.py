"""fp8 (OCP E4M3) KV cache on the GPU: fp16 / bf16 queries over a cache of
torch.float8_e4m3fn codes, K = k_scale * code value, V = v_scale * code value.

* every one of the 256 codes as a V value reaches the output exactly (one-token
  sequences: the attention weight is exactly 1), NaN codes as NaN;
* every finite code as a K value gives the closed-form two-token softmax
  sigmoid(q . k) (q chosen so that the score is about +-1, so a wrongly decoded code
  moves the result far outside the tolerance);
* random caches against the CPU oracle on the dequantised values (oracle/fp8.py), over
  head dims, group sizes, schedules, both cache forms and non-unit scales;
* NaN bytes in the unused tail of a last page never reach the output;
* at the benchmark's full size, the fp8 path equals the fp16 path run on the same values
  stored as fp16 (every E4M3 value is exact in fp16): with q.k on the VALU bitwise with
  unit scales and to one output ulp with power-of-two scales; with q.k on the matrix
  cores to fp32 rounding of the scores.
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
FP8 = torch.float8_e4m3fn


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _codes_to_device(codes: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(codes, np.uint8)).to(DEV).view(FP8)


def _quantize(kv: torch.Tensor, k_scale: float, v_scale: float) -> np.ndarray:
    """E4M3 codes (uint8, same shape) of a combined (pages, 2, 16, Hkv, D) cache."""
    x = kv.detach().float().cpu().numpy()
    codes = np.empty(x.shape, np.uint8)
    codes[:, 0] = fp8.encode(x[:, 0] / k_scale)
    codes[:, 1] = fp8.encode(x[:, 1] / v_scale)
    return codes


def _dequantize(codes: np.ndarray, k_scale: float, v_scale: float) -> np.ndarray:
    out = np.empty(codes.shape, np.float32)
    out[:, 0] = fp8.dequantize(codes[:, 0], k_scale)
    out[:, 1] = fp8.dequantize(codes[:, 1], v_scale)
    return out


def _round_to(x32: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    return torch.from_numpy(x32).to(dtype).float().numpy()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("v_scale", [1.0, 0.37])
def test_every_v_code_reaches_the_output_exactly(dtype, v_scale):
    # 2 sequences of one token each; their V rows (2 kv heads x 128 dims) hold all 256 codes
    codes = np.zeros((2, 2, 16, 2, 128), np.uint8)
    allc = np.arange(256, dtype=np.uint8).reshape(2, 128)
    codes[0, 1, 0] = allc
    codes[1, 1, 0] = allc[::-1]
    kv = _codes_to_device(codes)
    q = torch.randn(2, 2, 128, device=DEV).to(dtype)
    indptr = torch.tensor([0, 1, 2], dtype=torch.int32, device=DEV)
    ids = torch.tensor([0, 1], dtype=torch.int32, device=DEV)
    last = torch.ones(2, dtype=torch.int32, device=DEV)
    vals = np.stack([allc, allc[::-1]]).astype(np.uint8)              # (seq, head, dim)
    want = _round_to((fp8.decode(vals).astype(np.float32) * np.float32(v_scale)), dtype)
    for split, sched in ((1, 0), (0, 0), (0, 1), (3, 0)):
        _announce(f"V codes {dtype} v_scale={v_scale} split={split} schedule={sched}")
        out = attention.decode_attention(q, kv, indptr, ids, last, split_kv=split,
                                         schedule=sched, v_scale=v_scale)
        got = out.float().cpu().numpy()
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan), (split, sched)
        assert np.array_equal(got[~nan], want[~nan]), (split, sched)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("k_scale", [1.0, 0.5])
def test_every_k_code_gives_the_two_token_softmax(dtype, k_scale):
    finite = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], np.uint8)
    b = len(finite)
    hq, d = 4, 64
    codes = np.zeros((b, 2, 16, 1, d), np.uint8)
    codes[:, 0, 0, 0, 0] = finite                      # token 0: K = code at dim 0, else 0
    codes[:, 1, 0, 0, :] = 0x38                        # token 0: V = 1; token 1: K = V = 0
    x = fp8.decode(finite) * k_scale
    qv = np.where(x != 0, 1.0 / np.where(x != 0, x, 1.0), 1.0)
    q = torch.zeros(b, hq, d, dtype=dtype)
    q[:, :, 0] = torch.from_numpy(qv).to(dtype)[:, None]
    s = q[:, 0, 0].double().numpy() * x                # the exact score, about +-1 (0 for +-0)
    want = 1.0 / (1.0 + np.exp(-s))
    kv = _codes_to_device(codes)
    q = q.to(DEV)
    indptr = torch.arange(b + 1, dtype=torch.int32, device=DEV)
    ids = torch.arange(b, dtype=torch.int32, device=DEV)
    last = torch.full((b,), 2, dtype=torch.int32, device=DEV)
    for split, qk in ((1, 0), (0, 0), (1, 1), (0, 1)):
        _announce(f"K codes {dtype} k_scale={k_scale} split={split} qk_path={qk}")
        out = attention.decode_attention(q, kv, indptr, ids, last, split_kv=split, sm_scale=1.0,
                                         k_scale=k_scale, qk_path=qk)
        got = out.float().cpu().numpy()
        err = np.abs(got - want[:, None, None]).max()
        # fp32 softmax + exp2, then one output rounding (2^-9 for bf16 below 1)
        assert err <= (2e-3 if dtype == torch.bfloat16 else 1e-3), (split, qk, err)


CASES = [
    # (batch, lens, hq, hkv, d, dtype, page_table)
    (4, 512, 32, 8, 128, torch.float16, "contiguous"),
    (3, [1, 37, 300], 32, 8, 128, torch.bfloat16, "permuted"),
    (5, [0, 16, 17, 255, 1000], 8, 8, 64, torch.float16, "freelist"),
    (2, [700, 33], 16, 2, 256, torch.bfloat16, "permuted"),
    (2, 160, 64, 4, 128, torch.float16, "permuted"),
    (3, [1, 300, 40], 14, 2, 128, torch.bfloat16, "permuted"),     # 7 q heads per kv head
    (2, [900, 77], 128, 4, 128, torch.float16, "permuted"),       # 2 head chunks of 16
    (3, [513, 1, 64], 16, 4, 64, torch.bfloat16, "freelist"),     # 64-byte rows
    (3, [400, 9, 130], 24, 6, 128, torch.float16, "freelist"),    # 3 groups of 2 kv heads
    (2, [333, 65], 48, 12, 128, torch.bfloat16, "permuted"),      # 3 groups of 4 kv heads
    (4, [200, 0, 95, 31], 12, 6, 64, torch.float16, "freelist"),  # 64-byte rows, 3 groups of 2
]


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("scales", [(1.0, 1.0), (0.25, 0.03)])
def test_random_fp8_cache_matches_oracle(case, scales):
    batch, lens, hq, hkv, d, dtype, table = CASES[case]
    k_scale, v_scale = scales
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        batch, lens, hq, hkv, d, dtype=dtype, device=DEV, page_table=table, pool_pages=64,
        seed=case + 11)
    # stored codes are N(0, 1) / scale; the dequantised cache stays about N(0, 1), the
    # range the 1e-2 tolerance is stated for
    codes = _quantize(kv, k_scale, v_scale)
    deq = _dequantize(codes, k_scale, v_scale)
    want = ref.reference_attention_paged(to_np(q).astype(np.float32), deq, to_np(indptr),
                                         to_np(ids), to_np(last))
    kv8 = _codes_to_device(codes)
    for qk in (0, 1, 2):
        for split, sched in ((1, 0), (0, 0), (0, 1), (0, 2), (4, 0)):
            _announce(f"fp8 case {case} scales={scales} qk_path={qk} split={split} "
                      f"schedule={sched}")
            out = attention.decode_attention(q, kv8, indptr, ids, last, split_kv=split,
                                             schedule=sched, k_scale=k_scale,
                                             v_scale=v_scale, qk_path=qk)
            torch.cuda.synchronize()
            mx, mean = err_stats(out, want)
            assert mx <= 1e-2 and mean <= 1e-3, (qk, split, sched, mx, mean)
    # the (k_cache, v_cache) form over the same bytes
    _announce(f"fp8 case {case} separate caches")
    out = attention.decode_attention(q, (kv8[:, 0], kv8[:, 1]), indptr, ids, last, split_kv=0,
                                     k_scale=k_scale, v_scale=v_scale)
    mx, mean = err_stats(out, want)
    assert mx <= 1e-2 and mean <= 1e-3, (mx, mean)


def test_nan_bytes_in_the_page_tail_never_reach_the_output():
    lens = [1, 5, 15, 17, 31]
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(5, lens, 32, 8, 128, device=DEV,
                                                          page_table="permuted", seed=2)
    codes = _quantize(kv, 1.0, 1.0)
    ip, ix, ll = to_np(indptr), to_np(ids), to_np(last)
    for b in range(5):                                  # poison every slot past the end
        codes[ix[ip[b + 1] - 1], :, ll[b]:] = 0x7F
    want = ref.reference_attention_paged(to_np(q).astype(np.float32),
                                         _dequantize(codes, 1.0, 1.0), ip, ix, ll)
    kv8 = _codes_to_device(codes)
    for split in (1, 0, 2):
        _announce(f"NaN tail split={split}")
        out = attention.decode_attention(q, kv8, indptr, ids, last, split_kv=split)
        assert bool(torch.isfinite(out).all()), split
        mx, _ = err_stats(out, want)
        assert mx <= 1e-2, (split, mx)


def test_fp8_arguments_are_checked():
    q, kv, indptr, ids, last, _ = layout.synthesize(1, 32, 32, 8, 128, device=DEV)
    kv8 = _codes_to_device(_quantize(kv, 1.0, 1.0))
    with pytest.raises(ValueError, match="k_scale"):
        attention.decode_attention(q, kv8, indptr, ids, last, k_scale=0.0)
    with pytest.raises(ValueError, match="v_scale"):
        attention.decode_attention(q, kv8, indptr, ids, last, v_scale=float("nan"))
    with pytest.raises(ValueError, match="float8"):
        attention.decode_attention(q, kv, indptr, ids, last, k_scale=2.0)


@pytest.fixture(scope="module", params=[128, 64])
def metric_fp8(request):
    """Benchmark shape (B=32, ctx 8192, 32/8/128) and its D=64 form (64-byte rows: the LDS
    page ring and whole-row kv-head groups of the balanced schedule): random finite E4M3
    codes of moderate magnitude (|value| <= 3.75) and the same values as an fp16 cache."""
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(32, 8192, 32, 8, request.param,
                                                          device=DEV, page_table="permuted",
                                                          seed=9)
    g = torch.Generator(device=DEV)
    g.manual_seed(9)
    mag = torch.randint(0, 0x48, kv.shape, generator=g, device=DEV, dtype=torch.int32)
    sign = torch.randint(0, 2, kv.shape, generator=g, device=DEV, dtype=torch.int32) * 0x80
    codes = (mag | sign).to(torch.uint8)
    del kv
    table = torch.from_numpy(fp8.decode(np.arange(256)).astype(np.float16)).to(DEV)
    return q, codes, table, indptr, ids, last


@pytest.mark.parametrize("scales", [(1.0, 1.0), (2.0, 0.5)])
def test_full_size_fp8_equals_fp16_on_the_same_values(metric_fp8, scales):
    q, codes, table, indptr, ids, last = metric_fp8
    k_scale, v_scale = scales
    kv16 = table[codes.long()]
    kv16[:, 0] *= k_scale
    kv16[:, 1] *= v_scale                                # exact: powers of two, no overflow
    kv8 = codes.view(FP8)
    hint = attention.plan_hint(indptr.cpu())
    # the same work split for both caches (the fp8 defaults use more wavefronts), so the
    # same fp32 sums in the same order
    for qk, split, sched, h in ((2, 1, 0, 0), (2, 0, 0, hint), (2, 0, 1, 0), (2, 8, 0, 0),
                                (1, 1, 0, 0), (1, 0, 1, 0)):
        knobs = dict(waves_per_group=4, waves_per_cu=4, qk_path=qk)
        _announce(f"full size fp8 vs fp16 D={q.shape[-1]} scales={scales} qk_path={qk} "
                  f"split={split} schedule={sched}")
        a = attention.decode_attention(q, kv8, indptr, ids, last, split_kv=split,
                                       schedule=sched, max_pages_per_seq=h, k_scale=k_scale,
                                       v_scale=v_scale, **knobs)
        b = attention.decode_attention(q, kv16, indptr, ids, last, split_kv=split,
                                       schedule=sched, max_pages_per_seq=h, **knobs)
        # and the fp8 defaults agree with it to fp32 rounding of a different split
        c = attention.decode_attention(q, kv8, indptr, ids, last, split_kv=split,
                                       schedule=sched, max_pages_per_seq=h, k_scale=k_scale,
                                       v_scale=v_scale)
        torch.cuda.synchronize()
        assert float((c.float() - a.float()).abs().max()) <= 2e-3, (qk, split, sched)
        if qk == 1:
            # the MFMA q.k assigns dims to the matrix cores' k slots differently for fp8
            # loads (16 dims per lane) than for 16-bit loads (8 per lane), so the scores'
            # fp32 sums run in another order
            assert float((a.float() - b.float()).abs().max()) <= 2e-3, (qk, split, sched)
        elif scales == (1.0, 1.0):
            assert torch.equal(a, b), (qk, split, sched)
        else:
            # scaling V by 0.5 before or after the fp32 sums differs only where a matrix
            # core product falls into the fp32 subnormal range: one output ulp at most
            diff = (a.float() - b.float()).abs()
            assert bool((diff <= b.float().abs() * 2.0 ** -10 + 2.0 ** -24).all()), (qk, split,
                                                                                      sched)
    del kv16


def test_fp8_partials_match_oracle():
    # pass 1 alone over an fp8 cache: the reference's (O, m, l) partials of the dequantised
    # values (v_scale multiplies O only; k_scale enters the scores, hence m)
    from helpers import check_partials
    from oracle import split_kv as skv
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(2, [500, 61], 8, 2, 128, device=DEV,
                                                          page_table="permuted", seed=3)
    ks, vs = 0.5, 0.25
    codes = _quantize(kv, ks, vs)
    deq = _dequantize(codes, ks, vs)
    kv8 = _codes_to_device(codes)
    for S in (1, 3, 8):
        _announce(f"fp8 partials S={S}")
        po, pm, pl = attention.decode_partials(q, kv8, indptr, ids, last, S, k_scale=ks,
                                               v_scale=vs)
        torch.cuda.synchronize()
        O, m, l = skv.split_partials(to_np(q).astype(np.float32), deq, to_np(indptr),
                                     to_np(ids), to_np(last), S)
        check_partials(po, pm, pl, O, m, l, q.dtype)


@pytest.mark.parametrize("batch,d", [(65, 128), (2000, 128), (65, 64), (2000, 64)])
def test_ragged_fp8_charged_range_split_matches_oracle(batch, d):
    # a ragged batch over an fp8 cache with the plan hint: the balanced schedule groups
    # kv heads (rows of 128 bytes, or 64 read through the LDS page ring) and charges each
    # sequence start in its range split
    rng = np.random.default_rng(batch + 3)
    hi = 40 if batch > 100 else 2500
    lens = [int(x) for x in rng.integers(0, hi, size=batch)]
    lens[-1] = 3 * hi
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        batch, lens, 32, 8, d, device=DEV, page_table="permuted", seed=batch)
    codes = _quantize(kv, 0.5, 0.25)
    deq = _dequantize(codes, 0.5, 0.25)
    rows = list(range(0, batch, max(batch // 50, 1))) + [batch - 1]
    want = ref.reference_attention_paged(to_np(q).astype(np.float32), deq, to_np(indptr),
                                         to_np(ids), to_np(last), batch_subset=rows)
    kv8 = _codes_to_device(codes)
    hint = attention.plan_hint(indptr.cpu())
    _announce(f"fp8 ragged charged split batch={batch} d={d}")
    out = attention.decode_attention(q, kv8, indptr, ids, last, split_kv=0, schedule=1,
                                     max_pages_per_seq=hint, k_scale=0.5, v_scale=0.25)
    ref_out = attention.decode_attention(q, kv8, indptr, ids, last, split_kv=0, schedule=1,
                                         k_scale=0.5, v_scale=0.25)
    torch.cuda.synchronize()
    mx, mean = err_stats(out[rows], want[rows])
    assert mx <= 1e-2 and mean <= 1e-3, (mx, mean)
    assert torch.allclose(out.float(), ref_out.float(), atol=2e-3)


@pytest.mark.parametrize("batch,ctx,d", [(8, 500, 128), (64, 256, 128), (512, 200, 128),
                                         (16, 512, 64), (64, 200, 64)])
def test_short_uniform_fp8_one_pass_matches_oracle(batch, ctx, d):
    # a uniform batch of sequences of at most 32 pages over an fp8 cache with the plan
    # hint: the automatic schedule is one pass (D=128: 4 wavefronts per workgroup below 8
    # pairs per CU, one from there; D=64: 4, up to 2 pairs per CU); ctx 1024 stays
    # balanced; checked against the oracle and against the balanced schedule
    import dk_lib
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        batch, ctx, 32, 8, d, device=DEV, page_table="permuted", seed=batch + 7)
    codes = _quantize(kv, 0.5, 0.25)
    deq = _dequantize(codes, 0.5, 0.25)
    hint = attention.plan_hint(indptr.cpu())
    code = attention._DTYPE_CODE[torch.float16]
    opts = dk_lib.options(max_pages_per_seq=hint, kv_dtype=dk_lib.DK_KV_FP8_E4M3)
    if 4 * batch * 8 >= cus and (d == 128 or batch * 8 <= 2 * cus):
        assert dk_lib.plan_schedule(batch, 32, 8, d, ids.shape[0], code, 0, opts) == 1
    b256 = cus
    assert dk_lib.plan_schedule(b256, 32, 8, d, b256 * 64, code, 0,
                                dk_lib.options(max_pages_per_seq=64,
                                               kv_dtype=dk_lib.DK_KV_FP8_E4M3)) == 0
    rows = list(range(0, batch, max(batch // 40, 1))) + [batch - 1]
    want = ref.reference_attention_paged(to_np(q).astype(np.float32), deq, to_np(indptr),
                                         to_np(ids), to_np(last), batch_subset=rows)
    kv8 = _codes_to_device(codes)
    _announce(f"fp8 short uniform one pass batch={batch} ctx={ctx}")
    out = attention.decode_attention(q, kv8, indptr, ids, last, split_kv=0,
                                     max_pages_per_seq=hint, k_scale=0.5, v_scale=0.25)
    bal = attention.decode_attention(q, kv8, indptr, ids, last, split_kv=0, schedule=1,
                                     k_scale=0.5, v_scale=0.25)
    torch.cuda.synchronize()
    mx, mean = err_stats(out[rows], want[rows])
    assert mx <= 1e-2 and mean <= 1e-3, (mx, mean)
    assert torch.allclose(out.float(), bal.float(), atol=2e-3)
