"""The fused merge (dk_decode_attention_fused; decode_attention with `counters`): one
kernel launch whose last workgroup per (sequence, kv head, head chunk) merges the
partials, against the two-kernel call (pass 1 + merge kernel) on the same inputs.

Both compute every output with the same arithmetic in the same order, so the bar is bit
equality. Cases cover the explicit split (more splits than pages included), the balanced
schedule over ragged batches with sequences without pages at the start, inside, at the
end and everywhere, grouped kv heads (narrow rows), several head chunks, the MFMA q.k
path, sliding windows and soft-capping; the counters must be zero after every call, and
one counter array serves calls of different shapes in a row. CPU tests: argument checks.
"""
import ctypes

import numpy as np
import pytest
import torch

import attention
import dk_lib
import layout
from helpers import err_stats, to_np
from oracle import reference as ref

DEV = "cuda"


def _inputs(lens, hq=32, hkv=8, d=128, dtype=torch.float16, seed=0, kv8=False):
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        len(lens), lens, hq, hkv, d, dtype=dtype, device=DEV, page_table="freelist",
        pool_pages=sum((n + 15) // 16 for n in lens) + 5, seed=seed, q_scale=d ** -0.5 * 3)
    if kv8:
        kv = (kv.float() * 0.5).to(torch.float8_e4m3fn)
    return q, kv, indptr, ids, last


def _both(tens, split, counters, **kw):
    """(fused output, two-kernel output) with caller workspaces."""
    q, kv, indptr, ids, last = tens
    batch, hq, d = q.shape
    need = dk_lib.workspace_bytes(batch, hq, kv.shape[3], d, attention.resolve_split(split))
    outs = []
    for ctr in (counters, None):
        ws = torch.full((max(need, 256),), 0x7F, dtype=torch.uint8, device=DEV)   # NaN-ish
        outs.append(attention.decode_attention(q, kv, indptr, ids, last, split_kv=split,
                                               workspace=ws, counters=ctr, **kw))
    torch.cuda.synchronize()
    return outs


def _counters(n=1 << 16):
    return torch.zeros(n, dtype=torch.int32, device=DEV)


CASES = [
    # (label, lengths, shape kwargs, split, decode kwargs)
    ("split 4", [512, 512], {}, 4, {}),
    ("split 7 ragged", [1, 17, 300, 1000, 16], {}, 7, {}),
    ("split 64 > pages", [40, 900, 3], {}, 64, {}),
    ("split 3 with empty sequences", [0, 100, 0, 0, 257, 0], {}, 3, {}),
    ("balanced uniform", [4096] * 4, {}, 0, {}),
    ("balanced ragged", [5, 3000, 64, 700, 1, 1500, 33, 2048], {}, 0, {}),
    ("balanced empties first/middle/last", [0, 0, 300, 0, 800, 0, 0, 90, 0], {}, 0, {}),
    ("balanced all empty", [0, 0, 0], {}, 0, {}),
    ("balanced one long", [65536], {}, 0, {}),
    ("balanced many short", [int(x) for x in np.random.default_rng(3).integers(1, 90, 700)],
     {}, 0, {}),
    ("balanced D=64 grouped kv heads", [2048] * 8 + [0, 700], dict(d=64), 0, {}),
    ("balanced fp8 grouped kv heads", [3000, 0, 2500, 100], dict(kv8=True), 0, {}),
    ("balanced bf16 64/8 MFMA", [1200, 3300, 0, 77], dict(hq=64, dtype=torch.bfloat16), 0, {}),
    ("balanced 192/8 three chunks", [900, 0, 1800], dict(hq=192), 0, {}),
    ("split 5 48/2 chunks", [700, 1300], dict(hq=48, hkv=2), 5, {}),
    ("D=256 16/2 balanced", [1500, 2600, 0], dict(hq=16, hkv=2, d=256), 0, {}),
    ("window + cap", [300, 2000, 5000], {}, 0, dict(window=700, logit_cap=30.0)),
    ("split 6 window", [3000, 90], {}, 6, dict(window=129)),
    ("qk mfma forced, 2 waves", [2500, 1000], {}, 0, dict(qk_path=1, waves_per_group=2)),
]


@pytest.mark.gpu
@pytest.mark.parametrize("i", range(len(CASES)))
def test_fused_merge_equals_two_kernels_bitwise(i):
    label, lens, shape, split, kw = CASES[i]
    print(f"[case] fused {label}", flush=True)
    kv8 = shape.pop("kv8", False) if "kv8" in shape else False
    shape = dict(shape)
    tens = _inputs(lens, seed=i, kv8=kv8, **shape)
    ctr = _counters()
    hint = attention.plan_hint(tens[2].cpu())
    for h in (0, hint):   # without and with the plan hint (other schedules)
        fused, two = _both(tens, split, ctr, max_pages_per_seq=h, **kw)
        assert torch.equal(fused, two), (label, h, float((fused.float() - two.float()).abs().max()))
        assert torch.count_nonzero(ctr).item() == 0, (label, "counters left non-zero")
        empty = [b for b, n in enumerate(lens) if n == 0]
        if empty:
            assert torch.count_nonzero(fused[empty]).item() == 0, label
    if not kv8:   # and the oracle (the two-kernel path's own tests cover fp8 scales)
        q, kv, indptr, ids, last = tens
        want = ref.reference_attention_paged(
            to_np(q).astype(np.float32), to_np(kv).astype(np.float32), to_np(indptr),
            to_np(ids), to_np(last), window=kw.get("window"), logit_cap=kw.get("logit_cap"))
        rows = [b for b, n in enumerate(lens) if n > 0]
        if rows:
            mx, mean = err_stats(fused[rows], want[rows])
            assert mx <= 1e-2 and mean <= 1e-3, (label, mx, mean)


@pytest.mark.gpu
def test_one_counter_array_serves_calls_of_different_shapes_in_a_row():
    ctr = _counters()
    for k, (lens, shape, split) in enumerate([([3000, 10, 0, 900], {}, 0),
                                              ([50] * 3, dict(hq=16, hkv=4), 5),
                                              ([8192] * 2, {}, 0),
                                              ([0, 1], dict(d=64), 2),
                                              ([700] * 33, dict(hq=8, hkv=1), 0)]):
        print(f"[case] counters reuse {k}", flush=True)
        tens = _inputs(lens, seed=40 + k, **shape)
        fused, two = _both(tens, split, ctr)
        assert torch.equal(fused, two), k
        assert torch.count_nonzero(ctr).item() == 0, k


@pytest.mark.gpu
def test_library_scratch_path_is_deterministic():
    # decode_attention without a workspace uses the library's own scratch: equal to the
    # call with a caller workspace, and identical on repeat, also after a larger call has
    # grown that scratch (a sliding window's splits depend on the workspace size given)
    tens = _inputs([2000, 0, 33, 4100], seed=7)
    q, kv, indptr, ids, last = tens
    for split in (0, 3):
        a = attention.decode_attention(q, kv, indptr, ids, last, split_kv=split, window=900)
        big = _inputs([9000] * 16, seed=8)
        attention.decode_attention(*big, split_kv=0)
        b = attention.decode_attention(q, kv, indptr, ids, last, split_kv=split, window=900)
        _, two = _both(tens, split, None, window=900)
        torch.cuda.synchronize()
        assert torch.equal(a, b) and torch.equal(a, two), split


@pytest.mark.gpu
def test_fused_call_under_graph_capture_replays_like_eager():
    tens = _inputs([1500, 3000, 0, 700], seed=11)
    q, kv, indptr, ids, last = tens
    need = dk_lib.workspace_bytes(4, 32, 8, 128, 0)
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    ctr = _counters()
    out = torch.empty_like(q)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        attention.decode_attention(q, kv, indptr, ids, last, split_kv=0, out=out, workspace=ws,
                                   counters=ctr)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        attention.decode_attention(q, kv, indptr, ids, last, split_kv=0, out=out, workspace=ws,
                                   counters=ctr)
    for rep in range(3):
        q.copy_(torch.randn(q.shape, generator=torch.Generator(device=DEV).manual_seed(rep),
                            device=DEV).half())
        g.replay()
        torch.cuda.synchronize()
        _, two = _both(tens, 0, None)
        assert torch.equal(out, two), rep
        assert torch.count_nonzero(ctr).item() == 0, rep


# ---------------------------------------------------------------- CPU: argument checks

def _fused_call(lib, counters, num_counters):
    st = dk_lib.DkStrides(32 * 128, 128, 2 * 16 * 8 * 128, 16 * 8 * 128, 8 * 128, 128,
                          32 * 128, 128)
    return lib.dk_decode_attention_fused(0x10000, 0x20000, None, 0x30000, 0x40000, 0x50000,
                                         0x60000, 0x70000, 1 << 30, counters, num_counters,
                                         2, 32, 8, 128, 16, 64, 64, dk_lib.DK_F16,
                                         ctypes.byref(st), 4, None, None)


def test_fused_entry_point_checks_its_counters():
    lib = dk_lib.load()
    need = dk_lib.merge_counters(2, 32, 8, 128)
    assert need == 2 * 8                      # one per (sequence, kv head): one head chunk
    # 24 q heads per kv head: 2 chunks on the MFMA q.k path, 3 on the VALU one (8 heads
    # each); the count covers either path
    assert dk_lib.merge_counters(2, 192, 8, 128) == 2 * 8 * 3
    assert dk_lib.merge_counters(2, 30, 8, 128) == 0             # invalid shape
    assert _fused_call(lib, None, need) == dk_lib.DK_ENULL
    assert _fused_call(lib, 0x80000, need - 1) == dk_lib.DK_EWORKSPACE
    assert "merge counters" in lib.dk_last_error().decode()
    assert _fused_call(lib, 0x80002, need) == dk_lib.DK_EWORKSPACE
    assert "aligned" in lib.dk_last_error().decode()


def test_python_counters_need_a_caller_workspace():
    # checked before any device work; a CPU tensor also fails the device check first
    with pytest.raises(dk_lib.DecodeArgumentError):
        attention.decode_attention(torch.zeros(2, 32, 128, dtype=torch.float16),
                                   torch.zeros(4, 2, 16, 8, 128, dtype=torch.float16),
                                   torch.zeros(3, dtype=torch.int32),
                                   torch.zeros(4, dtype=torch.int32),
                                   torch.ones(2, dtype=torch.int32), split_kv=2,
                                   counters=torch.zeros(16, dtype=torch.int32))
