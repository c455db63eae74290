"""The Python entry point's per-signature plan cache and its library-owned workspace.

decode_attention validates its arguments once per signature (shapes, strides, dtypes,
devices, options) and reuses the validated plan; without a caller workspace it uses one
the library owns per (device, stream). CPU: invalid arguments are rejected on every call
(a failed validation is never cached). GPU: a cached call equals a freshly validated one
bit for bit, a different signature gets its own plan, and results do not depend on how
large earlier calls made the library's workspace.
"""
import pytest
import torch

import attention
import dk_lib
import layout

DEV = "cuda"


def test_invalid_arguments_are_rejected_on_every_call():
    q = torch.zeros(2, 32, 128, dtype=torch.float16)          # CPU: not accepted
    kv = torch.zeros(4, 2, 16, 8, 128, dtype=torch.float16)
    tabs = (torch.zeros(3, dtype=torch.int32), torch.zeros(4, dtype=torch.int32),
            torch.ones(2, dtype=torch.int32))
    for _ in range(3):
        with pytest.raises(dk_lib.DecodeArgumentError, match="CUDA"):
            attention.decode_attention(q, kv, *tabs, split_kv=2)
    assert not attention._PLANS or all(k[0][3].type == "cuda" for k in attention._PLANS)


def test_non_tensor_arguments_still_raise_type_errors():
    with pytest.raises(TypeError):
        attention.decode_attention(None, None, None, None, None)


def _inputs(lens, seed=0, d=128):
    return layout.synthesize_paged(len(lens), lens, 32, 8, d, device=DEV,
                                   page_table="permuted", seed=seed)[:5]


@pytest.mark.gpu
def test_cached_plan_equals_fresh_validation_and_signatures_stay_apart():
    a = _inputs([700, 1500, 33], seed=1)
    b = _inputs([4096, 10], seed=2)
    first = attention.decode_attention(*a, split_kv=0)
    again = attention.decode_attention(*a, split_kv=0)           # cached plan
    other = attention.decode_attention(*b, split_kv=0)           # another signature
    attention._PLANS.clear()
    fresh = attention.decode_attention(*a, split_kv=0)
    fresh_b = attention.decode_attention(*b, split_kv=0)
    torch.cuda.synchronize()
    assert torch.equal(first, again) and torch.equal(first, fresh)
    assert torch.equal(other, fresh_b)
    # an option is part of the signature: split 3 is not the split-0 plan
    s3 = attention.decode_attention(*a, split_kv=3)
    torch.cuda.synchronize()
    assert float((s3.float() - first.float()).abs().max()) < 1e-3


@pytest.mark.gpu
def test_library_workspace_gives_the_same_results_whatever_its_size():
    # the library's workspace only grows; the bytes a call passes are its own need, so a
    # sliding window's explicit splits (chosen to fit the workspace given) never change
    a = _inputs([2000, 0, 33, 4100], seed=7)
    for split in (0, 3):
        x = attention.decode_attention(*a, split_kv=split, window=900)
        attention.decode_attention(*_inputs([9000] * 16, seed=8), split_kv=0)   # grows it
        y = attention.decode_attention(*a, split_kv=split, window=900)
        need = dk_lib.workspace_bytes(4, 32, 8, 128, split)
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=DEV)
        z = attention.decode_attention(*a, split_kv=split, window=900, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(x, y) and torch.equal(x, z), split


@pytest.mark.gpu
def test_caller_out_and_a_side_stream_use_their_own_plan():
    a = _inputs([1200, 300], seed=3)
    want = attention.decode_attention(*a, split_kv=0)
    out = torch.full((2, 64, 128), float("nan"), dtype=torch.float16, device=DEV)[:, ::2]
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        got = attention.decode_attention(*a, split_kv=0, out=out)
    torch.cuda.synchronize()
    assert got is out and torch.equal(out, want)


def test_decode_plan_rejects_a_different_layout_before_any_device_work():
    # the guard runs before the launch: CPU tensors are enough to exercise it (the plan
    # itself needs GPU tensors, so build one around a fake plan object)
    plan = attention.DecodePlan.__new__(attention.DecodePlan)
    q = torch.zeros(2, 32, 128, dtype=torch.float16)
    kv = torch.zeros(4, 2, 16, 8, 128, dtype=torch.float16)
    tabs = (torch.zeros(3, dtype=torch.int32), torch.zeros(4, dtype=torch.int32),
            torch.ones(2, dtype=torch.int32))
    plan._guard = attention.DecodePlan._layout(q, kv, *tabs)
    plan._out_strides = None
    with pytest.raises(dk_lib.DecodeArgumentError, match="shape, strides"):
        plan.run(torch.zeros(3, 32, 128, dtype=torch.float16), kv, *tabs)
    with pytest.raises(dk_lib.DecodeArgumentError, match="shape, strides"):
        plan.run(q, torch.zeros(4, 2, 16, 8, 256, dtype=torch.float16)[..., ::2], *tabs)
    with pytest.raises(dk_lib.DecodeArgumentError, match="out differs"):
        plan.run(q, kv, *tabs, out=torch.zeros(2, 32, 128, dtype=torch.float16))
    # another dtype (q or the cache) or device (a page table) than planned
    with pytest.raises(dk_lib.DecodeArgumentError, match="dtype or device"):
        plan.run(q.to(torch.bfloat16), kv, *tabs)
    with pytest.raises(dk_lib.DecodeArgumentError, match="dtype or device"):
        plan.run(q, kv.to(torch.bfloat16), *tabs)
    with pytest.raises(dk_lib.DecodeArgumentError, match="dtype or device"):
        plan.run(q, kv, tabs[0].to("meta"), *tabs[1:])
    # a plan made with `out`: out must keep its strides, dtype and device
    plan._out_strides = q.stride()
    with pytest.raises(dk_lib.DecodeArgumentError, match="made with an out"):
        plan.run(q, kv, *tabs)
    with pytest.raises(dk_lib.DecodeArgumentError, match="out differs"):
        plan.run(q, kv, *tabs, out=torch.zeros(2, 32, 128, dtype=torch.bfloat16))
    with pytest.raises(dk_lib.DecodeArgumentError, match="out differs"):
        plan.run(q, kv, *tabs, out=torch.zeros(2, 32, 128, dtype=torch.float16, device="meta"))
    with pytest.raises(dk_lib.DecodeArgumentError, match="workspace must be on"):
        plan.run(q, kv, *tabs, out=torch.zeros(2, 32, 128, dtype=torch.float16),
                 workspace=torch.zeros(16, dtype=torch.uint8, device="meta"))


@pytest.mark.gpu
def test_decode_plan_runs_like_decode_attention():
    a = _inputs([700, 1500, 33], seed=5)
    for split in (0, 1, 4):
        hint = attention.plan_hint(a[2].cpu())
        plan = attention.DecodePlan(*a, split_kv=split, max_pages_per_seq=hint)
        got = plan.run(*a)
        want = attention.decode_attention(*a, split_kv=split, max_pages_per_seq=hint)
        torch.cuda.synchronize()
        assert torch.equal(got, want), split
        out = torch.empty_like(a[0])
        plan2 = attention.DecodePlan(*a, split_kv=split, out=out)
        assert plan2.run(*a, out=out) is out
        torch.cuda.synchronize()
        assert float((out.float() - want.float()).abs().max()) < 1e-3
