"""dk_decode_attention_noalloc: the entry point that allocates nothing (its partials go to
the library's static device scratch) against dk_decode_attention_ex with a caller-owned
workspace, both through the C ABI.

The two run the same kernels with the same schedule, so their outputs must agree bit for
bit. Calls come in pairs, the second with a smaller problem, so the second reads a
scratch that still holds the first call's partials (nothing in it needs to start at
zero). A call whose scratch would exceed DK_STATIC_SCRATCH_BYTES is rejected before any
device call (a CPU test).
"""
import ctypes

import pytest
import torch

import attention
import dk_lib
import layout

DEV = "cuda"


def _args(q, kv, indptr, ids, last, out):
    st = attention._strides(q, kv, out)
    B, hq, d = q.shape
    shape = (B, hq, kv.shape[3], d, 16, kv.shape[0], ids.shape[0], attention._DTYPE_CODE[q.dtype],
             ctypes.byref(st))
    return st, (q.data_ptr(), kv.data_ptr(), indptr.data_ptr(), ids.data_ptr(),
                last.data_ptr(), out.data_ptr()), shape


def _noalloc(lib, q, kv, indptr, ids, last, split, opts):
    out = torch.full_like(q, float("nan"))
    st, ptrs, shape = _args(q, kv, indptr, ids, last, out)
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.dk_decode_attention_noalloc(*ptrs, *shape, split, ctypes.byref(opts), stream)
    dk_lib.check(rc, "dk_decode_attention_noalloc")
    return out


def _with_workspace(lib, q, kv, indptr, ids, last, split, opts):
    out = torch.full_like(q, float("nan"))
    st, ptrs, shape = _args(q, kv, indptr, ids, last, out)
    need = dk_lib.workspace_bytes(q.shape[0], q.shape[1], kv.shape[3], q.shape[2], split)
    ws = torch.full((max(need, 1),), 0xFF, dtype=torch.uint8, device=q.device)
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.dk_decode_attention_ex(*ptrs[:6], ws.data_ptr(), need, *shape, split,
                                    ctypes.byref(opts), stream)
    dk_lib.check(rc, "dk_decode_attention_ex")
    return out


# (batch, context lengths, q heads, kv heads, head dim, dtype, split, plan hint);
# each case runs a larger problem and then a smaller one through the same scratch
CASES = [
    ((16, 4096, 32, 8, 128, torch.float16, 0, True), (2, 512, 32, 8, 128, torch.float16, 0, True)),
    ((24, "ragged", 32, 8, 128, torch.float16, 0, False), (5, "ragged", 32, 8, 128, torch.float16, 0, False)),
    ((8, 2048, 32, 8, 64, torch.bfloat16, 8, False), (3, 300, 32, 8, 64, torch.bfloat16, 4, False)),
    ((4, 8192, 64, 8, 128, torch.bfloat16, 0, False), (1, 1000, 64, 8, 128, torch.bfloat16, 0, False)),
    ((6, 1500, 16, 2, 256, torch.float16, 1, False), (2, 100, 16, 2, 256, torch.float16, 3, False)),
]


def _inputs(case, seed):
    B, ctx, hq, hkv, d, dtype, split, hint = case
    lens = layout.ragged_lengths(B, 1, 3000, seed=seed) if ctx == "ragged" else ctx
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        B, lens, hq, hkv, d, dtype=dtype, device=DEV, page_table="permuted", seed=seed)
    opts = dk_lib.options(max_pages_per_seq=attention.plan_hint(indptr.cpu()) if hint else 0)
    return (q, kv, indptr, ids, last), split, opts


@pytest.mark.gpu
@pytest.mark.parametrize("pair", range(len(CASES)))
def test_noalloc_matches_the_workspace_entry_point(pair):
    lib = dk_lib.load()
    for k, case in enumerate(CASES[pair]):
        print(f"[case] noalloc pair {pair} call {k}: {case}", flush=True)
        tens, split, opts = _inputs(case, seed=10 * pair + k)
        got = _noalloc(lib, *tens, split, opts)
        want = _with_workspace(lib, *tens, split, opts)
        torch.cuda.synchronize()
        assert torch.isfinite(want).all()
        assert torch.equal(got, want), (pair, k, float((got.float() - want.float()).abs().max()))


@pytest.mark.gpu
def test_noalloc_under_graph_capture_replays_like_eager():
    # a caller that captures the decode step into a HIP graph: the captured call allocates
    # nothing; each replay (with eager work between) equals the eager call of its inputs
    lib = dk_lib.load()
    tens, split, opts = _inputs((8, 2048, 32, 8, 128, torch.float16, 0, False), seed=3)
    q = tens[0]
    out = torch.empty_like(q)
    st, ptrs, shape = _args(*tens, out)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        lib.dk_decode_attention_noalloc(*ptrs, *shape, split, ctypes.byref(opts), stream.cuda_stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        rc = lib.dk_decode_attention_noalloc(*ptrs, *shape, split, ctypes.byref(opts),
                                             stream.cuda_stream)
    dk_lib.check(rc, "dk_decode_attention_noalloc (captured)")
    for rep in range(3):
        q.copy_(torch.randn(q.shape, generator=torch.Generator(device=DEV).manual_seed(rep),
                            device=DEV).to(q.dtype))
        graph.replay()
        torch.cuda.synchronize()
        want = _with_workspace(lib, *tens, split, opts)
        torch.cuda.synchronize()
        assert torch.equal(out, want), rep


def test_noalloc_rejects_problems_beyond_the_static_scratch():
    # checked before any device call, so this runs without a GPU
    lib = dk_lib.load()
    st = dk_lib.DkStrides(32 * 128, 128, 2 * 16 * 8 * 128, 16 * 8 * 128, 8 * 128, 128,
                          32 * 128, 128)
    big = 8192                      # balanced partials of 8192 sequences x 8 kv heads
    assert dk_lib.workspace_bytes(big, 32, 8, 128, 0) > dk_lib.STATIC_SCRATCH_BYTES
    rc = lib.dk_decode_attention_noalloc(0x10000, 0x20000, 0x30000, 0x40000, 0x50000, 0x60000,
                                         big, 32, 8, 128, 16, 1 << 20, big * 512, dk_lib.DK_F16,
                                         ctypes.byref(st), 0, None, None)
    assert rc == dk_lib.DK_EWORKSPACE
    assert "static scratch" in lib.dk_last_error().decode()
    # an explicit split that fits is not rejected for its size (it then fails on the
    # missing device, or runs on a GPU box: not called here)
    assert dk_lib.workspace_bytes(32, 32, 8, 128, 16) <= dk_lib.STATIC_SCRATCH_BYTES
