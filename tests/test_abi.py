"""CPU tests of the C ABI (libdk_decode.so) and of the host-side argument checks.

No kernel is launched here: every call below is rejected by argument validation before
any HIP call, or is a pure size/layout helper.
"""
import ctypes
import re
from pathlib import Path

import pytest
import torch

import attention
import dk_lib
import layout

HEADER = Path(__file__).resolve().parent.parent / "include" / "dk_decode.h"


def _declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(dk_[a-z_0-9]+)\s*\(", text)))


def test_library_loads_and_reports_abi_version():
    lib = dk_lib.load()
    assert lib.dk_abi_version() == dk_lib.ABI_VERSION
    assert lib.dk_last_error() == b""


def test_every_declared_symbol_is_exported():
    lib = dk_lib.load()
    names = _declared_functions()
    assert len(names) >= 9
    for n in names:
        assert hasattr(lib, n), f"{n} declared in dk_decode.h but not exported"
    assert set(names) == set(dk_lib.SIGNATURES), "ctypes signatures out of sync with header"


def test_workspace_and_partials_layout():
    # partial_O (B,Hq,S,D) f32 + partial_m/l (B,Hq,S) f32, each 256-byte aligned
    assert dk_lib.workspace_bytes(32, 32, 8, 128, 1) == 0
    o, m, l, total = dk_lib.partials_layout(32, 32, 128, 4)
    rows = 32 * 32 * 4
    assert o == 0 and m == rows * 128 * 4 and l == m + rows * 4 and total == l + rows * 4
    assert dk_lib.workspace_bytes(32, 32, 8, 128, 4) == total
    # balanced schedule: (2048 workgroup slots + batch * kv_heads pairs) * 4 heads rows
    rows_b = (2048 + 32 * 8) * 4
    assert dk_lib.workspace_bytes(32, 32, 8, 128, 0) == \
        ((rows_b * 128 * 4 + 255) // 256 * 256) + ((rows_b * 4 + 255) // 256 * 256) + rows_b * 4
    assert dk_lib.workspace_bytes(32, 30, 8, 128, 4) == 0      # invalid shape
    assert dk_lib.partials_layout(3, 5, 64, 1)[3] > 0
    with pytest.raises(dk_lib.DecodeArgumentError):
        dk_lib.partials_layout(1, 1, 64, 0)



@pytest.mark.parametrize("batch,hkv", [(1, 4096), (3, 2049), (2, 8192), (5, 2048)])
def test_balanced_workspace_covers_every_slot_with_many_head_chunks(batch, hkv):
    # Pass 1 of the balanced schedule writes slot rows (hc*(Wg + batch) + j + b)*heads for
    # head chunk hc < HC and range j < Wg. With more head chunks than kMaxWaves = 2048 the
    # grid falls back to one range per head chunk (Wg = 1), so the last slot row is
    # HC*(1 + batch)*heads - 1: the workspace must hold at least that many rows.
    d, heads = 64, 1                      # MHA: one q head per kv head
    rows = hkv * (1 + batch) * heads
    o, m, l, total = dk_lib.partials_layout(1, rows, d, 1)   # `rows` rows of D + m + l
    assert dk_lib.workspace_bytes(batch, hkv, hkv, d, 0) >= total

def _call(lib, **kw):
    """dk_decode_attention_ex with a valid metric-shaped problem, overridden by kw.
    Pointers are fake non-NULL 256-aligned values: validation rejects before any use."""
    args = dict(q=0x10000, kv=0x20000, indptr=0x30000, indices=0x40000, last=0x50000,
                out=0x60000, ws=0x70000, ws_bytes=1 << 30, batch=2, hq=32, hkv=8, d=128,
                page=16, num_pages=64, num_indices=64, dtype=dk_lib.DK_F16, split=4,
                strides=None, opts=None)
    args.update(kw)
    st = args["strides"]
    if st is None:
        st = dk_lib.DkStrides(32 * 128, 128, 2 * 16 * 8 * 128, 16 * 8 * 128, 8 * 128, 128,
                              32 * 128, 128)
    opts = args["opts"] or dk_lib.options()
    return lib.dk_decode_attention_ex(
        args["q"], args["kv"], args["indptr"], args["indices"], args["last"], args["out"],
        args["ws"], args["ws_bytes"], args["batch"], args["hq"], args["hkv"], args["d"],
        args["page"], args["num_pages"], args["num_indices"], args["dtype"], ctypes.byref(st),
        args["split"], ctypes.byref(opts), None)


@pytest.mark.parametrize("kw,code,needle", [
    (dict(d=96), dk_lib.DK_EINVAL, "head_dim"),
    (dict(page=8), dk_lib.DK_EINVAL, "page_size"),
    (dict(hq=30), dk_lib.DK_EINVAL, "divisible"),
    (dict(dtype=7), dk_lib.DK_EINVAL, "dtype"),
    (dict(split=5000), dk_lib.DK_EINVAL, "split_kv"),
    (dict(split=-1), dk_lib.DK_EINVAL, "split_kv"),
    (dict(split=0, ws_bytes=4096), dk_lib.DK_EWORKSPACE, "workspace"),
    (dict(batch=-1), dk_lib.DK_EINVAL, "batch"),
    (dict(num_indices=-1), dk_lib.DK_EINVAL, "num_indices"),
    (dict(num_pages=0), dk_lib.DK_EINVAL, "page pool"),
    (dict(q=None), dk_lib.DK_ENULL, "non-NULL"),
    (dict(out=None), dk_lib.DK_ENULL, "out"),
    (dict(ws=None), dk_lib.DK_EWORKSPACE, "workspace"),
    (dict(ws_bytes=100), dk_lib.DK_EWORKSPACE, "workspace"),
    (dict(ws=0x70004), dk_lib.DK_EWORKSPACE, "aligned"),
    (dict(q=0x10002), dk_lib.DK_EUNSUPPORTED, "aligned"),
    (dict(strides=dk_lib.DkStrides(32 * 128, 127, 2 * 16 * 8 * 128, 16 * 8 * 128, 8 * 128,
                                   128, 32 * 128, 128)), dk_lib.DK_EUNSUPPORTED, "strides"),
    (dict(strides=dk_lib.DkStrides(-1, 128, 0, 0, 0, 0, 0, 0)), dk_lib.DK_EINVAL, "non-negative"),
    (dict(opts=dk_lib.options(qk_path=3)), dk_lib.DK_EINVAL, "qk_path"),
    (dict(opts=dk_lib.options(waves_per_group=3)), dk_lib.DK_EINVAL, "waves_per_group"),
    (dict(opts=dk_lib.options(waves_per_cu=40)), dk_lib.DK_EINVAL, "waves_per_cu"),
    (dict(opts=dk_lib.options(max_pages_per_seq=-1)), dk_lib.DK_EINVAL, "max_pages_per_seq"),
    (dict(opts=dk_lib.options(schedule=3)), dk_lib.DK_EINVAL, "schedule"),
    (dict(opts=dk_lib.options(kv_dtype=1)), dk_lib.DK_EINVAL, "kv_dtype"),
    (dict(opts=dk_lib.options(logit_cap=-1.0)), dk_lib.DK_EINVAL, "logit_cap"),
    # a negative scale would flip the kernels' -inf masking of dead tokens to +inf
    (dict(opts=dk_lib.options(sm_scale=-0.1)), dk_lib.DK_EINVAL, "sm_scale"),
    (dict(opts=dk_lib.options(sinks=0x1002)), dk_lib.DK_EINVAL, "sinks"),
    (dict(opts=dk_lib.options(sm_scale=float("inf"))), dk_lib.DK_EINVAL, "sm_scale"),
    (dict(opts=dk_lib.options(logit_cap=float("nan"))), dk_lib.DK_EINVAL, "logit_cap"),
    (dict(opts=dk_lib.options(k_scale=2.0)), dk_lib.DK_EINVAL, "fp8 cache only"),
    (dict(opts=dk_lib.options(kv_dtype=dk_lib.DK_KV_FP8_E4M3, v_scale=-1.0)),
     dk_lib.DK_EINVAL, "v_scale"),
    (dict(opts=dk_lib.options(kv_dtype=dk_lib.DK_KV_FP8_E4M3, k_scale=float("inf"))),
     dk_lib.DK_EINVAL, "k_scale"),
    # an fp8 cache's strides are bytes: 8 elements is no longer a 16-byte row
    (dict(opts=dk_lib.options(kv_dtype=dk_lib.DK_KV_FP8_E4M3),
          strides=dk_lib.DkStrides(32 * 128, 128, 2 * 16 * 8 * 128, 16 * 8 * 128, 8 * 128 + 8,
                                   128, 32 * 128, 128)), dk_lib.DK_EUNSUPPORTED, "strides"),
    # strides whose byte products would wrap int64: refused, not wrapped past the checks
    (dict(strides=dk_lib.DkStrides(32 * 128, 128, 2 * 16 * 8 * 128, 16 * 8 * 128, 1 << 62,
                                   128, 32 * 128, 128)), dk_lib.DK_EUNSUPPORTED, "2^40"),
    (dict(strides=dk_lib.DkStrides(1 << 40, 128, 2 * 16 * 8 * 128, 16 * 8 * 128, 8 * 128,
                                   128, 32 * 128, 128)), dk_lib.DK_EUNSUPPORTED, "2^40"),
    # each stride in range, but the pool they address spans more than 2^62 bytes
    (dict(num_pages=1 << 31, strides=dk_lib.DkStrides(32 * 128, 128, (1 << 40) - 8,
                                                      16 * 8 * 128, 8 * 128, 128, 32 * 128,
                                                      128)), dk_lib.DK_EUNSUPPORTED, "2^62"),
    (dict(batch=1 << 24, hq=32, strides=dk_lib.DkStrides((1 << 40) - 8, 128,
                                                         2 * 16 * 8 * 128, 16 * 8 * 128,
                                                         8 * 128, 128, 32 * 128, 128)),
     dk_lib.DK_EUNSUPPORTED, "2^62"),
])
def test_invalid_arguments_are_rejected_before_launch(kw, code, needle):
    lib = dk_lib.load()
    rc = _call(lib, **kw)
    assert rc == code
    assert needle in lib.dk_last_error().decode()


def test_split_one_needs_no_workspace_and_batch_zero_is_a_noop():
    lib = dk_lib.load()
    assert _call(lib, batch=0, q=None, kv=None, out=None) == dk_lib.DK_OK
    # split 1 with no workspace: validation passes (the launch itself is not attempted
    # here: a zero-sized batch returns before it)
    assert _call(lib, batch=0, split=1, ws=None, ws_bytes=0) == dk_lib.DK_OK


def test_null_strides_and_partials_entry_point():
    lib = dk_lib.load()
    rc = lib.dk_decode_attention(0x10000, 0x20000, 0x30000, 0x40000, 0x50000, 0x60000, None, 0,
                                 1, 32, 8, 128, 16, 8, 8, 0, None, 1, None)
    assert rc == dk_lib.DK_ENULL
    st = dk_lib.DkStrides()
    rc = lib.dk_decode_partials(0x10000, 0x20000, 0x30000, 0x40000, 0x50000, None, 0, 1, 32, 8,
                                128, 16, 8, 8, 0, ctypes.byref(st), 0, None, None)
    assert rc == dk_lib.DK_EWORKSPACE
    rc = lib.dk_merge_partials(None, 0, None, 1, 32, 96, 0, 0, 0, 4, None)
    assert rc == dk_lib.DK_EINVAL
    # a workspace not 256-byte aligned is refused before any launch (like pass 1's)
    rc = lib.dk_merge_partials(0x10010, 1 << 20, 0x20000, 1, 32, 128, 0, 4096, 128, 4, None)
    assert rc == dk_lib.DK_EWORKSPACE and b"aligned" in lib.dk_last_error()


# ---------------------------------------------------------------- Python-side checks

def _cpu_inputs(dtype=torch.float16, d=64):
    q, kv, indptr, ids, last, _ = layout.synthesize(2, 40, 8, 2, d, dtype=dtype, device="cpu")
    return q, kv, indptr, ids, last


def test_python_rejects_cpu_tensors_like_the_reference():
    q, kv, indptr, ids, last = _cpu_inputs()
    with pytest.raises(RuntimeError, match="q must be on CUDA"):
        attention.decode_attention(q, kv, indptr, ids, last, split_kv=4)


def test_python_error_type_is_both_value_and_runtime_error():
    assert issubclass(dk_lib.DecodeArgumentError, ValueError)
    assert issubclass(dk_lib.DecodeArgumentError, RuntimeError)
    assert issubclass(layout.LayoutError, ValueError)
    assert issubclass(layout.LayoutError, AssertionError)


def test_layout_validate_catches_each_invariant():
    q, kv, indptr, ids, last = _cpu_inputs()
    lay = layout.PagedKVLayout(16, 64, 2, torch.float16)
    lay.validate(kv, indptr, ids, last)
    with pytest.raises(layout.LayoutError, match="5-D"):
        lay.validate(kv[0], indptr, ids, last)
    with pytest.raises(layout.LayoutError, match="kv_indptr"):
        lay.validate(kv, indptr, ids[:-1], last)
    with pytest.raises(layout.LayoutError, match="> 0"):
        lay.validate(kv, indptr, ids, last * 0)
    with pytest.raises(layout.LayoutError, match="<= page_size"):
        lay.validate(kv, indptr, ids, last + 16)
    with pytest.raises(layout.LayoutError, match="out of range"):
        lay.validate(kv, indptr, ids + 100, last)
    with pytest.raises(layout.LayoutError, match="dtype"):
        lay.validate(kv.float(), indptr, ids, last)


def test_build_block_table_matches_reference_semantics():
    indptr, ids, last = layout.build_block_table(3, 33, 16, device="cpu")
    assert indptr.tolist() == [0, 3, 6, 9]
    assert ids.tolist() == list(range(9))
    assert last.tolist() == [1, 1, 1]
    _, _, last = layout.build_block_table(2, 32, 16, device="cpu")
    assert last.tolist() == [16, 16]


def test_synthesize_draws_q_first_then_kv():
    q, kv, *_ = layout.synthesize(2, 20, 4, 2, 64, device="cpu", seed=5)
    g = torch.Generator(device="cpu")
    g.manual_seed(5)
    q2 = torch.randn(2, 4, 64, dtype=torch.float16, generator=g)
    kv2 = torch.randn(4, 2, 16, 2, 64, dtype=torch.float16, generator=g)
    assert torch.equal(q, q2) and torch.equal(kv, kv2)
    with pytest.raises(ValueError):
        layout.synthesize(1, 16, 6, 4, 64, device="cpu")


def test_synthesize_paged_freelist_is_unique_and_ragged():
    lens = layout.ragged_lengths(64, 128, 8192, seed=3)
    q, kv, indptr, ids, last, _ = layout.synthesize_paged(
        64, lens, 4, 1, 64, device="cpu", page_table="freelist", pool_pages=20000, seed=3)
    assert kv.shape[0] == 20000
    assert len(set(ids.tolist())) == ids.numel()                      # no aliasing
    assert int(ids.min()) >= 0 and int(ids.max()) < 20000
    assert layout.seq_lens(indptr, last).tolist() == lens
    assert ((last >= 1) & (last <= 16)).all()


def test_attention_bytes_matches_reference_model():
    # bench/microbench_cuda.py:114-121 (Q + KV + O) plus the int32 tables
    b = layout.attention_bytes(32, 8192, 32, 8, 128)
    assert b == 1_074_266_112 + 4 * 33 + 4 * 32 * 512 + 4 * 32


def test_plan_hint_reads_host_indptr_only():
    import attention
    assert attention.plan_hint([0, 3, 3, 10, 11]) == 7
    assert attention.plan_hint(torch.tensor([0, 512, 1024], dtype=torch.int32)) == 512
    assert attention.plan_hint([0]) == 0


def test_options_struct_matches_header():
    # dk_options: qk_path, waves_per_group, waves_per_cu, schedule, max_pages_per_seq
    # (int32), sm_scale (float), kv_dtype (int32), k_scale, v_scale, logit_cap (float),
    # window, reserved[1] (int32), sinks (const float*): 56 bytes
    assert ctypes.sizeof(dk_lib.DkOptions) == 56
    assert dk_lib.DkOptions.sinks.offset == 48
    fields = [(f[0], f[1]) for f in dk_lib.DkOptions._fields_]
    hdr = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    body = hdr[hdr.index("int32_t qk_path"):hdr.index("} dk_options;")]
    declared = re.findall(r"(int32_t|float\*|float) (\w+)", body)
    ctype = {"int32_t": ctypes.c_int32, "float": ctypes.c_float, "float*": ctypes.c_void_p}
    assert [n for _, n in declared] == [n for n, _ in fields]
    for (ty, n), (_, cty) in zip(declared, fields):
        base = cty._type_ if issubclass(cty, ctypes.Array) else cty
        assert base is ctype[ty], n


def test_python_merge_partials_refuses_cpu_partials_and_bad_shapes():
    po = torch.zeros(1, 4, 2, 128)
    pm, pl = torch.zeros(1, 4, 2), torch.ones(1, 4, 2)
    with pytest.raises(dk_lib.DecodeArgumentError, match="on CUDA"):
        attention.merge_partials(po, pm, pl)
    with pytest.raises(dk_lib.DecodeArgumentError, match=r"\(B, Hq, S\)"):
        attention.merge_partials(po, pm[:, :3], pl)
    with pytest.raises(dk_lib.DecodeArgumentError, match=r"\(B, Hq, S, D\)"):
        attention.merge_partials(po[0], pm, pl)


def test_merge_partials_refuses_out_strides_that_would_wrap():
    lib = dk_lib.load()
    rc = lib.dk_merge_partials(0x70000, 1 << 30, 0x60000, 2, 32, 128, dk_lib.DK_F16,
                               1 << 62, 128, 4, None)
    assert rc == dk_lib.DK_EUNSUPPORTED and "2^40" in lib.dk_last_error().decode()
    rc = lib.dk_merge_partials(0x70000, 1 << 30, 0x60000, 1 << 22, 32, 128, dk_lib.DK_F16,
                               (1 << 40) - 8, 128, 1, None)
    assert rc == dk_lib.DK_EUNSUPPORTED and "2^62" in lib.dk_last_error().decode()


def test_build_page_table_refuses_a_stride_that_would_wrap():
    lib = dk_lib.load()
    fake = ctypes.c_void_p(256)
    rc = lib.dk_build_page_table(fake, 1 << 62, fake, fake, 2, 16, fake, fake, 64, fake, None)
    assert rc == dk_lib.DK_EUNSUPPORTED and "req_stride" in lib.dk_last_error().decode()


@pytest.mark.parametrize("q_b,kv_p,num_pages", [(1 << 62, 8192, 64), (4096, 1 << 45, 64),
                                                 (4096, (1 << 40) - 8, 1 << 31)])
def test_append_refuses_strides_that_would_wrap(q_b, kv_p, num_pages):
    # the checks come before any pointer is used; every call is refused on the host
    lib = dk_lib.load()
    fake = ctypes.c_void_p(256)
    st = dk_lib.DkStrides(q_b, 128, kv_p, 4096, 1024, 128, 0, 0)
    rc = lib.dk_append_kv(fake, fake, fake, 1024, 128, fake, None, fake, fake, fake, None,
                          None, 0, 2, 32, 8, 128, 16, num_pages, 64, dk_lib.DK_F16,
                          ctypes.byref(st), None)
    assert rc == dk_lib.DK_EUNSUPPORTED and "2^62" in lib.dk_last_error().decode()
