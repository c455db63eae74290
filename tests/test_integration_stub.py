"""The reference-side binding a maintainer would paste into src/attention.py (the fenced
Python block under "Binding from the reference's Python" in the repository's integration
guide), run as written:
a bare ctypes stub over the plain dk_decode_attention entry point, which takes no
options (split_kv 0 is the balanced schedule without a plan hint).

CPU: the stub is found, compiles, and its argtypes agree with include/dk_decode.h and the
package's own binding (dk_lib.SIGNATURES). GPU: the stub against the fp32 oracle at
config 1 (B=2 ctx 512, contiguous pages) and at the metric config (B=32 ctx 8192, 32/8/128
fp16, permuted pages, all 32 sequences), for split_kv 1, 4 and 0 -- the reference's
src/attention.py:26-58 call shapes -- and bitwise equal to the package's decode_attention.
"""
import ctypes
import re
from pathlib import Path

import pytest
import torch

import dk_lib
import layout
from helpers import err_stats, to_np
from oracle import reference as ref

ROOT = Path(__file__).resolve().parent.parent
GUIDE = ROOT / "INTEGRATION.md"     # the integration guide holding the binding stub
DEV = "cuda"


def _stub_source() -> str:
    """The first fenced Python block after the guide's binding heading."""
    text = GUIDE.read_text()
    at = text.index("## Binding from the reference's Python")
    m = re.search(r"```python\n(.*?)```", text[at:], re.S)
    assert m, "no python block under the binding heading"
    return m.group(1)


def _load_stub():
    src = _stub_source().replace("/path/to/libdk_decode.so", str(dk_lib.LIB_PATH))
    ns = {}
    exec(compile(src, GUIDE.name, "exec"), ns)
    return ns


def test_stub_matches_the_header_and_the_package_binding():
    ns = _load_stub()
    lib = ns["_lib"]
    want_res, want_args = dk_lib.SIGNATURES["dk_decode_attention"]
    got = lib.dk_decode_attention.argtypes
    assert len(got) == len(want_args)
    for g, w in zip(got, want_args):
        if hasattr(w, "_type_") and issubclass(w, ctypes._Pointer):
            assert issubclass(g, ctypes._Pointer)
            assert [f[0] for f in g._type_._fields_] == [f[0] for f in w._type_._fields_]
        else:
            assert ctypes.sizeof(g) == ctypes.sizeof(w), (g, w)
    assert lib.dk_decode_attention.restype == want_res
    # the header declares as many parameters as the stub binds
    header = (ROOT / "include" / "dk_decode.h").read_text()
    decl = re.search(r"int dk_decode_attention\((.*?)\);", header, re.S).group(1)
    assert decl.count(",") + 1 == len(got)
    # workspace sizes agree with the package's
    for args in ((2, 32, 8, 128, 4), (32, 32, 8, 128, 0), (1, 32, 8, 64, 1)):
        assert lib.dk_workspace_bytes(*args) == dk_lib.workspace_bytes(*args)


@pytest.mark.gpu
@pytest.mark.parametrize("config", ["config1", "metric"])
def test_stub_against_oracle(config):
    import attention
    ns = _load_stub()
    if config == "config1":
        q, kv, indptr, ids, last, _ = layout.synthesize_paged(
            2, 512, 32, 8, 128, device=DEV, page_table="contiguous", seed=0)
    else:
        q, kv, indptr, ids, last, _ = layout.synthesize_paged(
            32, 8192, 32, 8, 128, device=DEV, page_table="permuted", seed=1)
    want = ref.reference_attention_paged(to_np(q), to_np(kv), to_np(indptr), to_np(ids),
                                         to_np(last))
    for split in (1, 4, 0):
        print(f"[case] integration stub {config} split_kv={split}", flush=True)
        out = ns["decode_attention"](q, kv, indptr, ids, last, split_kv=split)
        torch.cuda.synchronize()
        mx, mean = err_stats(out, want)
        assert mx <= 1e-2 and mean <= 1e-3, (config, split, mx, mean)
        pkg = attention.decode_attention(q, kv, indptr, ids, last, split_kv=split)
        torch.cuda.synchronize()
        assert torch.equal(out, pkg), (config, split)
