"""CPU tests that pin the oracle (oracle/) before it is trusted to check the HIP kernels.

Each check is independent of the oracle's own formulas: the reference's hand-worked
example, closed forms, torch's scaled_dot_product_attention in float64, and brute-force
float64 fixtures from tests/golden/make_golden.py. The mutation tests plant a plausible
mistake in a copy of the oracle and show that a check catches it.
"""
import math

import numpy as np
import pytest
import torch

from helpers import load_golden
from oracle import reference as ref
from oracle import split_kv as skv

GOLDEN_CASES = ["tiny_f16", "gqa4_d64_f16", "gqa8_d128_bf16", "mha_d128_f16"]


def _paged(lens, Hq, Hkv, D, P, seed, pool=0, dtype=np.float16, permute=True):
    """Random paged inputs (numpy): q, kv, indptr, indices, last."""
    rng = np.random.default_rng(seed)
    pages = [math.ceil(n / P) for n in lens]
    last = np.array([n - (p - 1) * P if p else P for n, p in zip(lens, pages)], np.int32)
    need = sum(pages)
    pool = max(pool, need, 1)
    ids = (rng.permutation(pool)[:need] if permute else np.arange(need)).astype(np.int32)
    indptr = np.zeros(len(lens) + 1, np.int32)
    indptr[1:] = np.cumsum(pages)
    q = rng.standard_normal((len(lens), Hq, D)).astype(dtype)
    kv = rng.standard_normal((pool, 2, P, Hkv, D)).astype(dtype)
    return q, kv, indptr, ids, last


def _sdpa(q, K, V):
    """torch SDPA in float64 with enable_gqa (kv head = q head // G). q (B,Hq,D), K,V (B,S,Hkv,D)."""
    qt = torch.from_numpy(np.asarray(q, np.float64))[:, :, None, :]
    kt = torch.from_numpy(np.asarray(K, np.float64)).permute(0, 2, 1, 3)
    vt = torch.from_numpy(np.asarray(V, np.float64)).permute(0, 2, 1, 3)
    o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, enable_gqa=True)
    return o[:, :, 0, :].numpy()


# ---------------------------------------------------------------- known answers

def _primer_inputs():
    """writeup/cuda_primer.md:31-43: D=4, P=2, one head, tokens
    K = [1,0,1,0], [0,1,0,1], [1,0,0,1], [0,1,1,0], all V = 0.5, q = [1,1,0,0]."""
    kv = np.zeros((2, 2, 2, 1, 4), np.float16)
    K = [[1, 0, 1, 0], [0, 1, 0, 1], [1, 0, 0, 1], [0, 1, 1, 0]]
    for t, k in enumerate(K):
        kv[t // 2, 0, t % 2, 0] = k
        kv[t // 2, 1, t % 2, 0] = 0.5
    q = np.array([[[1, 1, 0, 0]]], np.float16)
    return q, kv, np.array([0, 2], np.int32), np.array([0, 1], np.int32), np.array([2], np.int32)


def test_primer_known_answer():
    q, kv, indptr, ids, last = _primer_inputs()
    out = ref.reference_attention_paged(q, kv, indptr, ids, last)
    assert np.array_equal(out, np.full((1, 1, 4), 0.5, np.float32))


def test_primer_split_partials():
    # writeup/cuda_primer.md:505-540: two splits, each m=0.5, l=2.0, O=[1,1,1,1]
    q, kv, indptr, ids, last = _primer_inputs()
    O, m, l = skv.split_partials(q, kv, indptr, ids, last, 2)
    np.testing.assert_allclose(m[0, 0], [0.5, 0.5], rtol=0, atol=1e-15)
    np.testing.assert_allclose(l[0, 0], [2.0, 2.0], rtol=0, atol=1e-15)
    np.testing.assert_allclose(O[0, 0], np.ones((2, 4)), rtol=0, atol=1e-15)
    np.testing.assert_allclose(skv.merge_partials(O, m, l), np.full((1, 1, 4), 0.5), atol=1e-15)


# ---------------------------------------------------------------- closed forms

def test_single_token_returns_v0_exactly():
    q, kv, indptr, ids, last = _paged([1, 1, 1], 8, 2, 64, 16, seed=3)
    out = ref.reference_attention_paged(q, kv, indptr, ids, last)
    for b in range(3):
        v0 = kv[ids[indptr[b]], 1, 0].astype(np.float32)        # (Hkv, D)
        np.testing.assert_array_equal(out[b], np.repeat(v0, 4, axis=0))


def test_constant_v_gives_constant():
    q, kv, indptr, ids, last = _paged([37, 5], 4, 2, 16, 4, seed=4)
    kv[:, 1] = np.float16(-1.25)
    out = ref.reference_attention_paged(q, kv, indptr, ids, last)
    np.testing.assert_allclose(out, -1.25, rtol=0, atol=1e-6)


def test_equal_keys_give_mean_of_v():
    q, kv, indptr, ids, last = _paged([23], 4, 1, 8, 4, seed=5)
    kv[:, 0] = kv[0, 0, 0]
    out = ref.reference_attention_paged(q, kv, indptr, ids, last)
    K, V = ref.gather_paged_to_dense(kv, indptr, ids, last)
    np.testing.assert_allclose(out[0], np.repeat(V[0].mean(axis=0), 4, axis=0), atol=1e-6)


def test_dominant_key_selects_its_value():
    q, kv, indptr, ids, last = _paged([40], 2, 1, 8, 4, seed=6)
    q[:] = 0
    q[0, :, 0] = 1
    K, V = ref.gather_paged_to_dense(kv, indptr, ids, last)
    t = 17
    kv[ids[t // 4], 0, t % 4, 0, 0] = np.float16(400.0)     # score 400/sqrt(8) >> others
    out = ref.reference_attention_paged(q, kv, indptr, ids, last)
    np.testing.assert_allclose(out[0, 0], V[0, t, 0], atol=1e-6)


# ---------------------------------------------------------------- library cross-check

@pytest.mark.parametrize("lens,Hq,Hkv,D,P", [
    ([64, 64], 32, 8, 128, 16), ([37, 37, 37], 8, 2, 64, 16), ([5], 4, 4, 32, 4),
    ([130, 130], 8, 1, 64, 16), ([16], 16, 4, 256, 16),
])
def test_against_sdpa_float64(lens, Hq, Hkv, D, P):
    q, kv, indptr, ids, last = _paged(lens, Hq, Hkv, D, P, seed=sum(lens) + Hq)
    out = ref.reference_attention_paged(q, kv, indptr, ids, last)
    K, V = ref.gather_paged_to_dense(kv, indptr, ids, last)
    np.testing.assert_allclose(out, _sdpa(q.astype(np.float64), K, V), rtol=0, atol=2e-6)


def test_gather_identity_table_is_reshape():
    # with the identity block table, the gather is a reshape truncated to seq_len
    B, ctx, Hkv, D, P = 3, 45, 2, 8, 16
    q, kv, indptr, ids, last = _paged([ctx] * B, 4, Hkv, D, P, seed=7, permute=False)
    K, V = ref.gather_paged_to_dense(kv, indptr, ids, last)
    Kp = kv[:, 0].reshape(B, -1, Hkv, D)[:, :ctx].astype(np.float32)
    Vp = kv[:, 1].reshape(B, -1, Hkv, D)[:, :ctx].astype(np.float32)
    np.testing.assert_array_equal(K, Kp)
    np.testing.assert_array_equal(V, Vp)


# ---------------------------------------------------------------- golden fixtures

@pytest.mark.parametrize("name", GOLDEN_CASES)
def test_oracle_matches_golden(name):
    z, _ = load_golden(name)
    out = ref.reference_attention_paged(z["q_f32"], z["kv_f32"], z["kv_indptr"],
                                        z["kv_indices"], z["kv_last_page_len"])
    np.testing.assert_allclose(out, z["out"], rtol=0, atol=5e-6)


@pytest.mark.parametrize("name", GOLDEN_CASES)
def test_split_partials_match_golden(name):
    z, _ = load_golden(name)
    splits = sorted(int(k[len("partial_m_s"):]) for k in z if k.startswith("partial_m_s"))
    assert splits
    for S in splits:
        O, m, l = skv.split_partials(z["q_f32"], z["kv_f32"], z["kv_indptr"], z["kv_indices"],
                                     z["kv_last_page_len"], S)
        np.testing.assert_allclose(m, z[f"partial_m_s{S}"], rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(l, z[f"partial_l_s{S}"], rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(O, z[f"partial_o_s{S}"], rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(skv.merge_partials(O, m, l), z["out"], atol=1e-12)


# ---------------------------------------------------------------- split semantics

def test_partition_matches_reference_formula():
    # attention_ext.cu:249-252: pps = ceil(N/S); [s*pps, min(s*pps+pps, N))
    assert skv.partition(10, 4) == [(0, 3), (3, 6), (6, 9), (9, 10)]
    assert skv.partition(2, 4) == [(0, 1), (1, 2), (2, 2), (2, 2)]   # empty splits
    assert skv.partition(9, 3) == [(0, 3), (3, 6), (6, 9)]
    assert skv.partition(0, 3) == [(0, 0), (0, 0), (0, 0)]


@pytest.mark.parametrize("S", [1, 2, 3, 5, 7, 64])
def test_split_count_does_not_change_result(S):
    lens = [1, 17, 30, 64, 200, 0]
    q, kv, indptr, ids, last = _paged(lens, 8, 2, 32, 16, seed=11, pool=40)
    want = ref.reference_attention_paged(q, kv, indptr, ids, last)
    got = skv.split_kv_attention(q, kv, indptr, ids, last, S)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6)


def test_empty_split_sentinel_and_empty_sequence():
    q, kv, indptr, ids, last = _paged([20, 0], 2, 1, 8, 16, seed=12)
    O, m, l = skv.split_partials(q, kv, indptr, ids, last, 4)
    # sequence 0 has 2 pages: splits 2, 3 are empty; sequence 1 has none
    assert (m[0, :, 2:] == skv.EMPTY_M).all() and (l[0, :, 2:] == 0).all()
    assert (m[1] == skv.EMPTY_M).all() and (O[1] == 0).all()
    out = skv.merge_partials(O, m, l)
    assert np.array_equal(out[1], np.zeros_like(out[1]))
    np.testing.assert_array_equal(ref.reference_attention_paged(q, kv, indptr, ids, last)[1], 0)


# ---------------------------------------------------------------- ragged batches

def test_literal_padding_equals_masked_for_uniform_lengths():
    q, kv, indptr, ids, last = _paged([48, 48, 48], 8, 2, 64, 16, seed=13)
    a = ref.reference_attention_paged(q, kv, indptr, ids, last)
    b = ref.reference_attention_paged(q, kv, indptr, ids, last, literal=True)
    np.testing.assert_allclose(a, b, rtol=0, atol=1e-6)


def test_literal_padding_is_wrong_for_ragged_batches():
    # The reference pads short sequences with zero keys and softmaxes over them
    # (src/reference.py:40-43,91-94). With small scores the padding takes most of the
    # weight: the short sequence's output shrinks far beyond the 1e-2 tolerance.
    q, kv, indptr, ids, last = _paged([16, 1024], 8, 2, 64, 16, seed=14)
    q = (q.astype(np.float32) / 8).astype(np.float16)
    masked = ref.reference_attention_paged(q, kv, indptr, ids, last)
    literal = ref.reference_attention_paged(q, kv, indptr, ids, last, literal=True)
    assert np.abs(masked[0] - literal[0]).max() > 1e-1
    np.testing.assert_allclose(masked[1], literal[1], atol=1e-6)   # the longest is unaffected



# ---- the torch restatement of the literal path (bench.py's CPU baseline)

@pytest.mark.parametrize("lens,Hq,Hkv,D", [([48, 48, 48], 8, 2, 64), ([16, 1024, 0, 33], 8, 2, 64),
                                          ([300, 5], 32, 8, 128), ([17], 4, 4, 64)])
def test_torch_literal_path_matches_numpy_literal_oracle(lens, Hq, Hkv, D):
    from oracle import reference_torch as rt
    q, kv, indptr, ids, last = _paged(lens, Hq, Hkv, D, 16, seed=len(lens) + D)
    tq, tkv = torch.from_numpy(q), torch.from_numpy(kv)
    tabs = [torch.from_numpy(a) for a in (indptr, ids, last)]
    K, V = rt.gather_dense(tkv, *tabs)
    K0, V0 = ref.gather_paged_to_dense(kv, indptr, ids, last)
    np.testing.assert_array_equal(K.numpy(), K0)            # a copy: bit-exact
    np.testing.assert_array_equal(V.numpy(), V0)
    got = rt.reference_attention_paged_literal(tq, tkv, *tabs).numpy()
    want = ref.reference_attention_paged(q, kv, indptr, ids, last, literal=True)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6)
    if len(set(lens)) == 1:      # uniform lengths: also the masked (and SDPA-pinned) form
        np.testing.assert_allclose(got, ref.reference_attention_paged(q, kv, indptr, ids, last),
                                   rtol=0, atol=2e-6)


def test_torch_literal_path_catches_a_planted_gqa_mistake():
    # repeat (tile) instead of repeat_interleave puts q head h on kv head h % Hkv
    from oracle import reference_torch as rt
    q, kv, indptr, ids, last = _paged([64, 64], 8, 2, 64, 16, seed=5)
    tabs = [torch.from_numpy(a) for a in (indptr, ids, last)]
    K, V = rt.gather_dense(torch.from_numpy(kv), *tabs)
    g = 4
    k = K.repeat(1, 1, g, 1).permute(0, 2, 3, 1)
    v = V.repeat(1, 1, g, 1).permute(0, 2, 1, 3)
    qf = torch.from_numpy(q).float()
    bad = torch.matmul(torch.softmax(torch.matmul(qf.unsqueeze(2) * 64 ** -0.5, k), -1), v)
    want = ref.reference_attention_paged(q, kv, indptr, ids, last)
    assert np.abs(bad.squeeze(2).numpy() - want).max() > 1e-1


# ---------------------------------------------------------------- planted mistakes

def _oracle_with_modulo_gqa(q, kv, indptr, ids, last):
    """Copy of the oracle with a plausible bug: kv head = q head % Hkv (not // G)."""
    B, Hq, D = q.shape
    Hkv = kv.shape[3]
    perm = [h % Hkv for h in range(Hq)]
    out = np.zeros((B, Hq, D), np.float32)
    for b in range(B):
        k, v = ref._sequence_kv(kv, indptr, ids, last, b)
        for h in range(Hq):
            qs = (q[b, h].astype(np.float32) * np.float32(D ** -0.5))[None, None]
            out[b, h] = ref._softmax_attend(qs, k[:, perm[h]:perm[h] + 1],
                                            v[:, perm[h]:perm[h] + 1])[0, 0]
    return out


def test_planted_gqa_mistake_is_caught_by_sdpa():
    q, kv, indptr, ids, last = _paged([40, 40], 8, 2, 32, 16, seed=15)
    K, V = ref.gather_paged_to_dense(kv, indptr, ids, last)
    want = _sdpa(q.astype(np.float64), K, V)
    good = ref.reference_attention_paged(q, kv, indptr, ids, last)
    bad = _oracle_with_modulo_gqa(q, kv, indptr, ids, last)
    assert np.abs(good - want).max() < 2e-6
    assert np.abs(bad - want).max() > 1e-2


def test_planted_scale_mistake_is_caught_by_primer():
    # scaling by 1/D instead of 1/sqrt(D) breaks the primer's partial m = 0.5
    q, kv, indptr, ids, last = _primer_inputs()
    _, m_good, _ = skv.split_partials(q, kv, indptr, ids, last, 2)
    _, m_bad, _ = skv.split_partials(q, kv, indptr, ids, last, 2, scale=1 / 4)
    assert np.allclose(m_good, 0.5) and not np.allclose(m_bad, 0.5)


def test_planted_last_page_mistake_is_caught_by_golden():
    # using page_size tokens on the last page (ignoring kv_last_page_len) changes results
    z, _ = load_golden("gqa4_d64_f16")
    full = np.full_like(z["kv_last_page_len"], 16)
    bad = ref.reference_attention_paged(z["q_f32"], z["kv_f32"], z["kv_indptr"],
                                        z["kv_indices"], full)
    assert np.abs(bad - z["out"]).max() > 1e-2


# ---------------------------------------------------------------- page table from a slot map

from oracle import page_table as ptab  # noqa: E402


def _slot_map(lens, rows, seed, pool_pages=None):
    """req_to_token filled by a 16-token-page allocator over a shuffled free list."""
    rng = np.random.default_rng(seed)
    need = sum(-(-n // 16) for n in lens)
    perm = list(rng.permutation(pool_pages or need + 5))
    r2t = np.full((max(rows) + 1, max(lens + [1]) + 16), -1, np.int64)
    for r, n in zip(rows, lens):
        for p in range(-(-n // 16)):
            page = int(perm.pop())
            for t in range(p * 16, min(n, p * 16 + 16)):
                r2t[r, t] = page * 16 + t % 16
    return r2t


def test_page_table_known_answer():
    # hand-built: request in row 1 has 20 tokens on pages 7 then 3; row 0 has 16 tokens on
    # page 5; row 2 is empty
    r2t = np.zeros((3, 40), np.int64)
    r2t[1, :16] = 7 * 16 + np.arange(16)
    r2t[1, 16:20] = 3 * 16 + np.arange(4)
    r2t[0, :16] = 5 * 16 + np.arange(16)
    indptr, indices, last = ptab.build_page_table(r2t, [1, 0, 2], [20, 16, 0])
    assert indptr.tolist() == [0, 2, 3, 3]
    assert indices.tolist() == [7, 3, 5]
    assert last.tolist() == [4, 16, 0]


@pytest.mark.parametrize("seed", range(4))
def test_page_table_round_trip_reproduces_token_slots(seed):
    # the page table must describe exactly the slots the map holds, token by token, and
    # satisfy the layout invariants (src/layout.md:171-178)
    rng = np.random.default_rng(seed)
    lens = [int(x) for x in rng.integers(0, 80, size=9)]
    rows = [int(x) for x in rng.permutation(12)[:9]]
    r2t = _slot_map(lens, rows, seed)
    indptr, indices, last = ptab.build_page_table(r2t, rows, lens)
    assert indptr[0] == 0 and indptr[-1] == len(indices)
    for b, (r, n) in enumerate(zip(rows, lens)):
        np.testing.assert_array_equal(ptab.token_slots(indptr, indices, last, b), r2t[r, :n])
        assert (last[b] == 0) == (n == 0) and 0 <= last[b] <= 16


def test_planted_page_table_mistake_is_caught_by_round_trip():
    # a last-page length off by one (n % 16 instead of the 1..16 range) breaks the round
    # trip for lengths that are multiples of 16
    lens, rows = [32, 5], [0, 1]
    r2t = _slot_map(lens, rows, 3)
    indptr, indices, last = ptab.build_page_table(r2t, rows, lens)
    bad_last = np.array([n % 16 for n in lens], np.int32)
    ok = all(np.array_equal(ptab.token_slots(indptr, indices, last, b), r2t[r, :n])
             for b, (r, n) in enumerate(zip(rows, lens)))
    bad = all(np.array_equal(ptab.token_slots(indptr, indices, bad_last, b), r2t[r, :n])
              for b, (r, n) in enumerate(zip(rows, lens)))
    assert ok and not bad


# ---------------------------------------------------------------- RoPE + cache write

from oracle import append as oapp  # noqa: E402


def _hf_rope(x, pos, inv_freq):
    """transformers' Llama rotation (apply_rotary_pos_emb, rotate_half) in float64 with the
    same fp32 angles: an independent implementation of the rotate-half convention."""
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    ang = torch.from_numpy((np.float32(pos) * np.asarray(inv_freq, np.float32)).astype(np.float64))
    emb = torch.cat([ang, ang])
    cos, sin = emb.cos()[None, None], emb.sin()[None, None]
    t = torch.from_numpy(np.asarray(x, np.float64))[None, :, None, :]   # (1, H, 1, D)
    q_rot, _ = apply_rotary_pos_emb(t, t, cos, sin, unsqueeze_dim=1)
    return q_rot[0, :, 0].numpy()


@pytest.mark.parametrize("pos", [0, 1, 17, 2047, 70000])
def test_rope_matches_transformers_llama(pos):
    rng = np.random.default_rng(pos)
    x = rng.standard_normal((4, 64))
    inv = 1.0 / (500000.0 ** (np.arange(0, 64, 2) / 64))
    np.testing.assert_allclose(oapp.rope(x, pos, inv), _hf_rope(x, pos, inv), rtol=0, atol=1e-12)


def test_rope_identities():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 16))
    inv = 2.0 ** -np.arange(8)                      # exact angles for small integer positions
    np.testing.assert_array_equal(oapp.rope(x, 0, inv), x)
    for style in (0, 1):
        y = oapp.rope(x, 5, inv, style)
        # each rotated pair keeps its length
        if style == 0:
            n0, n1 = x[:, :8] ** 2 + x[:, 8:] ** 2, y[:, :8] ** 2 + y[:, 8:] ** 2
        else:
            n0, n1 = x[:, 0::2] ** 2 + x[:, 1::2] ** 2, y[:, 0::2] ** 2 + y[:, 1::2] ** 2
        np.testing.assert_allclose(n1, n0, rtol=1e-12)
        # rotations compose: R(3) R(5) = R(8)
        np.testing.assert_allclose(oapp.rope(oapp.rope(x, 3, inv, style), 5, inv, style),
                                   oapp.rope(x, 8, inv, style), atol=1e-12)


def test_rope_interleaved_known_answer():
    # D = 4, GPT-J pairs (0,1), (2,3); inv_freq (pi/2, 0) at position 1: the first pair
    # turns by 90 degrees, the second not at all
    y = oapp.rope([1.0, 2.0, 3.0, 4.0], 1, [np.pi / 2, 0.0], style=1)
    np.testing.assert_allclose(y, [-2.0, 1.0, 3.0, 4.0], atol=1e-6)


def test_append_writes_the_last_slot_of_each_sequence():
    kv = np.zeros((4, 2, 16, 1, 2))
    indptr, indices, last = [0, 2, 2, 3], [3, 1, 0], [5, 1, 16]
    k_new = np.array([[[1.0, 2.0]], [[3.0, 4.0]], [[5.0, 6.0]]])
    v_new = k_new + 10
    out, _ = oapp.append_kv(kv, None, k_new, v_new, indptr, indices, last)
    assert out[1, 0, 4, 0].tolist() == [1.0, 2.0] and out[1, 1, 4, 0].tolist() == [11.0, 12.0]
    assert out[0, 0, 15, 0].tolist() == [5.0, 6.0]
    assert np.count_nonzero(out) == 8                # sequence 1 has no pages: skipped


def test_planted_rope_sign_mistake_is_caught_by_transformers():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((2, 8))
    inv = 1.0 / (10000.0 ** (np.arange(0, 8, 2) / 8))
    ang = np.float32(9) * inv.astype(np.float32)
    bad = x.copy()
    bad[:, :4] = x[:, :4] * np.cos(ang) + x[:, 4:] * np.sin(ang)     # sign of sin flipped
    bad[:, 4:] = x[:, 4:] * np.cos(ang) - x[:, :4] * np.sin(ang)
    assert np.abs(bad - _hf_rope(x, 9, inv)).max() > 1e-2
    np.testing.assert_allclose(oapp.rope(x, 9, inv), _hf_rope(x, 9, inv), atol=1e-12)


# ---- fp8 (E4M3) cache format: oracle/fp8.py

def test_fp8_known_answers():
    from oracle import fp8
    known = {0x38: 1.0, 0x7E: 448.0, 0xFE: -448.0, 0x08: 2.0 ** -6, 0x01: 2.0 ** -9,
             0x07: 7 * 2.0 ** -9, 0x40: 2.0, 0x3C: 1.5, 0x00: 0.0, 0xB8: -1.0}
    for code, want in known.items():
        assert fp8.decode(code) == want, hex(code)
    assert np.signbit(fp8.decode(0x80)) and fp8.decode(0x80) == 0.0
    vals = fp8.decode(np.arange(256))
    assert np.isnan(vals).sum() == 2 and np.isnan(vals[0x7F]) and np.isnan(vals[0xFF])
    assert np.isfinite(vals).sum() == 254 and np.nanmax(vals) == 448.0
    # the non-negative finite codes are monotone: encode's search relies on it
    assert np.all(np.diff(vals[:0x7F]) > 0)


def test_fp8_decode_matches_torch_all_codes():
    from oracle import fp8
    codes = np.arange(256, dtype=np.uint8)
    t = torch.from_numpy(codes).view(torch.float8_e4m3fn).double().numpy()
    d = fp8.decode(codes)
    fin = np.isfinite(t)
    assert np.array_equal(np.isnan(t), np.isnan(d))
    assert np.array_equal(t[fin], d[fin]) and np.array_equal(np.signbit(t[fin]),
                                                             np.signbit(d[fin]))


def test_fp8_encode_matches_torch_rounding():
    from oracle import fp8
    fin = np.unique(fp8.decode(np.arange(0x7F)))
    mids = (fin[1:] + fin[:-1]) / 2                  # every tie
    x = np.concatenate([fin, -fin, mids, -mids, np.linspace(-520, 520, 100001),
                        np.array([448, 449, 463.9, 464, 464.1, 480, 1e9, -464, -470, np.nan,
                                  -0.0, 2.0 ** -10, 2.0 ** -11, 3 * 2.0 ** -11])])
    x = x.astype(np.float32)
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(fp8.encode(x), want)
    # round trip of every finite code
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], np.uint8)
    assert np.array_equal(fp8.encode(fp8.decode(codes)), codes)


def test_planted_fp8_bias_mistake_is_caught_by_torch():
    from oracle import fp8
    codes = np.arange(256, dtype=np.uint8)
    t = torch.from_numpy(codes).view(torch.float8_e4m3fn).double().numpy()
    wrong = fp8.decode(codes) * 2.0                  # exponent bias 6 instead of 7
    fin = np.isfinite(t)
    assert not np.array_equal(t[fin], wrong[fin])


def test_fp8_saturating_encode_matches_torch_clamp_then_convert():
    from oracle import fp8
    x = np.concatenate([np.linspace(-600, 600, 20001), [np.inf, -np.inf, np.nan, 464.0, -470.0]])
    x = x.astype(np.float32)
    want = torch.from_numpy(x).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    assert np.array_equal(fp8.encode_saturating(x), want.numpy())
    ranks = fp8.signed_rank(np.arange(256, dtype=np.uint8))
    vals = fp8.decode(np.arange(256, dtype=np.uint8))
    fin = np.isfinite(vals)
    # rank order is value order (ties only between +0 and -0)
    order = np.argsort(vals[fin], kind="stable")
    assert np.all(np.diff(ranks[fin][order]) >= 0)


def test_fp8_append_oracle_matches_float_append_then_torch_quantization():
    from oracle import append as oapp
    rng = np.random.default_rng(4)
    pages, hkv, d = 6, 2, 16
    codes = rng.integers(0, 256, (pages, 2, 16, hkv, d)).astype(np.uint8)
    q = rng.standard_normal((2, 4, d)).astype(np.float32)
    k_new = (rng.standard_normal((2, hkv, d)) * 300).astype(np.float32)   # some clamp
    v_new = rng.standard_normal((2, hkv, d)).astype(np.float32)
    indptr, ids, last = np.array([0, 2, 5]), np.array([3, 1, 0, 5, 2]), np.array([7, 16])
    inv = 1.0 / (10000.0 ** (np.arange(0, d, 2) / d))
    got, qo = oapp.append_kv_fp8(codes, q, k_new, v_new, indptr, ids, last, 0.5, 0.25,
                                 inv_freq=inv)
    flt, q_want = oapp.append_kv(np.zeros((pages, 2, 16, hkv, d), np.float32), q, k_new, v_new,
                                 indptr, ids, last, inv_freq=inv)
    np.testing.assert_array_equal(qo, q_want)
    for page, slot in ((1, 6), (2, 15)):
        for r, sc in ((0, 0.5), (1, 0.25)):
            x = torch.from_numpy(flt[page, r, slot].astype(np.float32)) / np.float32(sc)
            want = x.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
            np.testing.assert_array_equal(got[page, r, slot], want)
    untouched = np.ones((pages, 16), bool)
    untouched[1, 6] = untouched[2, 15] = False
    g, c = got.transpose(0, 2, 1, 3, 4), codes.transpose(0, 2, 1, 3, 4)   # (pages, 16, ...)
    np.testing.assert_array_equal(g[untouched], c[untouched])


# ---- logit soft-capping and sm_scale (extensions of the oracle)

@pytest.mark.parametrize("cap,scale", [(None, None), (1.5, None), (50.0, 0.0625), (0.7, 0.2)])
def test_softcap_matches_transformers_gemma2(cap, scale):
    from types import SimpleNamespace
    from transformers.models.gemma2.modeling_gemma2 import eager_attention_forward
    lens = [1, 16, 37]
    q, kv, indptr, ids, last = _paged(lens, 8, 2, 64, 16, seed=12, pool=8, dtype=np.float32)
    q = q * 3                                                  # scores large enough to cap
    got = ref.reference_attention_paged(q, kv, indptr, ids, last, sm_scale=scale,
                                        logit_cap=cap)
    module = SimpleNamespace(head_dim=64, num_key_value_groups=4, training=False)
    for b, n in enumerate(lens):
        k, v = ref._sequence_kv(kv, indptr, ids, last, b)
        qt = torch.from_numpy(q[b].astype(np.float64))[None, :, None, :]      # (1, Hq, 1, D)
        kt = torch.from_numpy(k.astype(np.float64)).permute(1, 0, 2)[None]   # (1, Hkv, S, D)
        vt = torch.from_numpy(v.astype(np.float64)).permute(1, 0, 2)[None]
        want, _ = eager_attention_forward(module, qt, kt, vt, None, scaling=scale,
                                          softcap=cap)
        np.testing.assert_allclose(got[b], want[0, 0].numpy(), rtol=2e-5, atol=2e-6)


def test_planted_softcap_mistake_is_caught_by_transformers():
    # capping the unscaled q.k and scaling afterwards (a plausible slip) must fail the pin
    from types import SimpleNamespace
    from transformers.models.gemma2.modeling_gemma2 import eager_attention_forward
    q, kv, indptr, ids, last = _paged([40], 4, 1, 64, 16, seed=2, dtype=np.float32)
    q = q * 3
    k, v = ref._sequence_kv(kv, indptr, ids, last, 0)
    cap, scale = 1.5, 64 ** -0.5
    raw = q[0].astype(np.float64) @ k[:, 0].T.astype(np.float64)          # (Hq, S)
    s_wrong = scale * cap * np.tanh(raw / cap)
    w = np.exp(s_wrong - s_wrong.max(-1, keepdims=True))
    wrong = (w / w.sum(-1, keepdims=True)) @ v[:, 0].astype(np.float64)
    module = SimpleNamespace(head_dim=64, num_key_value_groups=4, training=False)
    qt = torch.from_numpy(q[0].astype(np.float64))[None, :, None, :]
    kt = torch.from_numpy(k.astype(np.float64)).permute(1, 0, 2)[None]
    vt = torch.from_numpy(v.astype(np.float64)).permute(1, 0, 2)[None]
    want, _ = eager_attention_forward(module, qt, kt, vt, None, scaling=scale, softcap=cap)
    assert np.abs(wrong - want[0, 0].numpy()).max() > 1e-2
    good = ref.reference_attention_paged(q, kv, indptr, ids, last, logit_cap=cap)[0]
    np.testing.assert_allclose(good, want[0, 0].numpy(), rtol=2e-5, atol=2e-6)


# ---- attention sinks (an extension of the oracle)

@pytest.mark.parametrize("sink_scale,window", [(0.0, None), (1.0, None), (4.0, None),
                                               (1.0, 20)])
def test_sinks_match_transformers_gpt_oss(sink_scale, window):
    """The sink form against transformers' gpt-oss eager attention (its softmax over the
    scores and one sink logit per q head, sink column dropped), in float64; window: the
    last `window` tokens, as gpt-oss's sliding layers see them."""
    from types import SimpleNamespace
    from transformers.models.gpt_oss.modeling_gpt_oss import eager_attention_forward
    lens = [1, 16, 37, 60]
    q, kv, indptr, ids, last = _paged(lens, 8, 2, 64, 16, seed=21, pool=12, dtype=np.float32)
    q = q * 2
    rng = np.random.default_rng(5)
    sinks = (rng.standard_normal(8) * sink_scale).astype(np.float32)
    got = ref.reference_attention_paged(q, kv, indptr, ids, last, sinks=sinks, window=window)
    module = SimpleNamespace(num_key_value_groups=4, training=False,
                             sinks=torch.from_numpy(sinks.astype(np.float64)))
    for b, n in enumerate(lens):
        k, v = ref._sequence_kv(kv, indptr, ids, last, b)
        if window:
            k, v = k[-window:], v[-window:]
        qt = torch.from_numpy(q[b].astype(np.float64))[None, :, None, :]      # (1, Hq, 1, D)
        kt = torch.from_numpy(k.astype(np.float64)).permute(1, 0, 2)[None]   # (1, Hkv, S, D)
        vt = torch.from_numpy(v.astype(np.float64)).permute(1, 0, 2)[None]
        want, _ = eager_attention_forward(module, qt, kt, vt, None, scaling=64 ** -0.5)
        np.testing.assert_allclose(got[b], want[0, 0].numpy(), rtol=2e-5, atol=2e-6)


def test_sink_limits_and_planted_mistake():
    """A sink of -inf changes nothing; a very large one drives the output to zero; adding
    the sink to the numerator's weights as well (a plausible slip) fails the gpt-oss pin."""
    from types import SimpleNamespace
    from transformers.models.gpt_oss.modeling_gpt_oss import eager_attention_forward
    q, kv, indptr, ids, last = _paged([40, 7], 4, 1, 64, 16, seed=3, dtype=np.float32)
    plain = ref.reference_attention_paged(q, kv, indptr, ids, last)
    off = ref.reference_attention_paged(q, kv, indptr, ids, last,
                                        sinks=np.full(4, -np.inf, np.float32))
    np.testing.assert_array_equal(off, plain)
    big = ref.reference_attention_paged(q, kv, indptr, ids, last,
                                        sinks=np.full(4, 80.0, np.float32))
    assert np.abs(big).max() < 1e-20
    sinks = np.array([0.5, -1.0, 2.0, 0.0], np.float32)
    k, v = ref._sequence_kv(kv, indptr, ids, last, 0)
    s_ = (q[0].astype(np.float64) * 64 ** -0.5) @ k[:, 0].T.astype(np.float64)   # (Hq, S)
    top = np.maximum(s_.max(-1, keepdims=True), sinks[:, None])
    w = np.exp(s_ - top)
    # the slip: the sink's weight also multiplies a value (here the mean of V)
    den = w.sum(-1, keepdims=True) + np.exp(sinks[:, None] - top)
    wrong = (w @ v[:, 0].astype(np.float64) +
             np.exp(sinks[:, None] - top) * v[:, 0].mean(0)) / den
    module = SimpleNamespace(num_key_value_groups=4, training=False,
                             sinks=torch.from_numpy(sinks.astype(np.float64)))
    qt = torch.from_numpy(q[0].astype(np.float64))[None, :, None, :]
    kt = torch.from_numpy(k.astype(np.float64)).permute(1, 0, 2)[None]
    vt = torch.from_numpy(v.astype(np.float64)).permute(1, 0, 2)[None]
    want, _ = eager_attention_forward(module, qt, kt, vt, None, scaling=64 ** -0.5)
    assert np.abs(wrong - want[0, 0].numpy()).max() > 1e-3
    good = ref.reference_attention_paged(q, kv, indptr, ids, last, sinks=sinks)[0]
    np.testing.assert_allclose(good, want[0, 0].numpy(), rtol=2e-5, atol=2e-6)


# ---- sliding window (an extension of the oracle)

def _repage_last(kv, indptr, ids, last, b, window, P=16):
    """The last `window` tokens of sequence b copied into a fresh pool whose pages start at
    the window's first token (different page boundaries from the source)."""
    k, v = ref._sequence_kv(kv, indptr, ids, last, b)
    k, v = k[-window:], v[-window:]
    n = k.shape[0]
    pages = -(-n // P)
    pool = np.zeros((pages, 2, P) + k.shape[1:], np.float32)
    for t in range(n):
        pool[t // P, 0, t % P], pool[t // P, 1, t % P] = k[t], v[t]
    return pool, np.array([0, pages]), np.arange(pages), np.array([n - (pages - 1) * P])


@pytest.mark.parametrize("window", [1, 5, 16, 17, 100, 5000])
def test_window_equals_attention_over_the_last_tokens(window):
    lens = [1, 16, 17, 300, 1000]
    q, kv, indptr, ids, last = _paged(lens, 8, 2, 64, 16, seed=21, pool=100, dtype=np.float32)
    got = ref.reference_attention_paged(q, kv, indptr, ids, last, window=window)
    for b, n in enumerate(lens):
        pool, ip, ix, ll = _repage_last(kv, indptr, ids, last, b, window)
        want = ref.reference_attention_paged(q[b:b + 1], pool, ip, ix, ll)
        np.testing.assert_allclose(got[b], want[0], rtol=1e-6, atol=1e-6)
    if window >= max(lens):
        np.testing.assert_array_equal(got, ref.reference_attention_paged(q, kv, indptr, ids, last))
    if window == 1:                                  # only the new token: its V exactly
        for b in range(len(lens)):
            _, v = ref._sequence_kv(kv, indptr, ids, last, b)
            np.testing.assert_allclose(got[b].reshape(2, 4, 64), np.repeat(v[-1][:, None], 4, 1),
                                       rtol=1e-6, atol=1e-7)
