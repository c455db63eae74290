"""The reference's CPU oracle path restated in torch, literally: the form bench.py times
as the CPU baseline at the metric configuration.

TEST INFRASTRUCTURE ONLY. Imported by tests/ and by bench.py's CPU-baseline leg (as the
timed CPU path and the checker of the GPU output); never by the product code under
decode-kernel_amd/.

It follows /root/reference src/reference.py step for step, because its cost is what is
being measured:
  * gather_dense           src/reference.py:9-58: the whole page pool converted to fp32
                           on the host, then one slice copy per page (a Python loop over
                           the page table), zero padding past each sequence up to the
                           longest one
  * attend_dense           src/reference.py:61-96: GQA by repeat_interleave of the kv
                           heads, q scaled by 1/sqrt(D), scores by batched matmul, softmax
                           over every (padded) position, weighted sum by batched matmul
  * reference_attention_paged_literal   src/reference.py:99-108: the two in sequence
The padded softmax equals the per-sequence masked one whenever all sequences have the
same length (every configuration it is timed on); tests/test_oracle.py pins both
functions against the numpy restatement in oracle/reference.py (literal form).
"""
from __future__ import annotations

import torch


def gather_dense(kv_data, kv_indptr, kv_indices, kv_last_page_len):
    """Dense fp32 K, V (B, max_len, Hkv, D) on the host, zero past each sequence."""
    pool = kv_data.detach().to("cpu", torch.float32)     # (N_p, 2, P, Hkv, D)
    page = pool.shape[2]
    ptr = [int(x) for x in kv_indptr.cpu().tolist()]
    ids = [int(x) for x in kv_indices.cpu().tolist()]
    tail = [int(x) for x in kv_last_page_len.cpu().tolist()]
    batch = len(ptr) - 1
    lens = [max(0, (ptr[b + 1] - ptr[b] - 1) * page + tail[b]) for b in range(batch)]
    width = max(lens, default=0)
    K = torch.zeros((batch, width) + tuple(pool.shape[3:]), dtype=torch.float32)
    V = torch.zeros_like(K)
    for b in range(batch):
        at = 0
        for j in range(ptr[b], ptr[b + 1]):
            n = tail[b] if j == ptr[b + 1] - 1 else page
            K[b, at:at + n] = pool[ids[j], 0, :n]
            V[b, at:at + n] = pool[ids[j], 1, :n]
            at += n
    return K, V


def attend_dense(Q, K, V):
    """fp32 softmax(q k^T / sqrt(D)) v over all positions of K, V (B, S, Hkv, D); Q is
    (B, Hq, D) on the host. Returns (B, Hq, D) fp32."""
    q = Q.detach().to("cpu", torch.float32)
    group = q.shape[1] // K.shape[2]
    k = K.repeat_interleave(group, dim=2).permute(0, 2, 3, 1)    # (B, Hq, D, S)
    v = V.repeat_interleave(group, dim=2).permute(0, 2, 1, 3)    # (B, Hq, S, D)
    s = torch.matmul(q.unsqueeze(2) * q.shape[-1] ** -0.5, k)   # (B, Hq, 1, S)
    return torch.matmul(torch.softmax(s, dim=-1), v).squeeze(2)


def reference_attention_paged_literal(Q, kv_data, kv_indptr, kv_indices, kv_last_page_len):
    """gather_dense then attend_dense: the reference's reference_attention_paged."""
    K, V = gather_dense(kv_data, kv_indptr, kv_indices, kv_last_page_len)
    return attend_dense(Q, K, V)
