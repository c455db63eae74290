"""CPU oracle for the paged decode-attention path.

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as the checker,
and by bench.py's CPU-baseline leg. The product (decode-kernel_amd/) never imports it and
has no CPU fallback.

  reference.py  restatement of the reference's fp32 oracle (src/reference.py)
  split_kv.py   restatement of the two-pass split-KV algorithm (src/cuda_/attention_ext.cu)
"""
