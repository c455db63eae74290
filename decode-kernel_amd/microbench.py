"""Decode-attention microbenchmark sweep on MI355X, CSV in the reference's schema.

Counterpart of the reference's bench/microbench_cuda.py: the same sweep (context lengths x
batch sizes x split_kv), the same timing protocol (20 warm-up calls, then 100 timed calls
each preceded by a cache-flushing device fill and bracketed by events; unlike the
reference no host sync follows the fill, so host launch overhead overlaps it and the
events time the GPU work), and the same CSV columns:

    implementation, context_length, batch_size, split_kv, latency_ms_p50, latency_ms_p95,
    achieved_bw_gb_s, peak_bw_gb_s, bw_pct_of_peak, max_abs_err_vs_fp32

Implementations: `hip_naive` (split_kv 1, one pass), `hip_split_kv` (the reference's
ceil(N/S)-page partition + merge, for each split in the sweep) and `hip_auto` (split_kv 0
with the host plan hint: the library's own schedule; reported with split_kv 0).
FlashInfer has no ROCm build here; its rows are skipped as the reference skips them when
flashinfer is missing. Bytes are the reference's model (q + K/V + out,
microbench_cuda.py:114-121). The error column is against an fp32 PyTorch reference of
the same attention computed on the device (gather, scaled scores, softmax, weighted V).

    python decode-kernel_amd/microbench.py                  # full sweep
    python decode-kernel_amd/microbench.py --quick
    python decode-kernel_amd/microbench.py --out results/microbench_hip.csv
"""
from __future__ import annotations

import argparse
import csv
import math
import sys
from pathlib import Path

import numpy as np
import torch

sys.path.insert(0, str(Path(__file__).resolve().parent))

import attention  # noqa: E402
import layout  # noqa: E402
from dk_lib import workspace_bytes  # noqa: E402

NUM_Q_HEADS = 32
NUM_KV_HEADS = 8
HEAD_DIM = 128
PAGE_SIZE = 16
DTYPE = torch.float16
DEVICE = "cuda"
WARMUP_ITERS = 20
TIMED_ITERS = 100
FLUSH_BYTES = 1 << 30            # > the 256 MB Infinity Cache (the reference flushed 256 MB of L2)

COLUMNS = ["implementation", "context_length", "batch_size", "split_kv", "latency_ms_p50",
           "latency_ms_p95", "achieved_bw_gb_s", "peak_bw_gb_s", "bw_pct_of_peak",
           "max_abs_err_vs_fp32"]

FULL_CONTEXT_LENGTHS = [2048, 4096, 8192, 16384, 32768, 65536]
FULL_BATCH_SIZES = [1, 4, 16]
FULL_SPLIT_KVS = [1, 2, 4, 8, 16]
FULL_IMPLS = ["hip_naive", "hip_split_kv", "hip_auto"]
QUICK_CONTEXT_LENGTHS = [2048, 8192]
QUICK_BATCH_SIZES = [1]
QUICK_SPLIT_KVS = [1, 4, 8]
QUICK_IMPLS = ["hip_naive", "hip_split_kv", "hip_auto"]


def peak_bw_gb_s() -> float:
    """Published HBM bandwidth of the device (MI355X 8 TB/s), else from clock x bus width."""
    name = torch.cuda.get_device_properties(0).name.lower()
    known = {"mi355": 8000.0, "mi350": 8000.0, "mi325": 6000.0, "mi300": 5300.0}
    for key, bw in known.items():
        if key in name:
            return bw
    arch = getattr(torch.cuda.get_device_properties(0), "gcnArchName", "")
    if "gfx950" in arch:
        return 8000.0
    p = torch.cuda.get_device_properties(0)
    clock = getattr(p, "memory_clock_rate", 0)
    width = getattr(p, "memory_bus_width", 0)
    return clock * 1e3 * width / 8 * 2 / 1e9 if clock and width else float("nan")


def attention_bytes(batch, ctx, hq, hkv, d, elem_bytes=2) -> int:
    """The reference's bytes model: q + K/V of all tokens + out."""
    return batch * hq * d * elem_bytes * 2 + batch * ctx * hkv * d * elem_bytes * 2


def torch_reference(q, kv, indptr_h, indices, last_h, rows):
    """fp32 attention on the device for the sequences in `rows` (others NaN)."""
    b_, hq, d = q.shape
    hkv = kv.shape[3]
    out = torch.full((b_, hq, d), float("nan"), device=q.device)
    for b in rows:
        s, e = int(indptr_h[b]), int(indptr_h[b + 1])
        n = (e - s - 1) * PAGE_SIZE + int(last_h[b]) if e > s else 0
        if n == 0:
            out[b] = 0
            continue
        blk = kv[indices[s:e].long()].float()                 # (pages, 2, 16, Hkv, D)
        k = blk[:, 0].reshape(-1, hkv, d)[:n].permute(1, 2, 0).contiguous()   # (Hkv, D, n)
        v = blk[:, 1].reshape(-1, hkv, d)[:n].permute(1, 0, 2).contiguous()   # (Hkv, n, D)
        qs = q[b].float().view(hkv, hq // hkv, d) / math.sqrt(d)
        p = torch.softmax(torch.matmul(qs, k), dim=-1)
        out[b] = torch.matmul(p, v).reshape(hq, d)
    return out


def time_kernel(fn, flush, n_warmup=WARMUP_ITERS, n_timed=TIMED_ITERS):
    for _ in range(n_warmup):
        fn()
    torch.cuda.synchronize()
    lat = []
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(n_timed):
        flush.zero_()          # no host sync after it: the call's launch overlaps the fill
        e0.record()
        fn()
        e1.record()
        torch.cuda.synchronize()
        lat.append(e0.elapsed_time(e1))
    return sorted(lat)


def run_sweep(context_lengths, batch_sizes, split_kvs, implementations, out_path,
              check_rows: int = 4, timed_iters: int = TIMED_ITERS):
    if not torch.cuda.is_available():
        raise RuntimeError("a GPU is required for benchmarking")
    peak = peak_bw_gb_s()
    print(f"Peak HBM bandwidth: {peak:.0f} GB/s")
    print(f"GPU: {torch.cuda.get_device_name(0)}\n")
    flush = torch.empty(FLUSH_BYTES, dtype=torch.uint8, device=DEVICE)
    rows = []
    for ctx in context_lengths:
        for batch in batch_sizes:
            print(f"ctx={ctx:>6}  batch={batch:>3}", flush=True)
            q, kv, indptr, ids, last, _ = layout.synthesize_paged(
                batch, ctx, NUM_Q_HEADS, NUM_KV_HEADS, HEAD_DIM, dtype=DTYPE, device=DEVICE,
                page_table="permuted", seed=ctx + batch)
            indptr_h, last_h = indptr.cpu(), last.cpu()
            check = sorted({int(x) for x in np.linspace(0, batch - 1, min(check_rows, batch))})
            ref = torch_reference(q, kv, indptr_h, ids, last_h, check)
            hint = attention.plan_hint(indptr_h)
            total = attention_bytes(batch, ctx, NUM_Q_HEADS, NUM_KV_HEADS, HEAD_DIM)
            for impl in implementations:
                splits = split_kvs if impl == "hip_split_kv" else [1 if impl == "hip_naive" else 0]
                for skv in splits:
                    out = torch.empty_like(q)
                    ws = None
                    need = workspace_bytes(batch, NUM_Q_HEADS, NUM_KV_HEADS, HEAD_DIM, skv)
                    if need:
                        ws = torch.empty(need, dtype=torch.uint8, device=DEVICE)
                    fn = (lambda s=skv: attention.decode_attention(
                        q, kv, indptr, ids, last, split_kv=s, out=out, workspace=ws,
                        max_pages_per_seq=hint))
                    fn()
                    torch.cuda.synchronize()
                    err = float((out[check].float() - ref[check]).abs().max())
                    lat = time_kernel(fn, flush, n_timed=timed_iters)
                    p50, p95 = float(np.percentile(lat, 50)), float(np.percentile(lat, 95))
                    bw = (total / 1e9) / (p50 / 1e3)
                    print(f"  {impl:<14} split={skv:>2}  p50={p50:.4f}ms  bw={bw:.0f}GB/s  "
                          f"max_err={err:.1e}", flush=True)
                    rows.append({
                        "implementation": impl, "context_length": ctx, "batch_size": batch,
                        "split_kv": skv, "latency_ms_p50": round(p50, 4),
                        "latency_ms_p95": round(p95, 4), "achieved_bw_gb_s": round(bw, 2),
                        "peak_bw_gb_s": round(peak, 2),
                        "bw_pct_of_peak": round(100.0 * bw / peak, 2),
                        "max_abs_err_vs_fp32": round(err, 6)})
            print()
            del q, kv
    out_file = Path(out_path)
    out_file.parent.mkdir(parents=True, exist_ok=True)
    with out_file.open("w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=COLUMNS)
        w.writeheader()
        w.writerows(rows)
    print(f"Results written to {out_file}")
    return rows


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description="HIP decode attention microbenchmark")
    ap.add_argument("--out", default="results/microbench_hip.csv", help="output CSV path")
    ap.add_argument("--quick", action="store_true", help="small sweep for quick validation")
    ap.add_argument("--split-kv-only", action="store_true",
                    help="only the explicit split-KV rows")
    ap.add_argument("--timed-iters", type=int, default=TIMED_ITERS)
    return ap.parse_args(argv)


if __name__ == "__main__":
    args = parse_args()
    if args.quick:
        sweep = (QUICK_CONTEXT_LENGTHS, QUICK_BATCH_SIZES, QUICK_SPLIT_KVS, QUICK_IMPLS)
    else:
        sweep = (FULL_CONTEXT_LENGTHS, FULL_BATCH_SIZES, FULL_SPLIT_KVS, FULL_IMPLS)
    impls = ["hip_split_kv"] if args.split_kv_only else sweep[3]
    run_sweep(sweep[0], sweep[1], sweep[2], impls, args.out, timed_iters=args.timed_iters)
