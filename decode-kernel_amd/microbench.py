"""Decode-attention microbenchmark sweeps on MI355X, written as CSV in the reference's schema.

Counterpart of the reference's bench/microbench_cuda.py. Sweeps:

  reference  its own grid: context 2K-64K x batch 1/4/16 x split_kv 1-16, fp16 (config_id 0)
  config2    BASELINE config 2: batch 1/4/16/32/64 x context 4096 x split_kv 1-16, fp16
  config3    BASELINE config 3: batch 1/4 x context 32768/131072 x split_kv 16-128, bf16
  quick      a small validation grid

Timing protocol (the reference's): 20 warm-up calls, then 100 timed calls, each after a
cache-flushing 1 GiB device fill and bracketed by events. Unlike the reference no host
sync follows the fill, so the call's host launch overlaps it and the events time GPU
work. Rows: `hip_naive` (split_kv 1, one pass), `hip_split_kv` (the reference's
ceil(N/S)-page partition + merge, per split of the sweep) and `hip_auto` (split_kv 0 with
the host plan hint: the library's own schedule; reported as split_kv 0). FlashInfer has
no ROCm build here; its rows are left out, as the reference leaves them out without
flashinfer.

Columns: the reference's ten (bench/microbench_cuda.py:270-283; bytes are its model, q +
K/V + out, :114-121; the error is against an fp32 PyTorch attention computed on the
device) and four more: dtype, config_id (0 for the reference grid, else the BASELINE
config), fetch_bytes (bytes the call must read from HBM: K/V of the valid tokens, q and
the page tables; rocprofv3's measured FETCH_SIZE for the metric shape is in profiles/)
and cpu_cores (os.cpu_count() of the host).

    python decode-kernel_amd/microbench.py                        # reference grid
    python decode-kernel_amd/microbench.py --sweep config2 --out results/config2.csv
"""
from __future__ import annotations

import argparse
import csv
import math
import os
import sys
from pathlib import Path

import numpy as np
import torch

sys.path.insert(0, str(Path(__file__).resolve().parent))

import attention  # noqa: E402
import layout  # noqa: E402
from dk_lib import workspace_bytes  # noqa: E402

HQ, HKV, D, PAGE = 32, 8, 128, 16          # the reference's fixed head configuration
DEVICE = "cuda"
WARMUP_ITERS, TIMED_ITERS = 20, 100        # the reference's protocol
FLUSH_BYTES = 1 << 30                      # > the 256 MB Infinity Cache

REFERENCE_COLUMNS = ["implementation", "context_length", "batch_size", "split_kv",
                     "latency_ms_p50", "latency_ms_p95", "achieved_bw_gb_s", "peak_bw_gb_s",
                     "bw_pct_of_peak", "max_abs_err_vs_fp32"]
COLUMNS = REFERENCE_COLUMNS + ["dtype", "config_id", "fetch_bytes", "cpu_cores"]

# name -> (config_id, dtype, context lengths, batch sizes, split_kv values, implementations)
SWEEPS = {
    "reference": (0, torch.float16, [2048, 4096, 8192, 16384, 32768, 65536], [1, 4, 16],
                  [1, 2, 4, 8, 16], ["hip_naive", "hip_split_kv", "hip_auto"]),
    "config2": (2, torch.float16, [4096], [1, 4, 16, 32, 64], [1, 2, 4, 8, 16],
                ["hip_split_kv", "hip_auto"]),
    "config3": (3, torch.bfloat16, [32768, 131072], [1, 4], [16, 32, 64, 128],
                ["hip_split_kv", "hip_auto"]),
    "quick": (0, torch.float16, [2048, 8192], [1], [1, 4, 8],
              ["hip_naive", "hip_split_kv", "hip_auto"]),
}


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
        n = (e - s - 1) * PAGE + int(last_h[b]) if e > s else 0
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
              check_rows: int = 4, timed_iters: int = TIMED_ITERS, dtype=torch.float16,
              config_id: int = 0):
    """Time every (context, batch, implementation, split) point; write and return the rows."""
    if not torch.cuda.is_available():
        raise RuntimeError("the sweep runs on a GPU")
    peak = peak_bw_gb_s()
    dname = {torch.float16: "fp16", torch.bfloat16: "bf16"}[dtype]
    cores = os.cpu_count() or 1
    print(f"# {torch.cuda.get_device_name(0)}: peak {peak:.0f} GB/s, {dname}, "
          f"config_id {config_id}", flush=True)
    flush = torch.empty(FLUSH_BYTES, dtype=torch.uint8, device=DEVICE)
    rows = []
    for ctx in context_lengths:
        for batch in batch_sizes:
            q, kv, indptr, ids, last, _ = layout.synthesize_paged(
                batch, ctx, HQ, HKV, D, dtype=dtype, device=DEVICE, page_table="permuted",
                seed=ctx + batch)
            indptr_h, last_h = indptr.cpu(), last.cpu()
            check = sorted({int(x) for x in np.linspace(0, batch - 1, min(check_rows, batch))})
            ref = torch_reference(q, kv, indptr_h, ids, last_h, check)
            hint = attention.plan_hint(indptr_h)
            total = attention_bytes(batch, ctx, HQ, HKV, D)
            reads = layout.attention_bytes(batch, ctx, HQ, HKV, D) - batch * HQ * D * 2
            for impl in implementations:
                splits = split_kvs if impl == "hip_split_kv" else [1 if impl == "hip_naive" else 0]
                for skv in splits:
                    out = torch.empty_like(q)
                    need = workspace_bytes(batch, HQ, HKV, D, skv)
                    ws = torch.empty(need, dtype=torch.uint8, device=DEVICE) if need else None
                    fn = (lambda s=skv: attention.decode_attention(
                        q, kv, indptr, ids, last, split_kv=s, out=out, workspace=ws,
                        max_pages_per_seq=hint))
                    fn()
                    torch.cuda.synchronize()
                    err = float((out[check].float() - ref[check]).abs().max())
                    lat = time_kernel(fn, flush, n_timed=timed_iters)
                    p50, p95 = float(np.percentile(lat, 50)), float(np.percentile(lat, 95))
                    bw = (total / 1e9) / (p50 / 1e3)
                    print(f"ctx {ctx:6d} B {batch:3d} {impl:12s} split {skv:3d}: "
                          f"{p50 * 1e3:8.1f} us  {bw:7.0f} GB/s ({100 * bw / peak:4.1f} %)  "
                          f"err {err:.1e}", flush=True)
                    rows.append({
                        "implementation": impl, "context_length": ctx, "batch_size": batch,
                        "split_kv": skv, "latency_ms_p50": round(p50, 4),
                        "latency_ms_p95": round(p95, 4), "achieved_bw_gb_s": round(bw, 2),
                        "peak_bw_gb_s": round(peak, 2),
                        "bw_pct_of_peak": round(100.0 * bw / peak, 2),
                        "max_abs_err_vs_fp32": round(err, 6), "dtype": dname,
                        "config_id": config_id, "fetch_bytes": reads, "cpu_cores": cores})
            del q, kv
    out_file = Path(out_path)
    out_file.parent.mkdir(parents=True, exist_ok=True)
    with out_file.open("w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=COLUMNS)
        w.writeheader()
        w.writerows(rows)
    print(f"# {len(rows)} rows -> {out_file}")
    return rows


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description="HIP decode attention microbenchmark")
    ap.add_argument("--sweep", default="reference", choices=sorted(SWEEPS))
    ap.add_argument("--quick", action="store_true", help="same as --sweep quick")
    ap.add_argument("--out", default="results/microbench_hip.csv", help="output CSV path")
    ap.add_argument("--split-kv-only", action="store_true",
                    help="only the explicit split-KV rows")
    ap.add_argument("--timed-iters", type=int, default=TIMED_ITERS)
    return ap.parse_args(argv)


if __name__ == "__main__":
    args = parse_args()
    cid, dt, ctxs, batches, splits, impls = SWEEPS["quick" if args.quick else args.sweep]
    if args.split_kv_only:
        impls = ["hip_split_kv"]
    run_sweep(ctxs, batches, splits, impls, args.out, timed_iters=args.timed_iters, dtype=dt,
              config_id=cid)
