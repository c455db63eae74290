"""Benchmark of the split-KV paged decode-attention path on one MI355X.

Workload (BASELINE.json metric config): batch 32, context 8192 per sequence, 32 q heads,
8 kv heads, head_dim 128, fp16, page_size 16, page table a seeded random permutation of
the 16384-page pool; synthetic N(0,1) data already resident in HBM.

A step is one decode_attention call (pass 1 + pass 2) through the C ABI, with split_kv 0
(automatic schedule) and the plan hint max_pages_per_seq taken once from the host copy of
kv_indptr before the timed region (as a serving framework plans a batch). Before every
step a 1 GiB device fill evicts the 4 MB L2s and the 256 MB Infinity Cache, as the
reference flushes L2 before each timed call (bench/microbench_cuda.py:75-90,140-157);
HIP events on the launch stream bracket the call itself. The flush is enqueued without a
host sync, so host launch overhead is hidden behind it and the events measure GPU time.
The W warm-up steps are such flush + call steps too, after an untimed settling phase of
the same steps (0.3 s) that lets the GPU clocks reach their steady state.

Other shapes (--num-q-heads, --num-kv-heads, --head-dim, --batch, --ctx, --kv-dtype, and
--ragged-min for config 4's ragged mix) are for profiling; the JSON's config names the
workload measured.

Prints one JSON line. `value` is achieved algorithmic HBM bandwidth in TB/s
(bytes of the reference's model, bench/microbench_cuda.py:114-121, plus page tables,
divided by the p50 per-call time); `us_per_call` is the p50 time.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "decode-kernel_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = ("µs/call + achieved HBM TB/s (% peak), decode B=32 ctx=8k Hq32/Hkv8 d128")
PEAK_GBPS = 8000.0          # MI355X HBM3E
FLUSH_BYTES = 1 << 30
SETTLE_S = 0.3              # untimed flush + call steps before the warm-up
TRAFFIC_FILES = {"same": ROOT / "profiles" / "pass1_metric_hbm_traffic.md",
                 "fp8": ROOT / "profiles" / "pass1_metric_fp8_hbm_traffic.md"}


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--split", type=int, default=0, help="split_kv (0 = automatic)")
    ap.add_argument("--schedule", type=int, default=0,
                    help="split_kv 0: 0 automatic, 1 balanced, 2 one pass")
    ap.add_argument("--qk-path", type=int, default=0, help="0 default, 1 MFMA, 2 VALU")
    ap.add_argument("--waves", type=int, default=0, help="wavefronts per workgroup (0 = the library's default)")
    ap.add_argument("--waves-per-cu", type=int, default=0,
                    help="balanced schedule: wavefronts per CU (0 = default)")
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--ctx", type=int, default=8192)
    ap.add_argument("--num-q-heads", type=int, default=32)
    ap.add_argument("--num-kv-heads", type=int, default=8)
    ap.add_argument("--head-dim", type=int, default=128, choices=[64, 128, 256])
    ap.add_argument("--dtype", default="fp16", choices=["fp16", "bf16"])
    ap.add_argument("--kv-dtype", default="same", choices=["same", "fp8"],
                    help="cache element type: q's (the metric's fp16) or fp8 E4M3 (an "
                         "extension; random finite codes, unit scales)")
    ap.add_argument("--flush", default="write", choices=["write", "read"],
                    help="cache flush before each step: fill (write) or sum (read) 1 GiB")
    ap.add_argument("--page-table", default="permuted", choices=["permuted", "contiguous"],
                    help="page-table shape of the synthetic pool (the metric uses permuted)")
    ap.add_argument("--ragged-min", type=int, default=0, metavar="TOKENS",
                    help="ragged mix (config 4 with --batch 128 --ragged-min 128): "
                         "per-sequence lengths uniform in [TOKENS, ctx] (seeded), pages "
                         "drawn from a shuffled free list of 65536 pages, q scaled by "
                         "1/sqrt(head_dim)")
    ap.add_argument("--no-plan-hint", action="store_true",
                    help="do not pass the host-side max_pages_per_seq plan hint")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibration-copy", type=int, default=0, metavar="MIB",
                    help="after the run, copy a MIB-MiB device buffer twice (a kernel of "
                         "known traffic that scales rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--cpu-sample", type=int, default=16,
                    help="sequences of the workload the CPU baseline computes")
    a = ap.parse_args()
    if a.ragged_min and not 1 <= a.ragged_min <= a.ctx:
        ap.error(f"--ragged-min must be in [1, ctx={a.ctx}], got {a.ragged_min}")
    return a


def read_traffic(kv_dtype="same"):
    """HBM bytes per pass-1 launch recorded from rocprofv3 FETCH_SIZE + WRITE_SIZE."""
    path = TRAFFIC_FILES[kv_dtype]
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            try:
                return int(line.split(":", 1)[1].strip())
            except ValueError:
                return None
    return None


def cpu_baseline(q, kv, indptr, ids, last, out, sample):
    """The oracle (a numpy restatement of the reference's CPU path, src/reference.py) timed
    on `sample` sequences of the same workload; also returns its max-abs difference from
    the GPU output on those sequences."""
    import numpy as np
    from threadpoolctl import threadpool_info, threadpool_limits

    import torch

    from oracle.reference import reference_attention_paged

    cores = min(os.cpu_count() or 1, 16)
    as_np = lambda t: (t.float() if t.dtype == torch.bfloat16 else t).cpu().numpy()  # noqa: E731
    qn, kvn = as_np(q), as_np(kv)
    ipn, idn, ln = indptr.cpu().numpy(), ids.cpu().numpy(), last.cpu().numpy()
    subset = list(range(min(sample, q.shape[0])))
    with threadpool_limits(limits=cores):
        blas = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            want = reference_attention_paged(qn, kvn, ipn, idn, ln, batch_subset=subset)
            times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    err = float(np.abs(out[subset].float().cpu().numpy() - want[subset]).max())
    # scaled to the whole batch by pages (the sample's share of the work, also when ragged)
    pages = lambda bs: sum(max(int(ipn[b + 1]) - int(ipn[b]), 0) for b in bs)  # noqa: E731
    per_call_us = t * pages(range(q.shape[0])) / max(pages(subset), 1) * 1e6
    return per_call_us, blas, len(subset), err


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the decode path has no multi-GPU mode here)", file=sys.stderr)
        return 2

    import torch

    import attention
    import dk_lib
    import layout

    lib = dk_lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    dtype = torch.float16 if args.dtype == "fp16" else torch.bfloat16
    B, ctx, hq, hkv, d = args.batch, args.ctx, args.num_q_heads, args.num_kv_heads, args.head_dim
    # the recorded rocprofv3 traffic belongs to the metric's workload only
    metric_workload = ((B, ctx, hq, hkv, d) == (32, 8192, 32, 8, 128)
                       and args.page_table == "permuted" and not args.ragged_min)
    if args.ragged_min:
        lens = layout.ragged_lengths(B, args.ragged_min, ctx, seed=4)
        pool = max(65536, sum((n + 15) // 16 for n in lens))
        q, kv, indptr, ids, last, _ = layout.synthesize_paged(
            B, lens, hq, hkv, d, dtype=dtype, device=dev, page_table="freelist",
            pool_pages=pool, seed=1, q_scale=d ** -0.5)
    else:
        lens = ctx
        q, kv, indptr, ids, last, _ = layout.synthesize_paged(
            B, ctx, hq, hkv, d, dtype=dtype, device=dev, page_table=args.page_table, seed=1)
    kv_ref = kv                        # the cache's values for the CPU baseline
    kv8 = args.kv_dtype == "fp8"
    if kv8:
        # random finite E4M3 codes of moderate magnitude (|value| <= 3.75), unit scales;
        # the CPU baseline attends over the same values stored as fp16 (exact)
        import numpy as np
        g = torch.Generator(device=dev)
        g.manual_seed(1)
        codes = torch.randint(0, 0x48, kv.shape, generator=g, device=dev, dtype=torch.int32)
        codes |= torch.randint(0, 2, kv.shape, generator=g, device=dev,
                               dtype=torch.int32) * 0x80
        codes = codes.to(torch.uint8)
        from oracle import fp8 as fp8_oracle        # the CPU baseline's input only
        table = torch.from_numpy(fp8_oracle.decode(np.arange(256)).astype(np.float32))
        table = torch.nan_to_num(table).to(dev).to(dtype)
        del kv
        kv_ref = table[codes.long()]
        kv = codes.view(attention.KV_FP8)
    split = attention.resolve_split(args.split)
    nbytes = layout.attention_bytes(B, lens, hq, hkv, d, kv_elem_bytes=1 if kv8 else 0)
    out = torch.empty_like(q)
    ws_bytes = dk_lib.workspace_bytes(B, hq, hkv, d, split)
    p_total = dk_lib.partials_layout(B, hq, d, split)[3] if split else ws_bytes
    ws = torch.empty(max(ws_bytes, p_total), dtype=torch.uint8, device=dev)
    flush_buf = torch.ones(FLUSH_BYTES // 4, dtype=torch.float32, device=dev)

    def flush():
        # evict the caches: write (fill) or read (sum) a 1 GiB buffer
        if args.flush == "write":
            flush_buf.zero_()
        else:
            flush_buf.sum()
    strides = attention._strides(q, kv, out)
    # plan step, outside the timed region: the longest sequence's page count from the host
    # side of the page table (what a serving framework keeps on the host)
    hint = 0 if args.no_plan_hint else attention.plan_hint(indptr.cpu())
    opts = dk_lib.options(args.qk_path, args.waves, args.waves_per_cu, args.schedule, hint,
                          kv_dtype=dk_lib.DK_KV_FP8_E4M3 if kv8 else dk_lib.DK_KV_SAME)
    code = attention._DTYPE_CODE[dtype]
    # the schedule the full call runs (split_kv 0 resolves on the device's CU count)
    eff = dk_lib.plan_schedule(B, hq, hkv, d, ids.shape[0], code, split, opts)
    stream = torch.cuda.current_stream(dev)
    common = (q.data_ptr(), kv.data_ptr(), indptr.data_ptr(), ids.data_ptr(), last.data_ptr())
    shape = (B, hq, hkv, d, 16, kv.shape[0], ids.shape[0], code, ctypes.byref(strides))

    def full_call():
        return lib.dk_decode_attention_ex(*common, out.data_ptr(), ws.data_ptr(), ws.numel(),
                                          *shape, split, ctypes.byref(opts), stream.cuda_stream)

    def pass1_only():
        return lib.dk_decode_partials(*common, ws.data_ptr(), ws.numel(), *shape, split,
                                      ctypes.byref(opts), stream.cuda_stream)

    # The dominant kernel: with one pass it is the whole call; otherwise pass 1 alone.
    pass1_call = full_call if eff == 1 else pass1_only

    dk_lib.check(full_call(), "decode_attention")
    dk_lib.check(pass1_call(), "decode_partials")

    def timed(fn, steps):
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(steps)]
        for e0, e1 in evs:
            flush()
            e0.record(stream)
            fn()
            e1.record(stream)
        torch.cuda.synchronize()
        return [e0.elapsed_time(e1) * 1e3 for e0, e1 in evs]     # microseconds

    # Warm-up: W steps exactly like the timed ones (flush + call), after an untimed
    # settling phase of the same steps (at least SETTLE_S seconds) that brings the GPU's
    # clocks to their steady state; without it the first timed steps run slow.
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < SETTLE_S:
        timed(full_call, 20)
    timed(full_call, args.warmup)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    call_us = timed(full_call, args.steps)
    wall = time.perf_counter() - wall0
    pass1_us = timed(pass1_call, args.steps)
    call_us.sort()
    p50 = statistics.median(call_us)
    p95 = call_us[min(len(call_us) - 1, int(math.ceil(0.95 * len(call_us))) - 1)]
    p1_avg = statistics.fmean(pass1_us)
    achieved = nbytes / (p1_avg * 1e-6) / 1e9           # GB/s, pass-1 kernel alone
    # final correctness of the timed output
    dk_lib.check(full_call(), "decode_attention")
    torch.cuda.synchronize()
    finite = bool(torch.isfinite(out).all())
    # q.k path the library takes (its automatic rule: MFMA beyond 4 q heads per kv head
    # and for fp8 at D = 256)
    mfma_qk = args.qk_path == 1 or (args.qk_path == 0 and (hq // hkv > 4 or (kv8 and d >= 256)))
    qk_name = "mfma" if mfma_qk else "valu"

    ctx_label = f"U[{args.ragged_min},{ctx}]" if args.ragged_min else ctx
    table_label = "free-list" if args.ragged_min else args.page_table
    rec = {
        "metric": METRIC, "value": round(nbytes / (p50 * 1e-6) / 1e12, 4), "unit": "TB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(p50 / 1e3, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": args.dtype, "data": "synthetic",
        "config": {"workload": f"paged decode attention B={B} ctx={ctx_label} Hq={hq} "
                               f"Hkv={hkv} D={d} {args.dtype}"
                               f"{' (fp8 E4M3 cache)' if kv8 else ''} "
                               f"page_size=16 {table_label} pages",
                   "kv_dtype": "fp8_e4m3" if kv8 else args.dtype,
                   "batch": B, "context_length": ctx_label, "num_q_heads": hq,
                   "num_kv_heads": hkv,
                   "head_dim": d, "page_size": 16,
                   "split_kv": split,
                   "schedule": {1: "one pass"}.get(eff, "balanced + merge" if eff == 0
                                                   else f"split {eff} + merge"),
                   "plan_hint_max_pages": hint,
                   "qk_path": qk_name, "pv_path": "mfma"},
        "us_per_call": round(p50, 2), "us_per_call_p95": round(p95, 2),
        "pct_of_peak": round(100 * nbytes / (p50 * 1e-6) / (PEAK_GBPS * 1e9), 2),
        "bytes_per_call": nbytes, "wall_s_timed_loop": round(wall, 3),
        "pass1_us_avg": round(p1_avg, 2), "output_finite": finite,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_GBPS, 4),
                     "traffic": read_traffic(args.kv_dtype) if metric_workload else None,
                     "kernel": "dk_pass1_balanced" if eff == 0 else "dk_pass1_split"},
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        us, cores, n, err = cpu_baseline(q, kv_ref, indptr, ids, last, out, args.cpu_sample)
        rec["cpu_baseline"] = {
            "value": round(us, 1), "unit": "us/call", "cores": cores, "kind": "port",
            "tb_s": round(nbytes / (us * 1e-6) / 1e12, 5),
            "sample": f"numpy fp32 restatement of reference_attention_paged on {n} of {B} "
                      f"whole sequences, median of 3, scaled to the whole batch by "
                      f"pages"}
        rec["max_abs_err_vs_fp32"] = err
    print(json.dumps(rec), flush=True)
    if args.calibration_copy > 0:
        src = torch.ones(args.calibration_copy << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(2):
            dst.copy_(src)
        torch.cuda.synchronize()
    return 0


if __name__ == "__main__":
    sys.exit(main())
