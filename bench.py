"""Benchmark of the split-KV paged decode-attention path on one MI355X.

Default workload (BASELINE.json's metric config): batch 32, context 8192 per sequence,
32 q heads, 8 kv heads, head_dim 128, fp16, page_size 16, page table a seeded random
permutation of the 16384-page pool; synthetic N(0,1) data already resident in HBM.

A step is one decode_attention call (pass 1 + pass 2 when the schedule has one) through
the C ABI, with split_kv 0 (automatic schedule) and the plan hint max_pages_per_seq taken
once from the host copy of kv_indptr before the timed region (as a serving framework
plans a batch). Before every step a 1 GiB device fill evicts the 4 MB L2s and the 256 MB
Infinity Cache, as the reference flushes L2 before each timed call
(bench/microbench_cuda.py:75-90,140-157); HIP events on the launch stream bracket the call
itself. The flush is enqueued without a host sync, so host launch overhead is hidden
behind it and the events measure GPU time. The events are created with
hipEventDisableSystemFence (no system-scope cache writeback when one is recorded: ~1.8 us
less per call than default events, whose p50 the metric line also reports). The W warm-up steps are such flush + call
steps too, after an untimed settling phase of the same steps (at least 0.3 s, then until
three sets of 20 agree within 2 %, at most 2 s) that lets the GPU clocks reach their
steady state. Between workloads the run hands the previous one's device memory back to
the driver and waits for the driver's background clearing of it, which otherwise slows
the next workload's first ~0.1-0.5 s of steps by ~6.5 %.

Modes:
  (default)        one JSON line for the metric workload (or the shape given by --batch,
                   --ctx, --num-q-heads, --num-kv-heads, --head-dim, --dtype, --kv-dtype,
                   --ragged-min, --split ...), with `roofline` and `cpu_baseline`; on
                   the metric workload it also carries `baseline_configs`: the headline
                   point of every BASELINE config (its stated split, else the automatic
                   schedule) and the fp8 cache at the metric shape, timed the same way in
                   the same run after the metric and checked against the CPU oracle on
                   sampled sequences (--no-extra-configs leaves them out)
  --config N       BASELINE.json config N (1-5) on its own workloads: one JSON line per
                   (shape, split_kv) of the config's sweep, each with p50/p95 us, TB/s,
                   the fraction of 8 TB/s and the max-abs error against the CPU oracle on
                   sampled sequences
  --single-call    one flush and one call, no settling or warm-up (for rocprofv3 --pmc
                   counter runs, which then see exactly the call's dispatches); with
                   --no-check the call is the run's only decode dispatch (no checking call
                   before it, no correctness call after it)
  --graph          the latency-bound configs as a model runs them: N back-to-back calls on
                   N distinct caches (N x bytes >= 1 GiB, so no flush is needed between
                   calls; config 5's 16-layer step as stated), eager and captured in one
                   HIP graph and replayed, reported per call beside the flush + events
                   protocol's figure of the same shape (one JSON line per point)
  --host-overhead  host time per call of the Python entry points (back to back, no
                   flush): attention.decode_attention, DecodePlan.run with a preallocated
                   output, the bare C-ABI call, and a call that validates its arguments
                   afresh (no cached plan)

With the environment variable DK_TRACE set, every timed step is a roctx range ("step i")
holding a "flush" and a "call" range (rocprofv3 --marker-trace), around the library's own
ranges of each launch.

`value` is achieved algorithmic HBM bandwidth in TB/s (bytes of the reference's model,
bench/microbench_cuda.py:114-121, plus page tables, divided by the p50 per-call time);
`us_per_call` is the p50 time.

CPU baseline (default mode): the reference's CPU path (src/reference.py: the whole pool
to fp32, a per-page gather into zero-padded dense K/V, GQA by repeat_interleave, fp32
softmax attention) restated in torch (oracle/reference_torch.py), timed on the box's host
cores over the whole batch, gather and attention separately, median of 3. For a ragged
mix, where that padded form is wrong, the numpy per-sequence oracle (oracle/reference.py)
is timed on a sample of sequences instead. In every mode the baseline's outputs are also
the checker of the GPU output (max_abs_err_vs_fp32).
"""
from __future__ import annotations

import argparse
import ctypes
import hashlib
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
CONFIG_METRIC = "µs/call + achieved HBM TB/s (% peak), BASELINE config {n}"
PEAK_GBPS = 8000.0          # MI355X HBM3E
FLUSH_BYTES = 1 << 30
SETTLE_S = 0.3              # untimed flush + call steps before the warm-up, at least
SETTLE_MAX_S = 2.0          # ... and at most, while consecutive sets still disagree
SETTLE_AGREE = 1.02         # settled: the last 3 sets' p50s within 2 % of each other
# Device memory handed back to the driver (torch.cuda.empty_cache) is cleared by it in the
# background, and meanwhile HBM-bound kernels run ~6.5 % slower (metric shape 168 vs
# 157.7 us; 2 GiB released -> ~0.08 s of slow steps, 8 GiB -> ~0.25 s, 16 GiB -> ~0.5 s,
# i.e. ~32 GiB/s). After a release the run waits for that at half the rate.
RELEASE_WAIT_GIB_S = 16.0
# Host threads of the CPU baseline: the GPU box gives each GPU a 16-thread CPU share
# (whatever os.cpu_count() reports there), so at most that many.
CPU_THREADS_CAP = 16
TRAFFIC_FILES = {"same": ROOT / "profiles" / "pass1_metric_hbm_traffic.md",
                 "fp8": ROOT / "profiles" / "pass1_metric_fp8_hbm_traffic.md"}

# BASELINE.json configs as concrete workloads: (label, shape) with the split_kv values of
# the config's sweep (0 = the library's automatic schedule with the plan hint).
CONFIGS = {
    1: [dict(batch=2, ctx=512, dtype="fp16", table="contiguous", splits=(4, 0))],
    2: [dict(batch=b, ctx=4096, dtype="fp16", table="permuted", splits=(1, 2, 4, 8, 16, 0))
        for b in (1, 4, 16, 32, 64)],
    3: [dict(batch=b, ctx=c, dtype="bf16", table="permuted", splits=(16, 32, 64, 128, 0))
        for b in (1, 4) for c in (32768, 131072)],
    4: [dict(batch=128, ctx=8192, ragged_min=128, dtype="fp16", table="freelist",
             q_scale=128 ** -0.5, splits=(0, 1, 4, 16))],
    5: [dict(batch=32, ctx=2048, d=64, dtype="bf16", table="permuted", splits=(0,))],
}


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=0, choices=[0, 1, 2, 3, 4, 5],
                    help="run BASELINE.json config N's sweep (one JSON line per point)")
    ap.add_argument("--single-call", action="store_true",
                    help="one flush + one call, no settling / warm-up (counter runs)")
    ap.add_argument("--no-check", action="store_true",
                    help="--single-call: no checking call before the timed call and no "
                         "correctness call after it (the run's only decode dispatch)")
    ap.add_argument("--graph", action="store_true",
                    help="latency-bound configs as N back-to-back calls on N caches, eager "
                         "and under HIP-graph replay (see the modes)")
    ap.add_argument("--graph-point", default="",
                    help="--graph: only the point of this label (e.g. 'C2 B=1')")
    ap.add_argument("--host-overhead", action="store_true",
                    help="host us per call of attention.decode_attention (see the modes)")
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
    ap.add_argument("--sinks", action="store_true",
                    help="attention sinks (an extension, gpt-oss): one seeded N(0, 4) logit "
                         "per q head; the output is checked against the oracle's sink form "
                         "and no CPU baseline is timed")
    ap.add_argument("--page-size", type=int, default=16, metavar="TOKENS",
                    help="pages of TOKENS tokens (a multiple of 16; an extension): times "
                         "decode_attention, which reads them as 16-token sub-pages after "
                         "rewriting the page table on the device, checked against the "
                         "oracle on the original layout; no CPU baseline")
    ap.add_argument("--window", type=int, default=0, metavar="TOKENS",
                    help="sliding window (an extension): attend to each sequence's last "
                         "TOKENS tokens; bytes count the pages read; checked like --sinks")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra-configs", action="store_true",
                    help="default run: leave out the BASELINE configs' headline points")
    ap.add_argument("--calibration-copy", type=int, default=0, metavar="MIB",
                    help="after the run, copy a MIB-MiB device buffer twice (a kernel of "
                         "known traffic that scales rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--cpu-sample", type=int, default=0,
                    help="sequences the CPU baseline computes (0 = the whole batch for "
                         "uniform lengths, 8 for a ragged mix)")
    a = ap.parse_args(argv)
    if a.ragged_min and not 1 <= a.ragged_min <= a.ctx:
        ap.error(f"--ragged-min must be in [1, ctx={a.ctx}], got {a.ragged_min}")
    if a.single_call and a.config:
        ap.error("--single-call times the default workload; it does not combine with --config")
    if a.no_check and not a.single_call:
        ap.error("--no-check applies to --single-call")
    if a.graph and (a.config or a.single_call or a.host_overhead or a.page_size != 16):
        ap.error("--graph runs its own points; it does not combine with --config, "
                 "--single-call, --host-overhead or --page-size")
    if a.window < 0:
        ap.error(f"--window must be >= 0, got {a.window}")
    if (a.sinks or a.window) and a.config:
        ap.error("--sinks and --window apply to the default workload, not to --config sweeps")
    if a.page_size <= 0 or a.page_size % 16:
        ap.error(f"--page-size must be a positive multiple of 16, got {a.page_size}")
    if a.page_size != 16 and (a.config or a.single_call or a.host_overhead or a.ragged_min or
                              a.sinks or a.window or a.kv_dtype != "same"):
        ap.error("--page-size times the default uniform workload alone")
    return a


# Sources whose digest stamps a traffic measurement: every file the library is built from.
KERNEL_SOURCES = ROOT / "decode-kernel_amd" / "csrc"


def kernel_source_digest():
    """sha256 (16 hex digits) over the library's sources (decode-kernel_amd/csrc/*.h, *.hip,
    *.cpp, by name and content): a traffic figure measured on another digest does not
    describe the kernel this tree builds."""
    h = hashlib.sha256()
    for f in sorted(KERNEL_SOURCES.iterdir()):
        if f.suffix in (".h", ".hip", ".cpp"):
            h.update(f.name.encode() + b"\0" + f.read_bytes() + b"\0")
    return h.hexdigest()[:16]


def read_traffic(kv_dtype="same"):
    """(HBM bytes per pass-1 launch from rocprofv3 FETCH_SIZE + WRITE_SIZE, or None when the
    profile was measured on other kernel sources; the profile's stamp). The profile file
    holds `traffic_bytes_per_launch:`, `kernel_source_digest:` and `measured_at_commit:`
    lines."""
    path = TRAFFIC_FILES[kv_dtype]
    if not path.exists():
        return None, None
    fields = {}
    for line in path.read_text().splitlines():
        key, sep, val = line.partition(":")
        if sep and key in ("traffic_bytes_per_launch", "kernel_source_digest",
                           "measured_at_commit"):
            fields[key] = val.strip()
    try:
        traffic = int(fields["traffic_bytes_per_launch"])
    except (KeyError, ValueError):
        return None, None
    current = kernel_source_digest()
    stamp = {"file": str(path.relative_to(ROOT)), "commit": fields.get("measured_at_commit"),
             "kernel_source_digest": fields.get("kernel_source_digest"),
             "current_digest": current,
             "matches_build": fields.get("kernel_source_digest") == current}
    return (traffic if stamp["matches_build"] else None), stamp


def host_cpu():
    """(os.cpu_count(), threads the baseline uses, CPU model name)."""
    n = os.cpu_count() or 1
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return n, min(n, CPU_THREADS_CAP), model


def percentile(sorted_us, pct):
    return sorted_us[min(len(sorted_us) - 1, int(math.ceil(pct / 100 * len(sorted_us))) - 1)]


# ---------------------------------------------------------------- workloads

class Workload:
    """Synthetic decode inputs of one shape on the GPU, with the tables on the host."""

    def __init__(self, torch, layout, dev, batch, ctx, hq=32, hkv=8, d=128, dtype="fp16",
                 table="permuted", ragged_min=0, q_scale=1.0, kv_dtype="same", seed=1):
        self.torch = torch
        self.dtype_name = dtype
        self.dtype = torch.float16 if dtype == "fp16" else torch.bfloat16
        self.batch, self.ctx, self.hq, self.hkv, self.d = batch, ctx, hq, hkv, d
        self.ragged_min = ragged_min
        if ragged_min:
            self.lens = layout.ragged_lengths(batch, ragged_min, ctx, seed=4)
            pool = max(65536, sum((n + 15) // 16 for n in self.lens))
            q, kv, indptr, ids, last, _ = layout.synthesize_paged(
                batch, self.lens, hq, hkv, d, dtype=self.dtype, device=dev,
                page_table="freelist", pool_pages=pool, seed=seed, q_scale=q_scale)
            self.table = "free-list"
        else:
            self.lens = [ctx] * batch
            q, kv, indptr, ids, last, _ = layout.synthesize_paged(
                batch, ctx, hq, hkv, d, dtype=self.dtype, device=dev, page_table=table,
                seed=seed, q_scale=q_scale)
            self.table = table
        self.kv_ref = kv                      # the cache's values as q's dtype (CPU checks)
        self.kv8 = kv_dtype == "fp8"
        if self.kv8:
            kv = self._to_fp8(dev, kv)
        self.q, self.kv, self.indptr, self.ids, self.last = q, kv, indptr, ids, last
        self.indptr_host = indptr.cpu()
        self.bytes = layout.attention_bytes(batch, self.lens, hq, hkv, d,
                                            kv_elem_bytes=1 if self.kv8 else 0)

    def _to_fp8(self, dev, kv):
        # random finite E4M3 codes of moderate magnitude (|value| <= 3.75), unit scales;
        # the CPU checks attend over the same values stored as q's dtype (exact)
        import numpy as np
        torch = self.torch
        g = torch.Generator(device=dev)
        g.manual_seed(1)
        codes = torch.randint(0, 0x48, kv.shape, generator=g, device=dev, dtype=torch.int32)
        codes |= torch.randint(0, 2, kv.shape, generator=g, device=dev,
                               dtype=torch.int32) * 0x80
        codes = codes.to(torch.uint8)
        from oracle import fp8 as fp8_oracle        # the CPU checks' input only
        table = torch.from_numpy(fp8_oracle.decode(np.arange(256)).astype(np.float32))
        table = torch.nan_to_num(table).to(dev).to(self.dtype)
        self.kv_ref = table[codes.long()]
        return codes.view(torch.float8_e4m3fn)

    def label(self):
        ctx = f"U[{self.ragged_min},{self.ctx}]" if self.ragged_min else self.ctx
        return (f"paged decode attention B={self.batch} ctx={ctx} Hq={self.hq} Hkv={self.hkv} "
                f"D={self.d} {self.dtype_name}{' (fp8 E4M3 cache)' if self.kv8 else ''} "
                f"page_size=16 {self.table} pages")


class Caller:
    """One (workload, split_kv, options) through the C ABI, with its own output and
    workspace, and the timing protocol."""

    def __init__(self, lib, dk_lib, attention, wl, split, opts, stream):
        torch = wl.torch
        self.lib, self.dk_lib, self.wl, self.split, self.opts, self.stream = \
            lib, dk_lib, wl, split, opts, stream
        self.out = torch.empty_like(wl.q)
        ws_bytes = dk_lib.workspace_bytes(wl.batch, wl.hq, wl.hkv, wl.d, split)
        p_total = dk_lib.partials_layout(wl.batch, wl.hq, wl.d, split)[3] if split else ws_bytes
        self.ws = torch.empty(max(ws_bytes, p_total, 1), dtype=torch.uint8, device=wl.q.device)
        self.strides = attention._strides(wl.q, wl.kv, self.out)
        self.code = attention._DTYPE_CODE[wl.dtype]
        self.common = (wl.q.data_ptr(), wl.kv.data_ptr(), wl.indptr.data_ptr(),
                       wl.ids.data_ptr(), wl.last.data_ptr())
        self.shape = (wl.batch, wl.hq, wl.hkv, wl.d, 16, wl.kv.shape[0], wl.ids.shape[0],
                      self.code, ctypes.byref(self.strides))
        # the schedule the full call runs (split_kv 0 resolves on the device's CU count)
        self.schedule = dk_lib.plan_schedule(wl.batch, wl.hq, wl.hkv, wl.d, wl.ids.shape[0],
                                             self.code, split, opts)

    def full(self):
        return self.lib.dk_decode_attention_ex(*self.common, self.out.data_ptr(),
                                               self.ws.data_ptr(), self.ws.numel(), *self.shape,
                                               self.split, ctypes.byref(self.opts),
                                               self.stream.cuda_stream)

    def pass1(self):
        # split_kv 0 resolved to an explicit split: that split's pass 1 (the pass-1-only
        # entry point would take the balanced schedule)
        split = self.schedule if self.split == 0 and self.schedule > 1 else self.split
        return self.lib.dk_decode_partials(*self.common, self.ws.data_ptr(), self.ws.numel(),
                                           *self.shape, split, ctypes.byref(self.opts),
                                           self.stream.cuda_stream)

    def dominant(self):
        """The dominant kernel alone: the whole call in one pass, else pass 1."""
        return self.full if self.schedule == 1 else self.pass1

    def schedule_name(self):
        return {1: "one pass"}.get(self.schedule, "balanced + merge" if self.schedule == 0
                                    else f"split {self.schedule} + merge")


def roctx_ranges():
    """(push, pop) of the roctx library when DK_TRACE is set (to anything but "" or "0"),
    else None: the same library and switch as libdk_decode's launch ranges."""
    if os.environ.get("DK_TRACE", "") in ("", "0"):
        return None
    for name in ("librocprofiler-sdk-roctx.so.1", "libroctx64.so.4"):
        try:
            lib = ctypes.CDLL(name)
        except OSError:
            continue
        push, pop = lib.roctxRangePushA, lib.roctxRangePop
        push.argtypes, push.restype, pop.restype = [ctypes.c_char_p], ctypes.c_int, ctypes.c_int
        return push, pop
    return None


# The timed regions' events are HIP events created with hipEventDisableSystemFence: recording
# one writes its timestamp in stream order without the system-scope cache writeback and
# invalidation that a default event (torch.cuda.Event) performs, which hip_runtime_api.h
# recommends for timing on AMD GPUs. Stream order -- what lies between the two timestamps --
# is the same. Measured on one MI355X: a pair around an empty stream 3.9 us against 5.0 us
# for default events, and every decode call ~1.8 us less (metric shape 155.7 vs 157.5 us;
# the rocprofv3 average of the kernel is 155.5 us).
HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000


class HipEvents:
    """Timing events of the HIP runtime the process already loaded (through torch)."""

    def __init__(self, flags=HIP_EVENT_DISABLE_SYSTEM_FENCE):
        self.flags = flags
        lib = ctypes.CDLL(self._loaded_runtime())
        vp = ctypes.c_void_p
        lib.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(vp), ctypes.c_uint]
        lib.hipEventRecord.argtypes = [vp, vp]
        lib.hipEventSynchronize.argtypes = [vp]
        lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        lib.hipEventDestroy.argtypes = [vp]
        self.lib = lib

    @staticmethod
    def _loaded_runtime():
        # the library torch loaded: a second copy of the runtime would not know its streams
        try:
            with open("/proc/self/maps") as f:
                for line in f:
                    if "libamdhip64.so" in line:
                        return line.split()[-1]
        except OSError:
            pass
        return "libamdhip64.so"

    def _ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed: hipError {rc}")

    def pairs(self, n):
        out = []
        for _ in range(n):
            a, b = ctypes.c_void_p(), ctypes.c_void_p()
            self._ok(self.lib.hipEventCreateWithFlags(ctypes.byref(a), self.flags), "hipEventCreate")
            self._ok(self.lib.hipEventCreateWithFlags(ctypes.byref(b), self.flags), "hipEventCreate")
            out.append((a, b))
        return out

    def record(self, ev, stream):
        self._ok(self.lib.hipEventRecord(ev, ctypes.c_void_p(stream.cuda_stream)), "hipEventRecord")

    def elapsed_us(self, pairs):
        """Microseconds between each pair's events; destroys them."""
        out = []
        for a, b in pairs:
            self._ok(self.lib.hipEventSynchronize(b), "hipEventSynchronize")
            ms = ctypes.c_float()
            self._ok(self.lib.hipEventElapsedTime(ctypes.byref(ms), a, b), "hipEventElapsedTime")
            out.append(ms.value * 1e3)
            self.lib.hipEventDestroy(a)
            self.lib.hipEventDestroy(b)
        return out


class TorchEvents:
    """Default-flag events (torch.cuda.Event), the timing of earlier bench lines."""

    def __init__(self, torch):
        self.torch = torch

    def pairs(self, n):
        ev = self.torch.cuda.Event
        return [(ev(enable_timing=True), ev(enable_timing=True)) for _ in range(n)]

    def record(self, ev, stream):
        ev.record(stream)

    def elapsed_us(self, pairs):
        self.torch.cuda.synchronize()
        return [a.elapsed_time(b) * 1e3 for a, b in pairs]


class Timer:
    """Flush + events around each call, on the launch stream (each step a roctx range
    under DK_TRACE). events: "nofence" (HipEvents, the default) or "default" (TorchEvents)."""

    def __init__(self, torch, dev, stream, mode="write", events="nofence"):
        self.torch, self.stream, self.mode = torch, stream, mode
        self.buf = torch.ones(FLUSH_BYTES // 4, dtype=torch.float32, device=dev)
        self.ranges = roctx_ranges()
        self.nstep = 0
        self.events = HipEvents() if events == "nofence" else TorchEvents(torch)

    def flush(self):
        # evict the caches: write (fill) or read (sum) a 1 GiB buffer
        if self.mode == "write":
            self.buf.zero_()
        else:
            self.buf.sum()

    def run(self, fn, steps, events=None):
        ev = events or self.events
        evs = ev.pairs(steps)
        rg = self.ranges
        for e0, e1 in evs:
            if rg:
                rg[0](f"step {self.nstep}".encode())
                rg[0](b"flush")
            self.flush()
            if rg:
                rg[1]()
                rg[0](b"call")
            ev.record(e0, self.stream)
            fn()
            ev.record(e1, self.stream)
            if rg:
                rg[1]()
                rg[1]()
            self.nstep += 1
        self.torch.cuda.synchronize()
        return ev.elapsed_us(evs)     # microseconds

    def settle(self, fn):
        # untimed flush + call steps until the GPU clocks reach their steady state (without
        # it the first timed steps run slow): at least SETTLE_S, then until the last three
        # sets of 20 agree, at most SETTLE_MAX_S
        t0 = time.perf_counter()
        p50s = []
        while True:
            p50s.append(statistics.median(self.run(fn, 20)))
            t = time.perf_counter() - t0
            last = p50s[-3:]
            if t >= SETTLE_MAX_S or (t >= SETTLE_S and len(last) == 3
                                     and max(last) <= SETTLE_AGREE * min(last)):
                return


def release_device_memory(torch):
    """torch.cuda.empty_cache(), then a wait for the driver's background clearing of the
    released memory (it slows HBM-bound kernels while it runs)."""
    before = torch.cuda.memory_reserved()
    torch.cuda.empty_cache()
    released = max(before - torch.cuda.memory_reserved(), 0)
    time.sleep(released / (RELEASE_WAIT_GIB_S * 2**30))


# ---------------------------------------------------------------- CPU baseline leg

def _host_subproblem(wl, seqs):
    """q, kv pages and rebased page tables of sequences `seqs` on the host (the pages of
    those sequences only, so the CPU side never holds the whole pool)."""
    torch = wl.torch
    ip = wl.indptr_host.tolist()
    ids = wl.ids.cpu()
    pages = [ids[ip[b]:ip[b + 1]] for b in seqs]
    flat = torch.cat(pages) if pages else torch.zeros(0, dtype=torch.int32)
    kv = wl.kv_ref[flat.to(wl.kv_ref.device).long()].cpu()
    indptr = torch.zeros(len(seqs) + 1, dtype=torch.int32)
    indptr[1:] = torch.cumsum(torch.tensor([len(p) for p in pages], dtype=torch.int64), 0).to(torch.int32)
    return (wl.q[list(seqs)].cpu(), kv, indptr, torch.arange(len(flat), dtype=torch.int32),
            wl.last.cpu()[list(seqs)])


def cpu_baseline_literal(wl, seqs, threads, reps=3):
    """The reference's CPU path (oracle/reference_torch.py) on sequences `seqs`: median
    gather / attention / total seconds of `reps` runs, and the output (len(seqs), Hq, D)."""
    torch = wl.torch
    from oracle import reference_torch as rt
    q, kv, indptr, ids, last = _host_subproblem(wl, seqs)
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        g, a, out = [], [], None
        for _ in range(reps):
            t0 = time.perf_counter()
            K, V = rt.gather_dense(kv, indptr, ids, last)
            t1 = time.perf_counter()
            out = rt.attend_dense(q, K, V)
            t2 = time.perf_counter()
            del K, V
            g.append(t1 - t0)
            a.append(t2 - t1)
    finally:
        torch.set_num_threads(prev)
    tot = [x + y for x, y in zip(g, a)]
    return statistics.median(g), statistics.median(a), statistics.median(tot), out


def cpu_baseline_masked(wl, seqs, threads, reps=3):
    """The numpy per-sequence oracle (oracle/reference.py; masked, right for ragged mixes)
    on sequences `seqs`: median seconds of `reps` runs (gather and attention are not
    separable there: each sequence gathers its own pages), and the output."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle.reference import reference_attention_paged
    torch = wl.torch
    q, kv, indptr, ids, last = _host_subproblem(wl, seqs)
    as_np = lambda t: (t.float() if t.dtype == torch.bfloat16 else t).numpy()  # noqa: E731
    qn, kvn = as_np(q), as_np(kv)
    ipn, idn, ln = indptr.numpy(), ids.numpy(), last.numpy()
    times, out = [], None
    with threadpool_limits(limits=threads):
        for _ in range(reps):
            t0 = time.perf_counter()
            out = reference_attention_paged(qn, kvn, ipn, idn, ln)
            times.append(time.perf_counter() - t0)
    return statistics.median(times), torch.from_numpy(np.asarray(out))


def max_abs_err(got, want_rows, seqs):
    """max |got[seqs] - want| (want (len(seqs), Hq, D), fp32 on the host)."""
    g = got[list(seqs)].float().cpu()
    return float((g - want_rows.float()).abs().max()) if g.numel() else 0.0


# ---------------------------------------------------------------- modes

def make_opts(dk_lib, args, wl, split):
    hint = 0 if args.no_plan_hint else _plan_hint(wl)
    sinks = getattr(wl, "sinks", None)
    return dk_lib.options(args.qk_path, args.waves, args.waves_per_cu, args.schedule, hint,
                          kv_dtype=dk_lib.DK_KV_FP8_E4M3 if wl.kv8 else dk_lib.DK_KV_SAME,
                          window=getattr(args, "window", 0) or 0,
                          sinks=0 if sinks is None else sinks.data_ptr()), hint


def _plan_hint(wl):
    import attention
    return attention.plan_hint(wl.indptr_host)


def metric_run(args, torch, lib, dk_lib, attention, layout, dev, stream):
    wl = Workload(torch, layout, dev, args.batch, args.ctx, args.num_q_heads,
                  args.num_kv_heads, args.head_dim, args.dtype,
                  "freelist" if args.ragged_min else args.page_table, args.ragged_min,
                  q_scale=args.head_dim ** -0.5 if args.ragged_min else 1.0,
                  kv_dtype=args.kv_dtype)
    extension = bool(args.sinks or args.window)
    if args.sinks:
        g = torch.Generator(device="cpu")
        g.manual_seed(3)
        wl.sinks = (torch.randn(wl.hq, generator=g) * 2).to(dev)
    if args.window:
        # the pages a windowed call reads: those holding each sequence's last `window` tokens
        w = args.window
        first = [max(n - w, 0) // 16 * 16 for n in wl.lens]
        wl.bytes = layout.attention_bytes(wl.batch, [n - f for n, f in zip(wl.lens, first)],
                                          wl.hq, wl.hkv, wl.d,
                                          kv_elem_bytes=1 if wl.kv8 else 0)
    split = attention.resolve_split(args.split)
    opts, hint = make_opts(dk_lib, args, wl, split)
    c = Caller(lib, dk_lib, attention, wl, split, opts, stream)
    timer = Timer(torch, dev, stream, args.flush)
    if not args.no_check:
        dk_lib.check(c.full(), "decode_attention")
    default_us = None
    if args.single_call:
        steps, warmup = 1, 0
        torch.cuda.synchronize()
        call_us = timer.run(lambda: dk_lib.check(c.full(), "decode_attention"), 1)
        pass1_us = call_us if c.schedule == 1 else None
        wall = 0.0
    else:
        steps, warmup = args.steps, args.warmup
        dk_lib.check(c.dominant()(), "decode_partials")
        timer.settle(c.full)
        timer.run(c.full, warmup)
        torch.cuda.synchronize()
        wall0 = time.perf_counter()
        call_us = timer.run(c.full, steps)
        wall = time.perf_counter() - wall0
        pass1_us = timer.run(c.dominant(), steps)
        # the same steps between default-flag events (torch.cuda.Event), as earlier lines
        # timed them
        default_us = timer.run(c.full, steps, events=TorchEvents(torch))
    call_us.sort()
    p50 = statistics.median(call_us)
    p95 = percentile(call_us, 95)
    p1_avg = statistics.fmean(pass1_us) if pass1_us else p50
    achieved = wl.bytes / (p1_avg * 1e-6) / 1e9           # GB/s, the dominant kernel alone
    # final correctness of the timed output (a single call with --no-check keeps the timed
    # call's output as it is)
    if not args.no_check:
        dk_lib.check(c.full(), "decode_attention")
    torch.cuda.synchronize()
    finite = bool(torch.isfinite(c.out).all())
    hq, hkv, d = wl.hq, wl.hkv, wl.d
    mfma_qk = args.qk_path == 1 or (args.qk_path == 0 and (hq // hkv > 4 or (wl.kv8 and d >= 256)))
    metric_workload = ((wl.batch, wl.ctx, hq, hkv, d) == (32, 8192, 32, 8, 128)
                       and wl.table == "permuted" and not wl.ragged_min and not extension)
    rec = {
        "metric": METRIC, "value": round(wl.bytes / (p50 * 1e-6) / 1e12, 4), "unit": "TB/s",
        "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(p50 / 1e3, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": args.dtype, "data": "synthetic",
        "config": {"workload": wl.label(),
                   "kv_dtype": "fp8_e4m3" if wl.kv8 else args.dtype,
                   "batch": wl.batch,
                   "context_length": f"U[{wl.ragged_min},{wl.ctx}]" if wl.ragged_min else wl.ctx,
                   "num_q_heads": hq, "num_kv_heads": hkv, "head_dim": d, "page_size": 16,
                   "split_kv": split, "schedule": c.schedule_name(),
                   "plan_hint_max_pages": hint,
                   "qk_path": "mfma" if mfma_qk else "valu", "pv_path": "mfma"},
        "us_per_call": round(p50, 2), "us_per_call_p95": round(p95, 2),
        "pct_of_peak": round(100 * wl.bytes / (p50 * 1e-6) / (PEAK_GBPS * 1e9), 2),
        "timing_events": "hipEventDisableSystemFence",
        "us_per_call_default_events": (round(statistics.median(default_us), 2)
                                       if default_us else None),
        "bytes_per_call": wl.bytes, "wall_s_timed_loop": round(wall, 3),
        "pass1_us_avg": round(p1_avg, 2), "output_finite": finite,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_GBPS, 4),
                     "traffic": None, "traffic_from": None,
                     "kernel": "dk_pass1_balanced" if c.schedule == 0 else "dk_pass1_split"},
        "cpu_baseline": None,
    }
    if metric_workload:
        traffic, stamp = read_traffic(args.kv_dtype)
        rec["roofline"].update(traffic=traffic, traffic_from=stamp)
    if args.single_call:
        rec["mode"] = ("single call (no settling, no warm-up" +
                       (", no checking calls: the run's only decode dispatch)"
                        if args.no_check else ")"))
    if extension:
        # the reference has neither: no CPU baseline of its path; the output against the
        # oracle's masked form with the same options on the first and last sequences
        rec["config"].update({"sinks": bool(args.sinks), "window": args.window})
        from oracle.reference import reference_attention_paged
        seqs = oracle_sequences(wl)
        sub = _host_subproblem(wl, seqs)
        qn, kvn, ipn, idn, ln = (t.float().numpy() if t.is_floating_point() else t.numpy()
                                 for t in sub)
        want = reference_attention_paged(
            qn, kvn, ipn, idn, ln, window=args.window or None,
            sinks=None if not args.sinks else wl.sinks.cpu().numpy())
        rec["max_abs_err_vs_fp32"] = max_abs_err(c.out, torch.from_numpy(want), seqs)
        rec["oracle_sequences"] = seqs
    elif not args.no_cpu_baseline:
        ncpu, threads, model = host_cpu()
        if wl.ragged_min:
            n = min(args.cpu_sample or 8, wl.batch)
            seqs = list(range(n))
            t, want = cpu_baseline_masked(wl, seqs, threads)
            pages = lambda bs: sum(int(wl.indptr_host[b + 1] - wl.indptr_host[b]) for b in bs)  # noqa: E731
            total_us = t * pages(range(wl.batch)) / max(pages(seqs), 1) * 1e6
            base = {"value": round(total_us, 1), "unit": "us/call", "cores": threads,
                    "kind": "port",
                    "sample": f"numpy fp32 per-sequence oracle (oracle/reference.py; the "
                              f"reference's zero-padded form is wrong for ragged batches) on "
                              f"{n} of {wl.batch} sequences, median of 3, scaled to the "
                              f"whole batch by pages"}
        else:
            n = min(args.cpu_sample or wl.batch, wl.batch)
            seqs = list(range(n))
            tg, ta, tt, want = cpu_baseline_literal(wl, seqs, threads)
            scale = wl.batch / n
            base = {"value": round(tt * scale * 1e6, 1), "unit": "us/call", "cores": threads,
                    "kind": "port", "gather_us": round(tg * scale * 1e6, 1),
                    "attention_us": round(ta * scale * 1e6, 1),
                    "sample": f"the reference's CPU path (src/reference.py) restated in torch "
                              f"(oracle/reference_torch.py: pool to fp32, per-page gather into "
                              f"zero-padded dense K/V, repeat_interleave GQA, fp32 softmax "
                              f"attention) on {n} of {wl.batch} sequences"
                              f"{'' if n == wl.batch else ' (scaled to the batch)'}, "
                              f"median of 3, gather and attention timed separately"}
        base.update({"cpu_count": ncpu, "threads": threads, "cpu_model": model,
                     "threads_note": f"threads = min(os.cpu_count(), {CPU_THREADS_CAP}): the "
                                     f"GPU box's CPU share per GPU"})
        base["tb_s"] = round(wl.bytes / (base["value"] * 1e-6) / 1e12, 6)
        rec["cpu_baseline"] = base
        rec["max_abs_err_vs_fp32"] = max_abs_err(c.out, want, seqs)
    if metric_workload and not wl.kv8 and not args.single_call and not args.no_extra_configs:
        # the other BASELINE configs, measured in the same run after the metric
        del c, wl
        release_device_memory(torch)
        rec["baseline_configs"] = extra_points_run(args, torch, lib, dk_lib, attention,
                                                   layout, dev, stream, host_cpu()[1])
    print(json.dumps(rec), flush=True)
    if args.calibration_copy > 0:
        src = torch.ones(args.calibration_copy << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(2):
            dst.copy_(src)
        torch.cuda.synchronize()


def config_workload(torch, layout, dev, shape, kv_dtype="same"):
    """The Workload of one CONFIGS shape (a dict without its "splits")."""
    shape = dict(shape)
    shape.pop("splits", None)
    return Workload(torch, layout, dev, shape.pop("batch"), shape.pop("ctx"),
                    d=shape.pop("d", 128), kv_dtype=kv_dtype, **shape)


def oracle_sequences(wl):
    """Sequences the CPU oracle checks: the first and the last (one for very long
    contexts)."""
    return [0] if wl.batch == 1 or max(wl.lens) > 65536 else [0, wl.batch - 1]


def measure_point(args, dk_lib, attention, lib, timer, wl, split, stream, want=None,
                  seqs=None, settle=False):
    """p50 / p95 us of the full call (flush + events; settling steps when `settle`, then
    the warm-up), the dominant kernel's average, and the max-abs error of the output
    against `want` (the CPU oracle's rows of sequences `seqs`) when given."""
    torch = wl.torch
    opts, hint = make_opts(dk_lib, args, wl, split)
    c = Caller(lib, dk_lib, attention, wl, split, opts, stream)
    dk_lib.check(c.full(), "decode_attention")
    if settle:
        timer.settle(c.full)
    timer.run(c.full, args.warmup)
    us = sorted(timer.run(c.full, args.steps))
    p1 = timer.run(c.dominant(), args.steps)
    dk_lib.check(c.full(), "decode_attention")
    torch.cuda.synchronize()
    p50, p95 = statistics.median(us), percentile(us, 95)
    tbs = wl.bytes / (p50 * 1e-6) / 1e12
    res = {"split_kv": split, "schedule": c.schedule_name(), "plan_hint_max_pages": hint,
           "us_per_call": round(p50, 2), "us_per_call_p95": round(p95, 2),
           "tb_s": round(tbs, 4), "frac": round(tbs * 1e12 / (PEAK_GBPS * 1e9), 4),
           "dominant_kernel_us_avg": round(statistics.fmean(p1), 2),
           "bytes_per_call": wl.bytes, "output_finite": bool(torch.isfinite(c.out).all())}
    if want is not None:
        res["max_abs_err_vs_fp32"] = max_abs_err(c.out, want, seqs)
        res["oracle_sequences"] = seqs
    del c
    return res


# The BASELINE configs' headline points carried in the default run's line (each config's
# stated split where it names one, else the library's automatic schedule), plus the fp8
# cache at the metric shape (an extension).
EXTRA_POINTS = [
    (1, dict(CONFIGS[1][0]), 4, "same"),
    (1, dict(CONFIGS[1][0]), 0, "same"),
    *[(2, dict(s), 0, "same") for s in CONFIGS[2]],
    *[(3, dict(s), 0, "same") for s in CONFIGS[3]],
    (4, dict(CONFIGS[4][0]), 0, "same"),
    (5, dict(CONFIGS[5][0]), 0, "same"),
    (0, dict(batch=32, ctx=8192, dtype="fp16", table="permuted"), 0, "fp8"),
]


def extra_points_run(args, torch, lib, dk_lib, attention, layout, dev, stream, threads):
    """The EXTRA_POINTS, each checked against the CPU oracle on sampled sequences."""
    timer = Timer(torch, dev, stream, args.flush)
    out = []
    for cid, shape, split, kv_dtype in EXTRA_POINTS:
        wl = config_workload(torch, layout, dev, shape, kv_dtype)
        seqs = oracle_sequences(wl)
        want = None
        if not args.no_cpu_baseline:
            _, want = cpu_baseline_masked(wl, seqs, threads, reps=1)
        r = {"config_id": cid, "workload": wl.label()}
        # settled on each point: a point's first timed steps otherwise ran up to 5 % slow
        # after a different shape
        r.update(measure_point(args, dk_lib, attention, lib, timer, wl, split, stream, want,
                               seqs, settle=True))
        out.append(r)
        # each point's buffers come from fresh device allocations, as in a run of its own
        del wl, want
        release_device_memory(torch)
    return out


def config_run(args, torch, lib, dk_lib, attention, layout, dev, stream):
    """BASELINE config N: one JSON line per (shape, split_kv) point of its sweep."""
    ncpu, threads, model = host_cpu()
    timer = Timer(torch, dev, stream, args.flush)
    for shape in CONFIGS[args.config]:
        splits = shape["splits"]
        wl = config_workload(torch, layout, dev, shape)
        # the CPU oracle on sampled sequences: the checker of every split of this shape
        # and its CPU baseline
        seqs = oracle_sequences(wl)
        cpu_s, want = None, None
        if not args.no_cpu_baseline:
            cpu_s, want = cpu_baseline_masked(wl, seqs, threads, reps=1)
        # each shape settles its first split (the CPU oracle above left the GPU idle)
        settled = False
        for split in splits:
            if not settled:
                opts, _ = make_opts(dk_lib, args, wl, split)
                timer.settle(Caller(lib, dk_lib, attention, wl, split, opts, stream).full)
                settled = True
            m = measure_point(args, dk_lib, attention, lib, timer, wl, split, stream, want,
                              seqs)
            rec = {
                "metric": CONFIG_METRIC.format(n=args.config), "value": m["tb_s"],
                "unit": "TB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                "ms_per_step": round(m["us_per_call"] / 1e3, 5), "higher_is_better": True,
                "dtype": wl.dtype_name, "data": "synthetic",
                "config": {"config_id": args.config, "workload": wl.label(),
                           "batch": wl.batch, "context_length":
                               f"U[{wl.ragged_min},{wl.ctx}]" if wl.ragged_min else wl.ctx,
                           "num_q_heads": wl.hq, "num_kv_heads": wl.hkv, "head_dim": wl.d,
                           "split_kv": split, "schedule": m["schedule"],
                           "plan_hint_max_pages": m["plan_hint_max_pages"]},
                "us_per_call": m["us_per_call"], "us_per_call_p95": m["us_per_call_p95"],
                "frac": m["frac"], "pct_of_peak": round(100 * m["frac"], 2),
                "dominant_kernel_us_avg": m["dominant_kernel_us_avg"],
                "bytes_per_call": wl.bytes, "output_finite": m["output_finite"],
            }
            if want is not None:
                rec["max_abs_err_vs_fp32"] = m["max_abs_err_vs_fp32"]
                rec["oracle_sequences"] = seqs
                rec["cpu_baseline"] = {
                    "value": round(cpu_s * 1e6, 1), "unit": "us for the sampled sequences",
                    "cores": threads, "kind": "port", "cpu_count": ncpu, "cpu_model": model,
                    "sample": f"numpy fp32 per-sequence oracle (oracle/reference.py) on "
                              f"sequences {seqs}, one run"}
            print(json.dumps(rec), flush=True)
        del wl
        release_device_memory(torch)


# --graph points: the latency-bound configs, each as N back-to-back calls on N caches of
# its shape (label, BASELINE config, shape, split_kv, layers; 0 layers = enough for 1 GiB)
GRAPH_POINTS = [
    ("C1", 1, dict(CONFIGS[1][0]), 4, 0),
    ("C1 auto", 1, dict(CONFIGS[1][0]), 0, 0),
    ("C2 B=1", 2, dict(batch=1, ctx=4096, dtype="fp16", table="permuted"), 0, 0),
    ("C2 B=4", 2, dict(batch=4, ctx=4096, dtype="fp16", table="permuted"), 0, 0),
    ("C3 B=1 ctx 32768", 3, dict(batch=1, ctx=32768, dtype="bf16", table="permuted"), 0, 0),
    ("C5 step", 5, dict(CONFIGS[5][0]), 0, 16),     # the 16 attention layers of the step
]
GRAPH_MIN_BYTES = 1 << 30      # the N caches of a point together: > L2 + Infinity Cache


def graph_run(args, torch, lib, dk_lib, attention, layout, dev, stream):
    """Per point: the flush + events protocol's p50 for one call, then N calls on N
    distinct caches back to back (events around the whole sequence, no flush: the caches
    together exceed every cache level), eager and as one captured HIP graph replayed, as a
    model step runs its attention layers. Reports us per call of each; checks that every
    layer's output of a replay equals its eager output bit for bit."""
    timer = Timer(torch, dev, stream, args.flush)
    cap = torch.cuda.Stream(dev)
    points = [p for p in GRAPH_POINTS if not args.graph_point or p[0] == args.graph_point]
    if not points:
        raise SystemExit(f"--graph-point {args.graph_point!r}: no such point "
                         f"({', '.join(p[0] for p in GRAPH_POINTS)})")
    for label, cid, shape, split, layers in points:
        wl0 = config_workload(torch, layout, dev, shape)
        n = layers or max(16, -(-GRAPH_MIN_BYTES // wl0.bytes))
        wls = [wl0] + [config_workload(torch, layout, dev, dict(shape, seed=1 + i))
                       for i in range(1, n)]
        proto = measure_point(args, dk_lib, attention, lib, timer, wl0, split, stream,
                              settle=True)
        opts = [make_opts(dk_lib, args, wl, split)[0] for wl in wls]
        callers = [Caller(lib, dk_lib, attention, wl, split, o, cap)
                   for wl, o in zip(wls, opts)]

        def step():
            for c in callers:
                dk_lib.check(c.full(), "decode_attention")

        def timed(fn, reps):
            ev = timer.events
            evs = ev.pairs(reps)
            with torch.cuda.stream(cap):
                for e0, e1 in evs:
                    ev.record(e0, cap)
                    fn()
                    ev.record(e1, cap)
            torch.cuda.synchronize()
            return sorted(ev.elapsed_us(evs))

        # eager, back to back (the first steps also load every kernel before the capture)
        timed(step, max(args.warmup, 2))
        eager = timed(step, args.steps)
        want = [c.out.clone() for c in callers]
        for c in callers:
            c.out.fill_(float("nan"))
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cap):
            step()
        timed(g.replay, max(args.warmup, 2))
        graph = timed(g.replay, args.steps)
        same = all(torch.equal(c.out, w) for c, w in zip(callers, want))
        p50e, p50g = statistics.median(eager) / n, statistics.median(graph) / n
        rec = {
            "metric": "µs per call of N back-to-back calls on N caches (HIP graph replay)",
            "value": round(p50g, 2), "unit": "us/call", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "higher_is_better": False, "dtype": wl0.dtype_name,
            "data": "synthetic",
            "config": {"point": label, "config_id": cid, "workload": wl0.label(),
                       "split_kv": split, "schedule": proto["schedule"], "layers": n,
                       "bytes_per_call": wl0.bytes},
            "us_per_call_graph": round(p50g, 2),
            "us_per_call_graph_p95": round(percentile(graph, 95) / n, 2),
            "us_per_call_eager": round(p50e, 2),
            "us_per_call_protocol": proto["us_per_call"],
            "tb_s_graph": round(wl0.bytes / (p50g * 1e-6) / 1e12, 4),
            "frac_graph": round(wl0.bytes / (p50g * 1e-6) / (PEAK_GBPS * 1e9), 4),
            "us_per_replay": round(statistics.median(graph), 2),
            "graph_matches_eager": same,
        }
        print(json.dumps(rec), flush=True)
        if not same:
            raise RuntimeError(f"{label}: a graph replay's output differs from the eager call's")
        del g, callers, wls, wl0, want
        release_device_memory(torch)


def host_overhead_run(args, torch, lib, dk_lib, attention, layout, dev, stream):
    """Host microseconds per call, issued back to back (no flush, no sync inside the
    timed loop; the GPU runs behind): the bare C-ABI call with prebuilt arguments, the
    Python entry point with its cached plan, and the Python entry point validating its
    arguments afresh on every call (its cache cleared), as every call did before."""
    wl = Workload(torch, layout, dev, args.batch, args.ctx, args.num_q_heads,
                  args.num_kv_heads, args.head_dim, args.dtype, args.page_table)
    split = attention.resolve_split(args.split)
    opts, hint = make_opts(dk_lib, args, wl, split)
    c = Caller(lib, dk_lib, attention, wl, split, opts, stream)
    q, kv, ip, ids, last = wl.q, wl.kv, wl.indptr, wl.ids, wl.last

    def py():
        return attention.decode_attention(q, kv, ip, ids, last, split_kv=split,
                                          max_pages_per_seq=hint)

    def py_fresh():
        attention._PLANS.clear()
        return py()

    plan = attention.DecodePlan(q, kv, ip, ids, last, split_kv=split, max_pages_per_seq=hint,
                                out=c.out)

    def py_plan():
        return plan.run(q, kv, ip, ids, last, out=c.out)

    res = {}
    for name, fn in (("c_abi", c.full), ("decode_plan_run_with_out", py_plan),
                     ("decode_attention", py), ("decode_attention_unplanned", py_fresh)):
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        n = 200
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        t = time.perf_counter() - t0
        torch.cuda.synchronize()
        res[name] = round(t / n * 1e6, 2)
    print(json.dumps({"metric": "host us per decode call (issue only, back to back)",
                      "unit": "us", "config": {"workload": wl.label(), "split_kv": split,
                                               "plan_hint_max_pages": hint,
                                               "schedule": c.schedule_name()},
                      "host_us_per_call": res}), flush=True)


def wide_pages_run(args, torch, attention, dev, stream):
    """decode_attention over pages of args.page_size tokens (a multiple of 16): the page
    table is rewritten over 16-token sub-pages on the device inside every timed call. One
    JSON line; the output against the oracle on the original layout (first and last
    sequence)."""
    import numpy as np

    from oracle.reference import reference_attention_paged
    P, B, ctx = args.page_size, args.batch, args.ctx
    hq, hkv, d = args.num_q_heads, args.num_kv_heads, args.head_dim
    dtype = torch.float16 if args.dtype == "fp16" else torch.bfloat16
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    npg = -(-ctx // P)
    kv = torch.randn(B * npg, 2, P, hkv, d, generator=g, device=dev, dtype=dtype)
    q = torch.randn(B, hq, d, generator=g, device=dev, dtype=dtype)
    ids = torch.randperm(B * npg, generator=g, device=dev).to(torch.int32)
    indptr = torch.arange(B + 1, device=dev, dtype=torch.int32) * npg
    last = torch.full((B,), ctx - (npg - 1) * P, device=dev, dtype=torch.int32)
    out = torch.empty_like(q)
    hint = 0 if args.no_plan_hint else npg
    split = attention.resolve_split(args.split)

    def call():
        attention.decode_attention(q, kv, indptr, ids, last, split, out=out,
                                   max_pages_per_seq=hint, qk_path=args.qk_path,
                                   waves_per_group=args.waves, waves_per_cu=args.waves_per_cu,
                                   schedule=args.schedule)
    timer = Timer(torch, dev, stream, args.flush)
    call()
    timer.settle(call)
    timer.run(call, args.warmup)
    us = sorted(timer.run(call, args.steps))
    p50 = statistics.median(us)
    torch.cuda.synchronize()
    nbytes = B * ctx * hkv * d * 2 * 2 + 2 * B * hq * d * 2
    seqs = [0, B - 1] if B > 1 else [0]
    want = []
    for b in seqs:
        pages = ids[b * npg:(b + 1) * npg].long()
        kvb = kv[pages].float().cpu().numpy()
        want.append(reference_attention_paged(
            q[b:b + 1].float().cpu().numpy(), kvb, np.array([0, npg], np.int32),
            np.arange(npg, dtype=np.int32), last[b:b + 1].cpu().numpy())[0])
    err = float(np.abs(out[seqs].float().cpu().numpy() - np.stack(want)).max())
    print(json.dumps({
        "metric": "us/call of decode_attention over pages of a multiple of 16 tokens",
        "unit": "us", "value": round(p50, 2), "us_per_call_p95": round(percentile(us, 95), 2),
        "tb_s": round(nbytes / (p50 * 1e-6) / 1e12, 4),
        "pct_of_peak": round(100 * nbytes / (p50 * 1e-6) / (PEAK_GBPS * 1e9), 2),
        "config": {"workload": f"paged decode attention B={B} ctx={ctx} Hq={hq} Hkv={hkv} "
                               f"D={d} {args.dtype} page_size={P} permuted pages",
                   "split_kv": split, "plan_hint_max_pages": hint,
                   "path": "Python decode_attention (page table rewritten per call)"},
        "steps": args.steps, "warmup": args.warmup, "max_abs_err_vs_fp32": err,
        "oracle_sequences": seqs}), flush=True)


def main(argv=None):
    args = parse_args(argv)
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
    stream = torch.cuda.current_stream(dev)
    if args.host_overhead:
        host_overhead_run(args, torch, lib, dk_lib, attention, layout, dev, stream)
    elif args.config:
        config_run(args, torch, lib, dk_lib, attention, layout, dev, stream)
    elif args.graph:
        graph_run(args, torch, lib, dk_lib, attention, layout, dev, stream)
    elif args.page_size != 16:
        wide_pages_run(args, torch, attention, dev, stream)
    else:
        metric_run(args, torch, lib, dk_lib, attention, layout, dev, stream)
    return 0


if __name__ == "__main__":
    sys.exit(main())
