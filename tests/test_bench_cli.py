"""bench.py's contract on the CPU: the one-GPU limit, argument checks, and the recorded
HBM traffic it reports."""
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_ragged_lengths_beyond_the_context_are_refused_before_any_gpu_work():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--ragged-min", "9000"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "--ragged-min must be in [1, ctx=8192]" in r.stderr
    assert r.stdout == ""


@pytest.mark.parametrize("kv_dtype,algorithmic", [("same", 1_074_331_908),
                                                  ("fp8", 537_460_996)])
def test_recorded_traffic_is_stamped_and_close_to_the_algorithmic_bytes(kv_dtype, algorithmic):
    # profiles/*_hbm_traffic.md hold rocprofv3 FETCH_SIZE + WRITE_SIZE per launch, the commit
    # and the digest of the kernel sources they were measured on; the bench line reports the
    # bytes as roofline.traffic (null when the sources have changed since) and the stamp as
    # roofline.traffic_from. Every cache byte is read once: within 1 %.
    text = bench.TRAFFIC_FILES[kv_dtype].read_text()
    raw = int(text.split("traffic_bytes_per_launch:")[1].split()[0])
    assert abs(raw / algorithmic - 1.0) < 0.01, raw
    t, stamp = bench.read_traffic(kv_dtype)
    assert stamp["commit"] and len(stamp["kernel_source_digest"]) == 16
    assert stamp["current_digest"] == bench.kernel_source_digest()
    assert t == (raw if stamp["matches_build"] else None)


def test_traffic_from_other_kernel_sources_is_not_reported(tmp_path, monkeypatch):
    prof = tmp_path / "traffic.md"
    monkeypatch.setitem(bench.TRAFFIC_FILES, "same", prof)
    monkeypatch.setattr(bench, "ROOT", tmp_path)
    body = "traffic_bytes_per_launch: 1075613696\nmeasured_at_commit: 0123abcd\n"
    prof.write_text(body + f"kernel_source_digest: {bench.kernel_source_digest()}\n")
    t, stamp = bench.read_traffic("same")
    assert t == 1075613696 and stamp["matches_build"] and stamp["commit"] == "0123abcd"
    prof.write_text(body + "kernel_source_digest: 0000000000000000\n")
    t, stamp = bench.read_traffic("same")
    assert t is None and not stamp["matches_build"]
    prof.write_text(body)                                 # no digest recorded: not trusted
    assert bench.read_traffic("same")[0] is None


def test_kernel_source_digest_follows_every_library_source(tmp_path, monkeypatch):
    src = tmp_path / "csrc"
    src.mkdir()
    (src / "a.h").write_text("x")
    (src / "b.hip").write_text("y")
    (src / "notes.txt").write_text("not a source")
    monkeypatch.setattr(bench, "KERNEL_SOURCES", src)
    d0 = bench.kernel_source_digest()
    (src / "notes.txt").write_text("changed")
    assert bench.kernel_source_digest() == d0
    (src / "b.hip").write_text("y2")
    assert bench.kernel_source_digest() != d0
    (src / "b.hip").write_text("y")
    (src / "c.cpp").write_text("")
    assert bench.kernel_source_digest() != d0


def test_single_call_checks_and_graph_mode_combinations_are_refused():
    assert bench.parse_args(["--single-call", "--no-check"]).no_check
    assert bench.parse_args(["--graph", "--graph-point", "C2 B=1"]).graph
    for argv, needle in ((["--no-check"], "--no-check"),
                         (["--graph", "--config", "5"], "--graph"),
                         (["--graph", "--single-call"], "--graph")):
        r = subprocess.run([sys.executable, str(ROOT / "bench.py"), *argv],
                           capture_output=True, text=True, timeout=120)
        assert r.returncode == 2 and needle in r.stderr and r.stdout == ""


def test_graph_points_cover_the_latency_bound_configs():
    # config 1 at its stated split and automatic, config 2 at B=1 and B=4, config 3's
    # shortest single sequence, config 5's 16-layer step; every point's N caches together
    # exceed 1 GiB
    import torch

    import layout
    labels = [p[0] for p in bench.GRAPH_POINTS]
    assert labels == ["C1", "C1 auto", "C2 B=1", "C2 B=4", "C3 B=1 ctx 32768", "C5 step"]
    (c5,) = [p for p in bench.GRAPH_POINTS if p[1] == 5]
    assert c5[4] == 16 and c5[2]["d"] == 64 and c5[2]["dtype"] == "bf16"
    for label, cid, shape, split, layers in bench.GRAPH_POINTS:
        bytes_ = layout.attention_bytes(shape["batch"], [shape["ctx"]] * shape["batch"], 32, 8,
                                        shape.get("d", 128))
        n = layers or max(16, -(-bench.GRAPH_MIN_BYTES // bytes_))
        assert n * bytes_ >= bench.GRAPH_MIN_BYTES, label
    del torch


def test_roctx_ranges_are_off_without_dk_trace(monkeypatch):
    monkeypatch.delenv("DK_TRACE", raising=False)
    assert bench.roctx_ranges() is None
    monkeypatch.setenv("DK_TRACE", "0")
    assert bench.roctx_ranges() is None


def test_config_sweeps_follow_baseline_json():
    import json
    base = json.loads((ROOT / "BASELINE.json").read_text())
    assert len(base["configs"]) == len(bench.CONFIGS) == 5
    c1, = bench.CONFIGS[1]
    assert (c1["batch"], c1["ctx"], c1["table"], c1["splits"][0]) == (2, 512, "contiguous", 4)
    assert [s["batch"] for s in bench.CONFIGS[2]] == [1, 4, 16, 32, 64]
    assert all(s["ctx"] == 4096 and set(s["splits"]) >= {1, 2, 4, 8, 16}
               for s in bench.CONFIGS[2])
    assert {(s["batch"], s["ctx"]) for s in bench.CONFIGS[3]} == {
        (1, 32768), (1, 131072), (4, 32768), (4, 131072)}
    assert all(s["dtype"] == "bf16" and set(s["splits"]) >= {16, 32, 64, 128}
               for s in bench.CONFIGS[3])
    c4, = bench.CONFIGS[4]
    assert (c4["batch"], c4["ragged_min"], c4["ctx"], c4["table"]) == (128, 128, 8192, "freelist")
    c5, = bench.CONFIGS[5]
    assert (c5["batch"], c5["ctx"], c5["d"], c5["dtype"]) == (32, 2048, 64, "bf16")


def test_single_call_does_not_combine_with_a_config_sweep():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--single-call", "--config", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "--single-call" in r.stderr and r.stdout == ""


def test_extension_options_are_checked_while_parsing():
    """--sinks / --window apply to the default workload only, and a window is >= 0."""
    assert bench.parse_args(["--sinks", "--window", "128"]).window == 128
    assert bench.parse_args(["--page-size", "64"]).page_size == 64
    for argv, needle in ((["--sinks", "--config", "2"], "--sinks"),
                         (["--window", "-3"], "--window"),
                         (["--page-size", "24"], "--page-size"),
                         (["--page-size", "32", "--sinks"], "--page-size")):
        r = subprocess.run([sys.executable, str(ROOT / "bench.py"), *argv],
                           capture_output=True, text=True, timeout=120)
        assert r.returncode == 2 and needle in r.stderr and r.stdout == ""


def test_host_cpu_reports_count_threads_and_model():
    n, threads, model = bench.host_cpu()
    assert n >= 1 and 1 <= threads <= min(n, bench.CPU_THREADS_CAP) and model


@pytest.mark.parametrize("ragged", [False, True])
def test_cpu_baseline_legs_agree_with_the_oracle(ragged):
    # the two CPU-baseline forms on a small CPU-resident workload: the literal torch path
    # (uniform lengths) and the masked numpy oracle, on a subset of sequences
    import numpy as np
    import torch

    import layout
    from oracle.reference import reference_attention_paged
    wl = bench.Workload(torch, layout, "cpu", 5, 200, hq=8, hkv=2, d=64,
                        ragged_min=17 if ragged else 0, table="permuted")
    seqs = [0, 3, 4]
    want = reference_attention_paged(wl.q.numpy(), wl.kv.numpy(), wl.indptr.numpy(),
                                     wl.ids.numpy(), wl.last.numpy())[seqs]
    t, got = bench.cpu_baseline_masked(wl, seqs, threads=1, reps=1)
    assert t > 0 and np.abs(got.numpy() - want).max() < 1e-6
    if not ragged:
        tg, ta, tt, got = bench.cpu_baseline_literal(wl, seqs, threads=1, reps=1)
        assert tg > 0 and ta > 0 and abs(tt - tg - ta) < 1e-9
        assert np.abs(got.numpy() - want).max() < 2e-6
        assert bench.max_abs_err(torch.from_numpy(np.zeros((5, 8, 64), np.float16)), got, seqs) \
            == float(got.abs().max())


def test_default_line_carries_every_baseline_config():
    # the metric run's `baseline_configs`: config 1 at its stated split 4 and automatic,
    # every config 2 batch, all four config 3 shapes, the ragged mix and config 5, plus
    # the fp8 cache at the metric shape
    pts = bench.EXTRA_POINTS
    assert {cid for cid, *_ in pts} == {0, 1, 2, 3, 4, 5}
    assert [(s["batch"], split) for cid, s, split, _ in pts if cid == 1] == [(2, 4), (2, 0)]
    assert sorted(s["batch"] for cid, s, _, _ in pts if cid == 2) == [1, 4, 16, 32, 64]
    assert {(s["batch"], s["ctx"]) for cid, s, _, _ in pts if cid == 3} == {
        (1, 32768), (1, 131072), (4, 32768), (4, 131072)}
    assert [kv for cid, _, _, kv in pts if cid == 0] == ["fp8"]
    # shapes build as the config sweeps build them (on the CPU, at a small context; the
    # ragged mix's 65536-page free list is left out here)
    import torch

    import layout
    for cid, shape, _, kv in pts:
        if shape.get("ragged_min"):
            continue
        small = dict(shape, batch=2, ctx=64)
        wl = bench.config_workload(torch, layout, "cpu", small, "same")
        assert wl.d == shape.get("d", 128) and wl.dtype_name == shape["dtype"]
        assert bench.oracle_sequences(wl) == [0, 1]


def test_timing_events_skip_the_system_fence():
    # the timed regions' events are created with hipEventDisableSystemFence, whose value is
    # the HIP header's; earlier lines' default-flag events stay available for comparison
    import re
    header = Path("/opt/rocm/include/hip/hip_runtime_api.h")
    if header.exists():
        m = re.search(r"#define\s+hipEventDisableSystemFence\s+(0x[0-9a-fA-F]+)", header.read_text())
        assert m and int(m.group(1), 16) == bench.HIP_EVENT_DISABLE_SYSTEM_FENCE
    assert bench.HipEvents.__init__.__defaults__ == (bench.HIP_EVENT_DISABLE_SYSTEM_FENCE,)
    import inspect
    assert inspect.signature(bench.Timer).parameters["events"].default == "nofence"
