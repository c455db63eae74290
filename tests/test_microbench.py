"""The microbenchmark harness: CSV schema and bytes model of the reference's
bench/microbench_cuda.py (columns :222-236, bytes :114-121); a tiny sweep on the GPU."""
import csv

import pytest
import torch

import microbench


def test_columns_and_bytes_model_match_the_reference():
    assert microbench.REFERENCE_COLUMNS == [
        "implementation", "context_length", "batch_size", "split_kv", "latency_ms_p50",
        "latency_ms_p95", "achieved_bw_gb_s", "peak_bw_gb_s", "bw_pct_of_peak",
        "max_abs_err_vs_fp32"]
    assert microbench.COLUMNS == microbench.REFERENCE_COLUMNS + [
        "dtype", "config_id", "fetch_bytes", "cpu_cores"]
    # the BASELINE config grids
    cid, dt, ctxs, batches, splits, _ = microbench.SWEEPS["config2"]
    assert (cid, ctxs, batches, splits) == (2, [4096], [1, 4, 16, 32, 64], [1, 2, 4, 8, 16])
    cid, dt, ctxs, batches, splits, _ = microbench.SWEEPS["config3"]
    assert (cid, dt, ctxs, batches, splits) == (3, torch.bfloat16, [32768, 131072], [1, 4],
                                                [16, 32, 64, 128])
    # q + out + K/V (2 bytes each) at the reference's default shape
    assert microbench.attention_bytes(1, 2048, 32, 8, 128) == 2 * 32 * 128 * 2 + 2048 * 8 * 128 * 4
    args = microbench.parse_args(["--quick", "--out", "x.csv"])
    assert args.quick and args.out == "x.csv"
    assert microbench.parse_args(["--sweep", "config3"]).sweep == "config3"


@pytest.mark.gpu
def test_tiny_sweep_writes_the_csv(tmp_path):
    out = tmp_path / "mb.csv"
    rows = microbench.run_sweep([512], [2], [1, 3], ["hip_naive", "hip_split_kv", "hip_auto"],
                                str(out), timed_iters=3)
    got = list(csv.DictReader(out.open()))
    assert [r["implementation"] for r in got] == ["hip_naive", "hip_split_kv", "hip_split_kv",
                                                  "hip_auto"]
    assert len(rows) == 4 and all(float(r["max_abs_err_vs_fp32"]) <= 1e-2 for r in got)
    assert all(r["dtype"] == "fp16" and r["config_id"] == "0" and int(r["fetch_bytes"]) > 0
               and int(r["cpu_cores"]) >= 1 for r in got)
    assert all(float(r["latency_ms_p50"]) > 0 for r in got)
