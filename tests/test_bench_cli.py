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
def test_recorded_traffic_is_read_and_close_to_the_algorithmic_bytes(kv_dtype, algorithmic):
    # profiles/*_hbm_traffic.md hold rocprofv3 FETCH_SIZE + WRITE_SIZE per launch; the bench
    # line reports them as roofline.traffic. Every cache byte is read once: within 1 %.
    t = bench.read_traffic(kv_dtype)
    assert t is not None
    assert abs(t / algorithmic - 1.0) < 0.01, t
