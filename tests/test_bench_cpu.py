"""bench.py's host side: the one-GPU contract, the algorithmic work it credits
and the committed counter summary it reads (no GPU needed)."""

import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert msg["n_gpus"] == 2 and "one GPU" in msg["error"]


@pytest.mark.parametrize("B,H,n,d,tflop", [
    (1, 32, 1024, 128, 0.0258),     # cfg1
    (1, 32, 4096, 128, 0.412),      # cfg2 Q/Q
    (1, 32, 8192, 128, 1.650),      # cfg3 Q/Q
    (1, 8, 8192, 128, 0.412),       # cfg3 K/K
    (1, 32, 32768, 128, 26.389),    # cfg4
    (2, 48, 16384, 128, 19.79),     # cfg5, one layer (48 head relations)
])
def test_algorithmic_flops_match_the_published_counts(B, H, n, d, tflop):
    """12 d P per (b, h) relation with P = n(n+1)/2 causal pairs; the counts
    are the ones the benchmark definition quotes (three significant digits)."""
    got = bench.algorithmic_flops(B, H, n, d) / 1e12
    assert abs(got - tflop) <= 0.0005 * tflop + 5e-4, (got, tflop)


def test_cfg5_step_work_is_633_tflop():
    assert round(32 * bench.algorithmic_flops(2, 48, 16384, 128) / 1e12) == 633


def test_committed_traffic_summary_is_readable():
    s = bench.traffic_summary("cfg4")
    assert s is not None
    for k in ("forward_rowgrad", "col_grad"):  # the autograd path's two kernels
        assert s["bytes_per_launch"][k] > 0
        # read + write bytes add up to the total per launch
        assert abs(s["read_bytes"][k] + s["write_bytes"][k] - s["bytes_per_launch"][k]) <= 1e-6 * s["bytes_per_launch"][k]
    assert bench.traffic_summary("no-such-config") is None


def test_host_and_clock_helpers():
    import torch

    assert isinstance(bench.host_cpu(), str) and bench.host_cpu()
    clock = bench.gpu_clock(torch)  # no device here: only what the driver exposes, never an exception
    assert isinstance(clock, dict)
