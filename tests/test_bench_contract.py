"""The parts of bench.py's contract that run without a GPU.

* ``--gpus N`` with N > 1 exits with a message and status 2 before touching torch or the
  GPU (this build measures one GPU);
* the committed flash-kernel profile carries the three figures the bench line quotes beside
  its live roofline (HBM traffic per launch, the traced kernel average and the profile's
  date), and they agree with the FLOP count the line uses: the fraction at the traced
  average lies in the range the kernel reaches.
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.cpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402  (no torch import at module level)


def test_multi_gpu_request_exits_with_message():
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert res.returncode == 2
    assert "single GPU" in res.stderr
    assert res.stdout == ""


def test_committed_profile_feeds_the_bench_line():
    prof = bench.load_profile(os.path.join(ROOT, "profiles", "flash_attn_peaked_cfg2.md"))
    assert set(prof) == {"traffic_bytes_per_launch", "kernel_avg_us", "profile_date"}
    # algorithmic bytes of the launch: peaked Q, new K and V once, the output
    assert 1.4e9 < prof["traffic_bytes_per_launch"] < 1.0e10
    flops = 4 * 1 * 40 * 512 * 64 * 36864 * 128            # the line's flops_per_launch
    frac = flops / (prof["kernel_avg_us"] * 1e-6) / 2.5e15
    assert 0.40 < frac < 0.60
    y, m, d = (int(x) for x in prof["profile_date"].split("-"))
    assert 2026 <= y and 1 <= m <= 12 and 1 <= d <= 31
