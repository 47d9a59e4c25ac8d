"""bench.py's host-side contract: window statistics and the one-GPU guard."""

from __future__ import annotations

import statistics
import subprocess
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_timing_stats_quartiles_match_numpy():
    xs = [0.21, 0.2, 0.205, 0.22, 0.199, 0.31, 0.202, 0.203]
    st = bench.timing_stats(xs)
    q1, q3, p10 = np.percentile(xs, [25, 75, 10])  # numpy's default is the same linear interpolation
    assert st["windows"] == len(xs)
    assert abs(st["q1_ms"] - q1) < 1e-5 and abs(st["q3_ms"] - q3) < 1e-5 and abs(st["p10_ms"] - p10) < 1e-5
    assert abs(st["median_ms"] - statistics.median(xs)) < 1e-5
    assert abs(st["iqr_ms"] - (q3 - q1)) < 1e-5
    assert st["tukey_outliers"] == 1  # 0.31 lies beyond q3 + 1.5 IQR


def test_timing_stats_constant_windows_have_no_outliers():
    st = bench.timing_stats([1.0] * 5)
    assert st["iqr_ms"] == 0 and st["tukey_outliers"] == 0 and st["median_ms"] == 1.0


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one MI355X" in r.stderr
    assert r.stdout == ""
