"""The bench line's fixed parts, checked without a GPU: metric name, peaks, and the one-GPU guard."""

import json
import subprocess
import sys
from pathlib import Path

import bench

ROOT = Path(__file__).resolve().parents[1]


def test_metric_is_the_baseline_metric():
    baseline = json.loads((ROOT / "BASELINE.json").read_text())
    assert bench.METRIC == baseline["metric"]


def test_peaks_are_mi355x_dense_figures():
    assert bench.HBM_PEAK_TBS == 8.0  # HBM3E
    assert bench.BF16_PEAK_TFLOPS == 2500.0  # dense bf16 MFMA, no sparsity


def test_more_than_one_gpu_is_refused_with_a_message():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr and proc.stdout == ""
