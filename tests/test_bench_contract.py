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


def test_every_ceiling_names_a_probe_of_its_kernels_pattern():
    # reads per write and bytes per stream of each dominant kernel (the roofline's launch)
    patterns = {
        "c1": (1, 4096 * 4096 * 4),  # x fp32 in, y out
        "c2": (2, 16384 * 14336 * 2),  # a, b bf16 in, y out
        "c3": (1, 8 * 4096 * 32 * 128 * 2),  # the q call, in place of q
        "c4": (2, 65536 * 8192 * 2),  # the backward: x, dy in, dx out
        "rope": (1, 4 * (32 + 8) * 4096 * 128 * 2),  # q and k in, their rotations out
        "qk_norm_rope": (2, 4 * (32 + 8) * 4096 * 128 * 2),  # q/k and cotangents in, gradients out
    }
    for name, probe in bench.CEILINGS.items():
        if name == "c5":
            assert probe == "mfma_ceiling_softmax"
            continue
        reads, mib = probe[len("stream_"):].split("_")
        assert (int(reads.rstrip("r")), int(mib.rstrip("m")) << 20) == patterns[name], name
