"""bench.py host logic that needs no GPU: the multi-GPU refusal and the per-config report."""
import subprocess
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402
from mamba_amd.configs import C2, C4  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_scan_report_c2_fractions():
    rep = bench.scan_report(C2, dict(ms=0.5, eager_ms=0.52, graph=True, fwd=0.1, bwd_scan=0.38, bwd_reduce=0.02,
                                     lens=None))
    assert rep["launch"] == "hip graph" and rep["ms_fwd_bwd_eager"] == 0.52
    assert rep["tokens_per_s"] == round(4 * 2048 / 0.5e-3, 1)
    assert rep["algorithmic_mb"] == {"fwd": 202.9, "bwd": 355.0}
    assert abs(rep["hbm_frac"]["fwd_bwd"] - 557.9e6 / 0.5e-3 / 8e12) < 1e-3


def test_scan_report_varlen_counts_valid_tokens():
    lens = np.random.default_rng(0).integers(512, 8193, size=16).astype(np.int32)
    rep = bench.scan_report(C4, dict(ms=10.0, eager_ms=10.1, graph=False, fwd=3.0, bwd_scan=6.5, bwd_reduce=0.5,
                                     lens=lens))
    assert rep["tokens_per_s"] == round(int(lens.sum()) / 10e-3, 1)
    assert rep["valid_fraction"] == round(lens.sum() / (16 * 8192), 4)
    assert rep["algorithmic_mb"]["fwd"] < 5388  # valid-token reads are fewer than the padded size
