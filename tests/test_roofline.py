"""CPU tests of the measurement arithmetic: the algorithmic work per phase (ebr_amd.roofline) against a count of the
dense closed forms' products and against the roofline table of the benchmark plan (configs 0-2), and bench.py's
one-GPU guard.

The counts: fwd S = Q K^T, O = P V (two L x L x D products); bwd recomputes S and adds dP = dO V^T, dV = P^T dO,
dQ = dS K, dK = dS^T Q (five); bwd_bwd S, A = gQ K^T + Q gK^T (two), dP, Bm = dO gV^T, and hQ (two), hK (two), hV,
hdO (two): twelve (reference models/fused_attn/reference.py:32-91). Each product is 2 L^2 D flops.
"""

import os
import subprocess
import sys

import pytest

from ebr_amd import roofline

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

PRODUCTS = {"fwd": 2, "bwd": 5, "bwd_bwd": 12}
# Tensors of [L, D] read or written per slice (lse, 4 bytes a row, counted apart): fwd q, k, v -> o; bwd q, k, v, o,
# dO -> dq, dk, dv; bwd_bwd q, k, v, o, dO, gq, gk, gv -> hq, hk, hv, hdO.
TENSORS = {"fwd": 3 + 1, "bwd": 5 + 3, "bwd_bwd": 8 + 4}


@pytest.mark.parametrize("phase", ["fwd", "bwd", "bwd_bwd"])
def test_phase_work_matches_product_count(phase):
    B, H, L, D = 3, 5, 37, 24
    assert roofline.phase_flops(phase, B, H, L, D) == PRODUCTS[phase] * 2 * L * L * D * B * H
    for elem in (2, 4, 8):
        assert roofline.phase_bytes(phase, B, H, L, D, elem) == (TENSORS[phase] * L * D * elem + 4 * L) * B * H


# (B, H, L, D, element bytes, dtype): GFLOP, MB and t_roof (us) over the three phases, as the benchmark plan's
# roofline table states them (configs 0, 1, 2).
TABLE = [
    ((32, 8, 64, 64, 4, "fp32"), 2.55, 100.9, 16.6),
    ((768, 8, 81, 64, 2, "bf16"), 98.04, 1534.8, 191.8),
    ((64, 8, 900, 64, 2, "bf16"), 1008.60, 1421.1, 400.8),
]


@pytest.mark.parametrize("shape,gflop,mb,t_us", TABLE)
def test_config_totals(shape, gflop, mb, t_us):
    B, H, L, D, elem, dt = shape
    phases = ("fwd", "bwd", "bwd_bwd")
    f = sum(roofline.phase_flops(p, B, H, L, D) for p in phases) / 1e9
    by = sum(roofline.phase_bytes(p, B, H, L, D, elem) for p in phases) / 1e6
    t = sum(roofline.roof_time_s(p, B, H, L, D, elem, dt) for p in phases) * 1e6
    assert f == pytest.approx(gflop, abs=0.01)
    assert by == pytest.approx(mb, abs=0.1)
    assert t == pytest.approx(t_us, abs=0.1)


def test_bounds():
    """Sudoku is memory-bound in every phase, Maze MFMA-bound in every phase."""
    for p in ("fwd", "bwd", "bwd_bwd"):
        assert roofline.bound(p, 768, 8, 81, 64, 2, "bf16") == "hbm"
        assert roofline.bound(p, 64, 8, 900, 64, 2, "bf16") == "mfma"


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""
