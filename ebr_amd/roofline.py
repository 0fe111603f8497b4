"""MI355X peak constants and the algorithmic work of the three attention phases.

Work per (b, h) slice (FA2 convention: recomputed GEMMs counted, exp/elementwise excluded; s = element size):
    fwd      4 L^2 D flops   4 L D s + 4 L bytes   (read q, k, v; write o, lse)
    bwd     10 L^2 D flops   8 L D s + 4 L bytes   (read q, k, v, o, dO, lse; write dq, dk, dv)
    bwd_bwd 24 L^2 D flops  12 L D s + 4 L bytes   (read q, k, v, o, dO, gq, gk, gv, lse; write hq, hk, hv, hdO)
"""

from __future__ import annotations

PEAK_BF16_TFLOPS = 2516.6  # dense MFMA, 256 CU x 2.4 GHz x 4096 flop/clk/CU
PEAK_FP16_TFLOPS = 2516.6
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0

FLOP_COEF = {"fwd": 4, "bwd": 10, "bwd_bwd": 24}
TENSOR_IO = {"fwd": 4, "bwd": 8, "bwd_bwd": 12}


def phase_flops(phase: str, B: int, H: int, L: int, D: int) -> float:
    return float(FLOP_COEF[phase]) * L * L * D * B * H


def phase_bytes(phase: str, B: int, H: int, L: int, D: int, elem: int) -> float:
    return float(TENSOR_IO[phase] * L * D * elem + 4 * L) * B * H


def peak_tflops(dtype_name: str) -> float:
    return {"bf16": PEAK_BF16_TFLOPS, "fp16": PEAK_FP16_TFLOPS, "fp32": PEAK_FP32_TFLOPS}[dtype_name]


def roof_time_s(phase: str, B: int, H: int, L: int, D: int, elem: int, dtype_name: str) -> float:
    """max(flops / peak, bytes / HBM bandwidth) for one phase."""
    return max(
        phase_flops(phase, B, H, L, D) / (peak_tflops(dtype_name) * 1e12),
        phase_bytes(phase, B, H, L, D, elem) / (PEAK_HBM_GBS * 1e9),
    )


def bound(phase: str, B: int, H: int, L: int, D: int, elem: int, dtype_name: str) -> str:
    """'hbm' when the phase's bytes take longer at peak bandwidth than its flops at peak rate, else 'mfma'."""
    t_bytes = phase_bytes(phase, B, H, L, D, elem) / (PEAK_HBM_GBS * 1e9)
    t_flops = phase_flops(phase, B, H, L, D) / (peak_tflops(dtype_name) * 1e12)
    return "hbm" if t_bytes >= t_flops else "mfma"


__all__ = [
    "bound",
    "PEAK_BF16_TFLOPS",
    "PEAK_FP32_TFLOPS",
    "PEAK_HBM_GBS",
    "phase_bytes",
    "phase_flops",
    "peak_tflops",
    "roof_time_s",
]
