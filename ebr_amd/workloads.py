"""BASELINE workloads of the attention path and their seeded synthetic inputs.

Inputs follow the documented recipe: a CPU ``torch.Generator`` seeded with ``seed`` draws fp32 N(0, 1) tensors of shape
[B, H, L, D] in the order Q, K, V, dO, R1, R2, R3; Q, K and V are multiplied by ``qkv_scale`` (1/sqrt(64) for the bf16
configurations) and all seven are cast to the workload dtype. R1..R3 are the cotangents of dQ, dK, dV that the
backward of the backward receives.
"""

from __future__ import annotations

from typing import Optional

import torch

CONFIGS = {
    0: dict(name="nqueens8_attn_fp32", B=32, H=8, L=64, D=64, dtype=torch.float32, qkv_scale=None),
    1: dict(name="sudoku_attn_bf16", B=768, H=8, L=81, D=64, dtype=torch.bfloat16, qkv_scale=0.125),
    2: dict(name="maze_attn_bf16", B=64, H=8, L=900, D=64, dtype=torch.bfloat16, qkv_scale=0.125),
    # config 4's attention (5120 sequences of a 10 x 10 board, 8 heads of 64); its descent calls fwd and bwd only
    4: dict(name="config4_attn_bf16", B=5120, H=8, L=100, D=64, dtype=torch.bfloat16, qkv_scale=0.125),
}


def seeded_inputs(
    B: int, H: int, L: int, D: int, dtype: torch.dtype = torch.float32, seed: int = 0, qkv_scale: Optional[float] = None
):
    g = torch.Generator("cpu").manual_seed(seed)
    ts = [torch.randn((B, H, L, D), generator=g, dtype=torch.float32) for _ in range(7)]
    if qkv_scale is not None:
        for i in range(3):
            ts[i] = ts[i] * qkv_scale
    return tuple(t.to(dtype) for t in ts)


__all__ = ["CONFIGS", "seeded_inputs"]
