"""Layers of the energy network (the attention path's callers): fp32-weight linear layers cast at use, rms_norm,
SwiGLU and 2D rotary position embeddings.

Behaviour follows reference ``models/layers.py``: ``trunc_normal_init_`` (:16-34, truncated normal rescaled to the
requested std), ``rms_norm`` (:37-42, fp32 statistics, input dtype out), ``CastedLinear`` (:45-57, fp32 weights with
std 1/sqrt(fan_in), cast to the input dtype), ``SwiGLU`` (:74-84, intermediate round(2/3 * expansion * hidden) rounded
up to a multiple of 256) and the broadcast 2D RoPE (:93-143: first half of each head rotates with the cell's row,
second half with its column). ``quarter_swap``, ``RotaryTable2D`` and ``RopeFused`` (:143-172) give the same rotation as
full [N, D] tables for the fused RoPE split (``ebr_amd.fused_attn.rope_split``).
"""

from __future__ import annotations

import math
from typing import NamedTuple

import torch
import torch.nn.functional as F
from torch import nn

RMS_NORM_EPS = 1e-5
ROPE_THETA = 10000.0


def trunc_normal_init_(tensor: torch.Tensor, std: float = 1.0, lower: float = -2.0, upper: float = 2.0) -> torch.Tensor:
    """In place: normal truncated to [lower, upper] standard units, scaled so the truncated law has std ``std``."""
    with torch.no_grad():
        if std == 0:
            return tensor.zero_()
        # Inverse-CDF sampling of the truncated standard normal, then a variance correction for the truncation.
        cdf_lo = 0.5 * (1.0 + math.erf(lower / math.sqrt(2.0)))
        cdf_hi = 0.5 * (1.0 + math.erf(upper / math.sqrt(2.0)))
        phi = lambda x: math.exp(-0.5 * x * x) / math.sqrt(2.0 * math.pi)  # noqa: E731
        mass = cdf_hi - cdf_lo
        var = 1.0 + (lower * phi(lower) - upper * phi(upper)) / mass - ((phi(lower) - phi(upper)) / mass) ** 2
        scale = std / math.sqrt(var)
        tensor.uniform_(2.0 * cdf_lo - 1.0, 2.0 * cdf_hi - 1.0)
        tensor.erfinv_().mul_(math.sqrt(2.0) * scale)
        return tensor.clamp_(lower * scale, upper * scale)


def rms_norm(x: torch.Tensor, variance_epsilon: float) -> torch.Tensor:
    """Unit RMS over the last dim, statistics in fp32, result in the input dtype."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + variance_epsilon)).to(x.dtype)


class CastedLinear(nn.Module):
    """y = x W^T (+ b) with fp32 parameters cast to x.dtype at every call. ``impl="splitk"`` takes the weight
    gradients as split-K GEMMs with fp32 partials (``ebr_amd.linear``); the values are those of ``F.linear``."""

    def __init__(self, in_features: int, out_features: int, bias: bool, impl: str = "eager") -> None:
        super().__init__()
        w = torch.empty(out_features, in_features)
        self.weight = nn.Parameter(trunc_normal_init_(w, std=in_features**-0.5))
        self.bias = nn.Parameter(torch.zeros(out_features)) if bias else None
        self.impl = check_linear_impl(impl)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        b = None if self.bias is None else self.bias.to(x.dtype)
        if self.impl == "splitk":
            from ebr_amd import linear

            return linear.linear(x, self.weight.to(x.dtype), b)
        return F.linear(x, self.weight.to(x.dtype), b)


def check_linear_impl(impl: str) -> str:
    if impl not in ("eager", "splitk"):
        raise ValueError(f"linear impl must be 'eager' or 'splitk', got {impl!r}")
    return impl


def swiglu_intermediate(hidden_size: int, expansion: float) -> int:
    n = round(expansion * hidden_size * 2 / 3)
    return ((n + 255) // 256) * 256


class SwiGLU(nn.Module):
    """down(silu(gate) * up) with gate, up the halves of one projection; ``impl="fused"`` runs the activation (and its
    first and second derivatives) as one HIP kernel each (``ebr_amd.block.swiglu``)."""

    def __init__(self, hidden_size: int, expansion: float, impl: str = "eager") -> None:
        super().__init__()
        if impl not in ("eager", "fused"):
            raise ValueError(f"SwiGLU impl must be 'eager' or 'fused', got {impl!r}")
        inter = swiglu_intermediate(hidden_size, expansion)
        self.gate_up_proj = CastedLinear(hidden_size, 2 * inter, bias=False)
        self.down_proj = CastedLinear(inter, hidden_size, bias=False)
        self.impl = impl

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.impl == "fused":
            from ebr_amd import block

            return self.down_proj(block.swiglu(self.gate_up_proj(x)))
        gate, up = self.gate_up_proj(x).chunk(2, dim=-1)
        return self.down_proj(F.silu(gate) * up)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


class RotaryEmbedding2D(nn.Module):
    """cos/sin tables for a ``height x width`` board: rows for the first half of D, columns for the second."""

    def __init__(self, dim: int, height: int, width: int, base: float = ROPE_THETA) -> None:
        super().__init__()
        half = dim // 2
        inv = 1.0 / (base ** (torch.arange(0, half, 2, dtype=torch.float32) / half))  # as reference layers.py:103
        ang_h = torch.arange(height, dtype=torch.float32)[:, None] * inv[None, :]
        ang_w = torch.arange(width, dtype=torch.float32)[:, None] * inv[None, :]
        ang_h, ang_w = ang_h.repeat(1, 2), ang_w.repeat(1, 2)
        self.register_buffer("cos_h", ang_h.cos(), persistent=False)
        self.register_buffer("sin_h", ang_h.sin(), persistent=False)
        self.register_buffer("cos_w", ang_w.cos(), persistent=False)
        self.register_buffer("sin_w", ang_w.sin(), persistent=False)

    def forward(self):
        return (self.cos_h, self.cos_w), (self.sin_h, self.sin_w)


def apply_rope(cos_sin, q: torch.Tensor, k: torch.Tensor):
    """2D RoPE on q, k of shape [B, N, heads, D] with N = height * width (row-major cells)."""
    (cos_h, cos_w), (sin_h, sin_w) = cos_sin
    hgt, wid = cos_h.shape[0], cos_w.shape[0]

    def rot(x: torch.Tensor) -> torch.Tensor:
        b, n, nh, d = x.shape
        xg = x.reshape(b, hgt, wid, nh, d).to(cos_h.dtype)
        r, c = xg[..., : d // 2], xg[..., d // 2 :]
        r = r * cos_h[None, :, None, None, :] + rotate_half(r) * sin_h[None, :, None, None, :]
        c = c * cos_w[None, None, :, None, :] + rotate_half(c) * sin_w[None, None, :, None, :]
        return torch.cat((r, c), dim=-1).to(x.dtype).reshape(b, n, nh, d)

    return rot(q), rot(k)


class RopeFused(NamedTuple):
    """Tables of the fused RoPE split (``rope_impl = "fused"``): fp32 [N, D] cos and signed sin."""

    cos: torch.Tensor
    sin: torch.Tensor


def quarter_swap(x: torch.Tensor) -> torch.Tensor:
    """The quarters (a, b, c, d) of the last dim as (b, a, d, c): rotate_half of each half without its sign."""
    shape = x.shape
    return x.reshape(*shape[:-1], 2, 2, shape[-1] // 4).flip(-2).reshape(shape)


class RotaryTable2D(nn.Module):
    """``RotaryEmbedding2D`` as full [height * width, D] tables: cell i * width + j has its row i angles in the first
    half of D and its column j angles in the second, and rotate_half's sign is folded into sin, so the rotation is
    ``x * cos + quarter_swap(x) * sin``."""

    def __init__(self, dim: int, height: int, width: int, base: float = ROPE_THETA) -> None:
        super().__init__()
        if dim % 4:
            raise ValueError(f"the fused RoPE split needs head_dim divisible by 4, got {dim}")
        (cos_h, cos_w), (sin_h, sin_w) = RotaryEmbedding2D(dim, height, width, base)()
        rows = torch.arange(height).repeat_interleave(width)
        cols = torch.arange(width).repeat(height)
        sign = torch.ones(dim)
        sign[: dim // 4] = -1.0
        sign[dim // 2 : dim // 2 + dim // 4] = -1.0
        self.register_buffer("cos_table", torch.cat((cos_h[rows], cos_w[cols]), dim=-1).float(), persistent=False)
        self.register_buffer(
            "sin_table", (torch.cat((sin_h[rows], sin_w[cols]), dim=-1) * sign).float(), persistent=False
        )

    def forward(self) -> RopeFused:
        return RopeFused(self.cos_table, self.sin_table)


__all__ = [
    "RMS_NORM_EPS",
    "CastedLinear",
    "RopeFused",
    "RotaryEmbedding2D",
    "RotaryTable2D",
    "quarter_swap",
    "SwiGLU",
    "apply_rope",
    "check_linear_impl",
    "rms_norm",
    "rotate_half",
    "swiglu_intermediate",
    "trunc_normal_init_",
]
