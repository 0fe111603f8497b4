"""Dense CPU restatement of the reference's fused 2D-RoPE split and merge (test infrastructure only).

Follows, in the build's own code:
- ``models/layers.py:143-146``               quarter_swap: the quarters (a, b, c, d) of the last dim -> (b, a, d, c).
- ``models/layers.py:81-104, 149-172``       the 2D rotary tables: head dims [0, D/2) rotate by the cell's row, [D/2, D)
  by its column, each half rotate_half-style (first half of the half pairs with the second); the fused table folds
  rotate_half's sign into sin, so that rotation = x * cos + quarter_swap(x) * sin.
- ``models/fused_attn/rope_split.py:32-50``  ref_split: [B, N, 3*H*D] -> rotated q, k and plain v, [B, H, N, D]
  contiguous; fp32 arithmetic (fp64 for fp64), rounded once to the dtype; optional per-head temperature applied to
  the rounded q and rounded again.
- ``models/fused_attn/rope_split.py:53-66``  ref_merge: the adjoint, [B, H, N, D] x 3 -> [B, N, 3*H*D]; the
  temperature's adjoint is applied (and rounded) first.

Pinning (``tests/test_rope_oracle.py``): the split equals the textbook broadcast 2D RoPE (rotate_half on each half,
``ebr_amd.layers.apply_rope``) on the full tables; the split preserves each rotated pair's norm; split and merge are
adjoint (<split(x), y> = <x, merge(y)> in fp64); the merge equals torch autograd's VJP of the split; the temperature
path equals the rounded two-step product.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

Tensor = torch.Tensor


def _ct(x: Tensor) -> torch.dtype:
    return torch.float64 if x.dtype == torch.float64 else torch.float32


def quarter_swap(x: Tensor) -> Tensor:
    """Swap the first two and the last two quarters of the last dim: (a, b, c, d) -> (b, a, d, c)."""
    d = x.shape[-1]
    q = d // 4
    return torch.cat([x[..., q : 2 * q], x[..., :q], x[..., 3 * q :], x[..., 2 * q : 3 * q]], dim=-1)


def rotary_tables(dim: int, height: int, width: int, base: float = 10000.0) -> Tuple[Tensor, Tensor]:
    """fp32 [height * width, dim] cos and signed sin of the fused 2D RoPE (cell i * width + j: row i in the first
    half of dim, column j in the second)."""
    half = dim // 2
    inv = 1.0 / (base ** (torch.arange(0, half, 2, dtype=torch.float32) / half))  # half / 2 frequencies
    ang_r = torch.arange(height, dtype=torch.float32)[:, None] * inv[None, :]
    ang_c = torch.arange(width, dtype=torch.float32)[:, None] * inv[None, :]
    rows = torch.arange(height).repeat_interleave(width)
    cols = torch.arange(width).repeat(height)
    ang = torch.cat([ang_r[rows], ang_r[rows], ang_c[cols], ang_c[cols]], dim=-1)  # [N, dim]
    sign = torch.ones(dim)
    sign[: dim // 4] = -1.0
    sign[half : half + dim // 4] = -1.0
    return ang.cos(), ang.sin() * sign


def ref_split(qkv: Tensor, cos: Tensor, sin: Tensor, heads: int,
              qscale: Optional[Tensor] = None) -> Tuple[Tensor, Tensor, Tensor]:
    b, n, c3 = qkv.shape
    d = c3 // (3 * heads)
    ct = _ct(qkv)
    x = qkv.reshape(b, n, 3, heads, d)
    c = cos.to(ct)[None, :, None, :]
    s = sin.to(ct)[None, :, None, :]

    def rot(t: Tensor) -> Tensor:
        t = t.to(ct)
        return (t * c + quarter_swap(t) * s).to(qkv.dtype)

    q, k, v = rot(x[:, :, 0]), rot(x[:, :, 1]), x[:, :, 2]
    if qscale is not None and qscale.numel() > 0:
        q = (q.to(ct) * qscale.to(ct).view(1, 1, -1, 1)).to(qkv.dtype)
    return tuple(t.transpose(1, 2).contiguous() for t in (q, k, v))


def ref_merge(dq: Tensor, dk: Tensor, dv: Tensor, cos: Tensor, sin: Tensor,
              qscale: Optional[Tensor] = None) -> Tensor:
    b, h, n, d = dq.shape
    ct = _ct(dq)
    c = cos.to(ct)[None, None]
    s = sin.to(ct)[None, None]

    def adj(g: Tensor) -> Tensor:
        g = g.to(ct)
        return (g * c + quarter_swap(g * s)).to(dq.dtype)

    if qscale is not None and qscale.numel() > 0:
        dq = (dq.to(ct) * qscale.to(ct).view(1, -1, 1, 1)).to(dq.dtype)
    out = torch.stack([adj(dq), adj(dk.to(dq.dtype)), dv.to(dq.dtype)], dim=2)  # [B, H, 3, N, D]
    return out.permute(0, 3, 2, 1, 4).reshape(b, n, 3 * h * d)


def make_rope_inputs(B: int, N: int, H: int, D: int, dtype: torch.dtype = torch.float32, seed: int = 0):
    """Seeded qkv [B, N, 3*H*D] and three cotangents [B, H, N, D] (CPU generator; fp32 N(0, 1) then cast)."""
    g = torch.Generator("cpu").manual_seed(seed)
    qkv = torch.randn((B, N, 3 * H * D), generator=g).to(dtype)
    gs = tuple(torch.randn((B, H, N, D), generator=g).to(dtype) for _ in range(3))
    return qkv, gs


def grid_shape(n: int) -> Tuple[int, int]:
    """A height x width board with height * width = n (the squarest one)."""
    h = int(math.isqrt(n))
    while n % h:
        h -= 1
    return h, n // h
