"""Fused second-order softmax attention on gfx950: ``fused_attention(q, k, v, scale=None)`` on [B, H, N, D] tensors
(drop-in for reference ``models/fused_attn/__init__.py``)."""

from ebr_amd.fused_attn.ops import fused_attention, implementation

__all__ = ["fused_attention", "implementation"]
