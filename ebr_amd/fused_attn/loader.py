"""Selection of the fused attention implementation (the reference's ``models/fused_attn/loader.py:1-36`` contract).

``EBR_FUSED_ATTN_IMPL``:
- ``auto`` (default) and ``hip``: GPU tensors run the gfx950 HIP library ``libebr_attn.so``; tensors off the GPU run
  the dense torch functions. If the library cannot be loaded, a GPU call raises ``RuntimeError`` naming the reason.
  The reference's ``auto`` would fall back to its dense functions on the GPU instead; here a GPU caller never gets
  another implementation than the one it asked for without being told.
- ``triton``: the reference's "kernels or an error" mode, which its training scripts export
  (``scripts/train.sh:15``); here the same as ``hip``.
- ``reference``: the dense torch functions for every tensor, on the GPU too (the reference's forced dense path).
"""

from __future__ import annotations

import os

from ebr_amd import _capi

_MODES = ("auto", "hip", "triton", "reference")


def mode() -> str:
    m = os.environ.get("EBR_FUSED_ATTN_IMPL", "auto").lower()
    if m not in _MODES:
        raise ValueError(f"EBR_FUSED_ATTN_IMPL must be one of {_MODES}, got {m!r}")
    return m


def hip_library():
    """The loaded ``libebr_attn.so`` (ctypes), or RuntimeError naming why it cannot be loaded."""
    try:
        return _capi.load()
    except RuntimeError as exc:
        raise RuntimeError(
            f"EBR_FUSED_ATTN_IMPL={mode()}: the gfx950 fused attention library is unavailable: {exc}"
        ) from exc


def available() -> bool:
    """Whether the HIP library loads (it does not say whether a GPU is present)."""
    try:
        hip_library()
        return True
    except (RuntimeError, ValueError):
        return False


__all__ = ["available", "hip_library", "mode"]
