"""Selection of the fused attention implementation (mirrors reference ``models/fused_attn/loader.py:1-36``).

``EBR_FUSED_ATTN_IMPL``:
- ``auto`` (default), ``hip``: the gfx950 HIP library ``libebr_attn.so``. If it cannot be loaded the op raises
  ``RuntimeError`` naming the reason. Unlike the reference's ``auto``, there is no dense fallback: this build ships
  only the HIP kernels, so a missing library is an error, never a silent change of implementation.
- ``triton``: accepted as an alias of ``hip`` (the reference's "kernel or error" mode, which training scripts export).
- ``reference``: the reference forces its dense PyTorch path here; this build has none to force and raises
  ``RuntimeError``. Use the ``math`` attention backend for an eager path.
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
    """The loaded ``libebr_attn.so`` (ctypes), or RuntimeError when the selected mode cannot provide it."""
    m = mode()
    if m == "reference":
        raise RuntimeError(
            "EBR_FUSED_ATTN_IMPL=reference: this build ships no dense fused-attention fallback; "
            "select the 'math' attention backend for the eager path"
        )
    try:
        return _capi.load()
    except RuntimeError as exc:
        raise RuntimeError(f"EBR_FUSED_ATTN_IMPL={m}: the gfx950 fused attention library is unavailable: {exc}") from exc


def available() -> bool:
    try:
        hip_library()
        return True
    except (RuntimeError, ValueError):
        return False


__all__ = ["available", "hip_library", "mode"]
