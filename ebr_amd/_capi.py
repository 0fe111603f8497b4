"""ctypes binding of ``libebr_attn.so`` (declared in ``include/ebr_attn.h``, ``include/ebr_rope.h``,
``include/ebr_descent.h`` and ``include/ebr_block.h``).

The library is built in-tree by ``ebr_amd.build`` into ``ebr_amd/_lib/``. Loading needs only the HIP runtime, so the
symbols can be checked on a machine without a GPU; every compute entry point needs a gfx950 device.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path
from typing import Optional

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libebr_attn.so"

DTYPE_F32, DTYPE_BF16, DTYPE_F16, DTYPE_F64 = 0, 1, 2, 3
OP_FWD, OP_BWD, OP_BWD_BWD = 0, 1, 2
ERR_HIP_BASE = 1000
ERR_NOALLOC_SIZE = 6
ERR_PLAN = 7
PLAN_AUTO, PLAN_GENERIC, PLAN_RESIDENT, PLAN_PERSISTENT, PLAN_LONG = 0, 1, 2, 3, 4  # EBR_PLAN_*
NOALLOC_SCRATCH_BYTES = 16 * 1024 * 1024  # EBR_NOALLOC_SCRATCH_BYTES
ABI_VERSION = 3

_P = ctypes.c_void_p
_I64P = ctypes.POINTER(ctypes.c_int64)
_F32P = ctypes.c_void_p  # fp32 device pointers are passed as raw addresses

# name -> (restype, argtypes); mirrors include/ebr_*.h
SIGNATURES = {
    "ebr_attn_fwd": (
        ctypes.c_int,
        [ctypes.c_int] * 5 + [ctypes.c_float] + [_P, _I64P] * 3 + [_P, _F32P, _P],
    ),
    "ebr_attn_bwd": (
        ctypes.c_int,
        [ctypes.c_int] * 5 + [ctypes.c_float] + [_P, _I64P] * 3 + [_P, _F32P] + [_P, _I64P] + [_P] * 3 + [_F32P, _P],
    ),
    "ebr_attn_bwd_bwd": (
        ctypes.c_int,
        [ctypes.c_int] * 5
        + [ctypes.c_float]
        + [_P, _I64P] * 3
        + [_P, _F32P]
        + [_P, _I64P] * 4
        + [_P] * 4
        + [_F32P, _P],
    ),
    "ebr_attn_fwd_plan": (
        ctypes.c_int,
        [ctypes.c_int] * 5 + [ctypes.c_float] + [_P, _I64P] * 3 + [_P, _F32P, _P, ctypes.c_int],
    ),
    "ebr_attn_bwd_plan": (
        ctypes.c_int,
        [ctypes.c_int] * 5
        + [ctypes.c_float]
        + [_P, _I64P] * 3
        + [_P, _F32P]
        + [_P, _I64P]
        + [_P] * 3
        + [_F32P, _P, ctypes.c_int],
    ),
    "ebr_attn_bwd_bwd_plan": (
        ctypes.c_int,
        [ctypes.c_int] * 5
        + [ctypes.c_float]
        + [_P, _I64P] * 3
        + [_P, _F32P]
        + [_P, _I64P] * 4
        + [_P] * 4
        + [_F32P, _P, ctypes.c_int],
    ),
    "ebr_attn_bwd_bwd_noalloc": (
        ctypes.c_int,
        [ctypes.c_int] * 5
        + [ctypes.c_float]
        + [_P, _I64P] * 3
        + [_P, _F32P]
        + [_P, _I64P] * 4
        + [_P] * 4
        + [_P],
    ),
    "ebr_attn_scratch_bytes": (ctypes.c_int64, [ctypes.c_int] * 5),
    # include/ebr_rope.h
    "ebr_rope_split": (
        ctypes.c_int,
        [ctypes.c_int] * 5 + [_P, ctypes.c_int64, ctypes.c_int64] + [_F32P] * 3 + [_P] * 3 + [_P],
    ),
    "ebr_rope_merge": (
        ctypes.c_int,
        [ctypes.c_int] * 5 + [_P, _I64P] * 3 + [_F32P] * 3 + [_P, _P],
    ),
    # include/ebr_descent.h
    "ebr_descent_noisy_point": (
        ctypes.c_int,
        [ctypes.c_int] * 4 + [ctypes.c_float] + [_P, _P, _F32P, _P, _P],
    ),
    "ebr_descent_noisy_point_bwd": (
        ctypes.c_int,
        [ctypes.c_int] * 4 + [ctypes.c_float] + [_P] * 4,
    ),
    "ebr_descent_step_project": (
        ctypes.c_int,
        [ctypes.c_int] * 2 + [ctypes.c_int64, ctypes.c_float] + [_P, _P, _F32P, _P, _P, _P, _F32P, _P],
    ),
    "ebr_descent_step_project_bwd": (
        ctypes.c_int,
        [ctypes.c_int] * 2 + [ctypes.c_int64, ctypes.c_float] + [_P, _P, _F32P, _P, _F32P, _P, _P, _P, _P, _P],
    ),
    # include/ebr_block.h
    "ebr_block_rmsnorm": (ctypes.c_int, [ctypes.c_int, ctypes.c_int64, ctypes.c_int, ctypes.c_float] + [_P] * 3),
    "ebr_block_rmsnorm_bwd": (ctypes.c_int, [ctypes.c_int, ctypes.c_int64, ctypes.c_int, ctypes.c_float] + [_P] * 4),
    "ebr_block_rmsnorm_bwd2": (ctypes.c_int, [ctypes.c_int, ctypes.c_int64, ctypes.c_int, ctypes.c_float] + [_P] * 6),
    "ebr_block_swiglu": (ctypes.c_int, [ctypes.c_int, ctypes.c_int64, ctypes.c_int] + [_P] * 3),
    "ebr_block_swiglu_bwd": (ctypes.c_int, [ctypes.c_int, ctypes.c_int64, ctypes.c_int] + [_P] * 4),
    "ebr_block_swiglu_bwd2": (ctypes.c_int, [ctypes.c_int, ctypes.c_int64, ctypes.c_int] + [_P] * 6),
    "ebr_attn_error_string": (ctypes.c_char_p, [ctypes.c_int]),
    "ebr_attn_abi_version": (ctypes.c_int, []),
    "ebr_attn_arch": (ctypes.c_char_p, []),
}

_LOCK = threading.Lock()
_LIB: Optional[ctypes.CDLL] = None
_ERROR: Optional[str] = None


def load(path: Optional[Path] = None) -> ctypes.CDLL:
    """Load the library once (raises RuntimeError with the reason when it cannot be loaded)."""
    global _LIB, _ERROR
    with _LOCK:
        if _LIB is not None and path is None:
            return _LIB
        p = Path(path) if path is not None else LIB_PATH
        try:
            if not p.exists():
                raise FileNotFoundError(f"{p} not built (run `python -m ebr_amd.build`)")
            lib = ctypes.CDLL(str(p))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            if lib.ebr_attn_abi_version() != ABI_VERSION:
                raise RuntimeError(f"ABI version {lib.ebr_attn_abi_version()} != expected {ABI_VERSION}")
        except Exception as exc:  # reported to the caller, never silently replaced
            if path is None:
                _ERROR = f"{type(exc).__name__}: {exc}"
            raise RuntimeError(f"cannot load {p}: {type(exc).__name__}: {exc}") from exc
        if path is None:
            _LIB, _ERROR = lib, None
        return lib


def load_error() -> Optional[str]:
    return _ERROR


def error_string(code: int) -> str:
    lib = load()
    return lib.ebr_attn_error_string(int(code)).decode()


def check(code: int, what: str) -> None:
    """Turn a non-zero return code into the exception the reference raises for the same condition."""
    if code == 0:
        return
    msg = f"{what}: {error_string(code)} (code {code})"
    if code == 1:
        raise TypeError(msg)
    if code in (2, ERR_PLAN):  # a forced plan that does not apply is a bad argument, as an unknown plan key is
        raise ValueError(msg)
    raise RuntimeError(msg)


def strides3(t) -> ctypes.Array:
    """Element strides of the B, H and L dimensions of a [B, H, L, D] tensor."""
    s = t.stride()
    return (ctypes.c_int64 * 3)(s[0], s[1], s[2])
