"""Custom ops and autograd wiring of the fused second-order attention (drop-in for reference
``models/fused_attn/ops.py``).

Ops (``torch.ops.ebr_fused.*``, functional, fresh contiguous outputs, same schemas as the reference):
- ``attn_fwd(q, k, v, scale) -> (o, lse)``                                      reference ops.py:65-77
- ``attn_bwd(q, k, v, o, lse, do, scale) -> (dq, dk, dv)``                      reference ops.py:80-95
- ``attn_bwd_bwd(q, k, v, o, lse, do, dq, gq, gk, gv, scale) -> (hq, hk, hv, hdo)``  reference ops.py:98-121
They are registered for the HIP device ("cuda" in PyTorch-ROCm) only and call the gfx950 kernels of
``libebr_attn.so`` on torch's current stream. A tensor on another device gets no kernel (the dispatcher raises).

Autograd (reference ops.py:124-190): ``_FusedAttn`` (fwd; backward = ``_FusedAttnBwd``) and ``_FusedAttnBwd`` (bwd;
backward = attn_bwd_bwd) with ``setup_context`` so ``torch.func.grad`` can differentiate them, and
``fused_attention`` kept one opaque dynamo node by ``allow_in_graph``.
"""

# No ``from __future__ import annotations``: custom_op schema inference needs real type objects.
from typing import Optional, Tuple, Union

import ctypes

import torch

from ebr_amd import _capi
from ebr_amd.fused_attn.loader import hip_library

Tensor = torch.Tensor

_DTYPE_CODE = {
    torch.float32: _capi.DTYPE_F32,
    torch.bfloat16: _capi.DTYPE_BF16,
    torch.float16: _capi.DTYPE_F16,
    torch.float64: _capi.DTYPE_F64,
}


def default_scale(q: Tensor, scale: Optional[float]) -> float:
    """D ** -0.5 unless given (reference models/fused_attn/reference.py:19-20)."""
    return float(q.shape[-1] ** -0.5) if scale is None else float(scale)


def lse_dtype_for(x: Tensor) -> torch.dtype:
    """lse is fp32; fp64 inputs keep fp64 (reference reference.py:14-16)."""
    return torch.float64 if x.dtype == torch.float64 else torch.float32


def implementation(device: Union[torch.device, str] = "cuda") -> str:
    """'hip' when the gfx950 kernels serve ``device``, else 'none' (reference ops.py:23-27 names its two)."""
    if torch.device(device).type != "cuda":
        return "none"
    try:
        hip_library()
        return "hip"
    except RuntimeError:
        return "none"


def _check(q: Tensor, k: Tensor, v: Tensor) -> None:
    """Shape/dtype contract of reference ops.py:51-57."""
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError(
            f"fused attention expects q, k, v of identical shape [B, H, N, D]; got {q.shape}, {k.shape}, {v.shape}"
        )
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError(f"fused attention expects one dtype; got {q.dtype}, {k.dtype}, {v.dtype}")
    if not (q.device == k.device == v.device):
        raise ValueError(f"fused attention expects one device; got {q.device}, {k.device}, {v.device}")


def _check_like(q: Tensor, **named: Tensor) -> None:
    """o, dO and the cotangents are read as [B, H, N, D] and lse as [B, H, N] by q's sizes (the C ABI takes only
    those), so a tensor of another shape or device is refused before any launch."""
    for name, t in named.items():
        want = q.shape[:-1] if name == "lse" else q.shape
        if t.shape != want or t.device != q.device:
            raise ValueError(f"fused attention: {name} is {tuple(t.shape)} on {t.device}, expected {tuple(want)} on "
                             f"{q.device}")


def _dtype_code(t: Tensor) -> int:
    code = _DTYPE_CODE.get(t.dtype)
    if code is None:
        raise TypeError(
            f"fused attention: unsupported dtype {t.dtype} (gfx950 kernels take float32, bfloat16, float16, float64)"
        )
    return code


def _align(t: Tensor) -> int:
    """Row-start alignment the kernels need: 16 bytes, or the element (8 bytes) for the fp64 kernels."""
    return 8 if t.dtype == torch.float64 else 16


def _rows(t: Tensor) -> Tensor:
    """Keep any B/H/L strides (views of a fused qkv projection, expanded zero rows) when every row start is aligned
    and D is unit-stride; otherwise copy (reference triton_kernels.py:598-601 keeps unit-D views)."""
    es, al = t.element_size(), _align(t)
    ok = t.stride(-1) == 1 and t.data_ptr() % al == 0
    ok = ok and all(s >= 0 and (s * es) % al == 0 for s in t.stride()[:3])
    return t if ok else t.contiguous()


def _contig(t: Tensor) -> Tensor:
    return t if t.is_contiguous() and t.data_ptr() % 16 == 0 else t.contiguous()


def _stream(t: Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _scratch(op: int, q: Tensor) -> Tuple[Optional[Tensor], int]:
    if q.dtype == torch.float64:  # the fp64 kernels need none
        return None, 0
    B, H, L, D = q.shape
    nbytes = int(hip_library().ebr_attn_scratch_bytes(op, B, H, L, D))
    if nbytes <= 0:
        return None, 0
    buf = torch.empty((nbytes + 3) // 4, device=q.device, dtype=torch.float32)
    return buf, buf.data_ptr()


# ----------------------------------------------------------------------------------------------------------------------
# Ops
# ----------------------------------------------------------------------------------------------------------------------


@torch.library.custom_op("ebr_fused::attn_fwd", mutates_args=(), device_types="cuda")
def attn_fwd(q: Tensor, k: Tensor, v: Tensor, scale: float) -> Tuple[Tensor, Tensor]:
    _check(q, k, v)
    lib = hip_library()
    code = _dtype_code(q)
    q, k, v = _rows(q), _rows(k), _rows(v)
    B, H, L, D = q.shape
    o = torch.empty((B, H, L, D), device=q.device, dtype=q.dtype)
    lse = torch.empty((B, H, L), device=q.device, dtype=lse_dtype_for(q))
    with torch.cuda.device(q.device):
        rc = lib.ebr_attn_fwd(
            code, B, H, L, D, ctypes.c_float(scale),
            q.data_ptr(), _capi.strides3(q), k.data_ptr(), _capi.strides3(k), v.data_ptr(), _capi.strides3(v),
            o.data_ptr(), lse.data_ptr(), _stream(q),
        )  # fmt: skip
    _capi.check(rc, "ebr_attn_fwd")
    return o, lse


@attn_fwd.register_fake
def _(q: Tensor, k: Tensor, v: Tensor, scale: float) -> Tuple[Tensor, Tensor]:
    o = torch.empty_like(q, memory_format=torch.contiguous_format)
    lse = q.new_empty(q.shape[:-1], dtype=lse_dtype_for(q))
    return o, lse


@torch.library.custom_op("ebr_fused::attn_bwd", mutates_args=(), device_types="cuda")
def attn_bwd(
    q: Tensor, k: Tensor, v: Tensor, o: Tensor, lse: Tensor, do: Tensor, scale: float
) -> Tuple[Tensor, Tensor, Tensor]:
    _check(q, k, v)
    _check_like(q, o=o, lse=lse, do=do)
    do = do.to(q.dtype)  # reference ops.py:84
    lib = hip_library()
    code = _dtype_code(q)
    q, k, v, do = _rows(q), _rows(k), _rows(v), _rows(do)
    o, lse = _contig(o.to(q.dtype)), _contig(lse.to(lse_dtype_for(q)))
    B, H, L, D = q.shape
    dq, dk, dv = (torch.empty((B, H, L, D), device=q.device, dtype=q.dtype) for _ in range(3))
    scratch, sp = _scratch(_capi.OP_BWD, q)
    with torch.cuda.device(q.device):
        rc = lib.ebr_attn_bwd(
            code, B, H, L, D, ctypes.c_float(scale),
            q.data_ptr(), _capi.strides3(q), k.data_ptr(), _capi.strides3(k), v.data_ptr(), _capi.strides3(v),
            o.data_ptr(), lse.data_ptr(), do.data_ptr(), _capi.strides3(do),
            dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), sp, _stream(q),
        )  # fmt: skip
    _capi.check(rc, "ebr_attn_bwd")
    del scratch  # the caching allocator keeps it valid for work already queued on this stream
    return dq, dk, dv


@attn_bwd.register_fake
def _(
    q: Tensor, k: Tensor, v: Tensor, o: Tensor, lse: Tensor, do: Tensor, scale: float
) -> Tuple[Tensor, Tensor, Tensor]:
    f = lambda x: torch.empty_like(x, memory_format=torch.contiguous_format)  # noqa: E731
    return f(q), f(k), f(v)


@torch.library.custom_op("ebr_fused::attn_bwd_bwd", mutates_args=(), device_types="cuda")
def attn_bwd_bwd(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    o: Tensor,
    lse: Tensor,
    do: Tensor,
    dq: Tensor,
    gq: Tensor,
    gk: Tensor,
    gv: Tensor,
    scale: float,
) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    del dq  # part of the op contract; the kernels recompute dS tile by tile (reference reference.py:74)
    _check(q, k, v)
    _check_like(q, o=o, lse=lse, do=do, gq=gq, gk=gk, gv=gv)
    lib = hip_library()
    code = _dtype_code(q)
    q, k, v = _rows(q), _rows(k), _rows(v)
    do = _rows(do.to(q.dtype))
    gq, gk, gv = _rows(gq.to(q.dtype)), _rows(gk.to(q.dtype)), _rows(gv.to(q.dtype))
    o, lse = _contig(o.to(q.dtype)), _contig(lse.to(lse_dtype_for(q)))
    B, H, L, D = q.shape
    hq, hk, hv, hdo = (torch.empty((B, H, L, D), device=q.device, dtype=q.dtype) for _ in range(4))
    scratch, sp = _scratch(_capi.OP_BWD_BWD, q)
    with torch.cuda.device(q.device):
        rc = lib.ebr_attn_bwd_bwd(
            code, B, H, L, D, ctypes.c_float(scale),
            q.data_ptr(), _capi.strides3(q), k.data_ptr(), _capi.strides3(k), v.data_ptr(), _capi.strides3(v),
            o.data_ptr(), lse.data_ptr(), do.data_ptr(), _capi.strides3(do),
            gq.data_ptr(), _capi.strides3(gq), gk.data_ptr(), _capi.strides3(gk), gv.data_ptr(), _capi.strides3(gv),
            hq.data_ptr(), hk.data_ptr(), hv.data_ptr(), hdo.data_ptr(), sp, _stream(q),
        )  # fmt: skip
    _capi.check(rc, "ebr_attn_bwd_bwd")
    del scratch
    return hq, hk, hv, hdo


@attn_bwd_bwd.register_fake
def _(q, k, v, o, lse, do, dq, gq, gk, gv, scale):
    f = lambda x: torch.empty_like(x, memory_format=torch.contiguous_format)  # noqa: E731
    return f(q), f(k), f(v), f(do)


# ----------------------------------------------------------------------------------------------------------------------
# Autograd: fwd -> bwd -> bwd_bwd (reference ops.py:124-185)
# ----------------------------------------------------------------------------------------------------------------------


def _zero_rows(like: Tensor) -> Tensor:
    """An all-zero cotangent as one zero row expanded to [B, H, L, D] (strides 0, 0, 0, 1): no L x D memory is written.
    The reference materialises ``zeros_like`` here (ops.py:147-149); the values are identical."""
    return torch.zeros((like.shape[-1],), device=like.device, dtype=like.dtype).expand(like.shape)


class _FusedAttnBwd(torch.autograd.Function):
    """(q, k, v, o, lse, do) -> (dq, dk, dv); its backward is attn_bwd_bwd."""

    @staticmethod
    def forward(q, k, v, o, lse, do, scale):
        return torch.ops.ebr_fused.attn_bwd(q, k, v, o, lse, do, scale)

    @staticmethod
    def setup_context(ctx, inputs, output):
        q, k, v, o, lse, do, scale = inputs
        ctx.save_for_backward(q, k, v, o, lse, do, output[0])
        ctx.scale = scale
        # Unused outputs arrive as None (not as materialised zero tensors) and become expanded zero rows below.
        ctx.set_materialize_grads(False)

    @staticmethod
    def backward(ctx, gq, gk, gv):
        q, k, v, o, lse, do, dq = ctx.saved_tensors
        gq = _zero_rows(q) if gq is None else gq.to(q.dtype)
        gk = _zero_rows(k) if gk is None else gk.to(k.dtype)
        gv = _zero_rows(v) if gv is None else gv.to(v.dtype)
        hq, hk, hv, hdo = torch.ops.ebr_fused.attn_bwd_bwd(q, k, v, o, lse, do, dq, gq, gk, gv, ctx.scale)
        return hq, hk, hv, None, None, hdo, None


class _FusedAttn(torch.autograd.Function):
    """(q, k, v) -> o; its backward is _FusedAttnBwd (itself differentiable)."""

    @staticmethod
    def forward(q, k, v, scale):
        o, lse = torch.ops.ebr_fused.attn_fwd(q, k, v, scale)
        return o, lse

    @staticmethod
    def setup_context(ctx, inputs, output):
        q, k, v, scale = inputs
        o, lse = output
        ctx.mark_non_differentiable(lse)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.scale = scale

    @staticmethod
    def backward(ctx, do, dlse):
        del dlse  # lse is marked non-differentiable
        q, k, v, o, lse = ctx.saved_tensors
        dq, dk, dv = _FusedAttnBwd.apply(q, k, v, o, lse, do, ctx.scale)
        return dq, dk, dv, None


def _fused_attention_apply(q: Tensor, k: Tensor, v: Tensor, scale: float) -> Tensor:
    o, _ = _FusedAttn.apply(q, k, v, scale)
    return o


# One opaque node for dynamo; AOTAutograd then traces the Functions, so compiled graphs hold the three custom ops.
_fused_attention_apply = torch._dynamo.allow_in_graph(_fused_attention_apply)


def fused_attention(q: Tensor, k: Tensor, v: Tensor, scale: Optional[float] = None) -> Tensor:
    """Non-causal softmax attention, ``[B, H, N, D]`` in and out, differentiable to second order."""
    return _fused_attention_apply(q, k, v, default_scale(q, scale))


__all__ = ["attn_bwd", "attn_bwd_bwd", "attn_fwd", "default_scale", "fused_attention", "implementation"]
