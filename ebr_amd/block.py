"""Fused pointwise work of the energy network's blocks on gfx950 (kernels ``ebr_amd/csrc/ebr_block.hip``, C ABI
``include/ebr_block.h``): ``rms_norm`` over the last dimension and the SwiGLU activation ``silu(gate) * up``, each
differentiable twice, as the graded latent descent needs (the energy's gradient is taken with ``create_graph`` and the
training loss differentiates it again).

- ``rms_norm(x, eps)``      reference models/layers.py:37-42
- ``swiglu(gate_up)``       reference models/layers.py:74-84 (``gate, up = gate_up.chunk(2, -1)``; ``silu(gate) * up``)

Ops (``torch.ops.ebr_fused.*``, HIP device only; a missing library raises): ``block_rmsnorm``, ``block_rmsnorm_bwd``,
``block_rmsnorm_bwd2``, ``block_swiglu``, ``block_swiglu_bwd``, ``block_swiglu_bwd2``. Autograd: each op's backward
is the next op, so the functions are differentiable to second order; the second backward is not itself
differentiable. The arithmetic is fp32 (fp64 for fp64 tensors), each output rounded once to the dtype where eager
autograd chains several rounded kernels, so 16-bit results differ from eager by rounding only.
"""

# No ``from __future__ import annotations``: custom_op schema inference needs real type objects.
from typing import Tuple

import torch
from torch.autograd.function import once_differentiable

from ebr_amd import _capi
from ebr_amd.fused_attn.loader import hip_library
from ebr_amd.fused_attn.ops import _DTYPE_CODE, _stream

Tensor = torch.Tensor


def _code(t: Tensor) -> int:
    code = _DTYPE_CODE.get(t.dtype)
    if code is None:
        raise TypeError(f"fused block: unsupported dtype {t.dtype}")
    return code


def _c(t: Tensor) -> Tensor:
    return t if t.is_contiguous() else t.contiguous()


def _rows(x: Tensor) -> Tuple[int, int]:
    if x.dim() < 1:
        raise ValueError(f"fused block: expected a tensor with a last dim, got {tuple(x.shape)}")
    return x.numel() // max(1, x.shape[-1]), x.shape[-1]


def _like(t: Tensor, shape, ref: Tensor, name: str) -> None:
    """An operand the kernels index by ``ref``'s rows (the C ABI takes only ``ref``'s sizes)."""
    if tuple(t.shape) != tuple(shape) or t.device != ref.device:
        raise ValueError(f"fused block: {name} is {tuple(t.shape)} on {t.device}, expected {tuple(shape)} on "
                         f"{ref.device}")


def _half(gu: Tensor) -> int:
    if gu.dim() < 1 or gu.shape[-1] % 2:
        raise ValueError(f"fused block: swiglu needs an even last dim, got {tuple(gu.shape)}")
    return gu.shape[-1] // 2


# ---------------------------------------------------------------------------------------------------------------------
# rms_norm
# ---------------------------------------------------------------------------------------------------------------------


@torch.library.custom_op("ebr_fused::block_rmsnorm", mutates_args=(), device_types="cuda")
def rmsnorm_op(x: Tensor, eps: float) -> Tensor:
    lib = hip_library()
    x = _c(x)
    rows, C = _rows(x)
    y = torch.empty_like(x)
    if y.numel() == 0:
        return y
    with torch.cuda.device(x.device):
        rc = lib.ebr_block_rmsnorm(_code(x), rows, C, eps, x.data_ptr(), y.data_ptr(), _stream(x))
    _capi.check(rc, "ebr_block_rmsnorm")
    return y


@rmsnorm_op.register_fake
def _(x, eps):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


@torch.library.custom_op("ebr_fused::block_rmsnorm_bwd", mutates_args=(), device_types="cuda")
def rmsnorm_bwd_op(x: Tensor, dy: Tensor, eps: float) -> Tensor:
    lib = hip_library()
    _like(dy, x.shape, x, "dy")
    x, dy = _c(x), _c(dy.to(x.dtype))
    rows, C = _rows(x)
    dx = torch.empty_like(x)
    if dx.numel() == 0:
        return dx
    with torch.cuda.device(x.device):
        rc = lib.ebr_block_rmsnorm_bwd(_code(x), rows, C, eps, x.data_ptr(), dy.data_ptr(), dx.data_ptr(), _stream(x))
    _capi.check(rc, "ebr_block_rmsnorm_bwd")
    return dx


@rmsnorm_bwd_op.register_fake
def _(x, dy, eps):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


@torch.library.custom_op("ebr_fused::block_rmsnorm_bwd2", mutates_args=(), device_types="cuda")
def rmsnorm_bwd2_op(x: Tensor, dy: Tensor, c: Tensor, eps: float) -> Tuple[Tensor, Tensor]:
    lib = hip_library()
    _like(dy, x.shape, x, "dy")
    _like(c, x.shape, x, "c")
    x, dy, c = _c(x), _c(dy.to(x.dtype)), _c(c.to(x.dtype))
    rows, C = _rows(x)
    gx, gdy = torch.empty_like(x), torch.empty_like(x)
    if gx.numel() == 0:
        return gx, gdy
    with torch.cuda.device(x.device):
        rc = lib.ebr_block_rmsnorm_bwd2(
            _code(x), rows, C, eps, x.data_ptr(), dy.data_ptr(), c.data_ptr(), gx.data_ptr(), gdy.data_ptr(),
            _stream(x),
        )  # fmt: skip
    _capi.check(rc, "ebr_block_rmsnorm_bwd2")
    return gx, gdy


@rmsnorm_bwd2_op.register_fake
def _(x, dy, c, eps):
    like = torch.empty_like(x, memory_format=torch.contiguous_format)
    return like, torch.empty_like(like)


class _RmsNormBwd(torch.autograd.Function):
    @staticmethod
    def forward(x, dy, eps):
        return torch.ops.ebr_fused.block_rmsnorm_bwd(x, dy, eps)

    @staticmethod
    def setup_context(ctx, inputs, output):
        x, dy, eps = inputs
        ctx.save_for_backward(x, dy)
        ctx.eps = eps

    @staticmethod
    @once_differentiable
    def backward(ctx, c):
        x, dy = ctx.saved_tensors
        gx, gdy = torch.ops.ebr_fused.block_rmsnorm_bwd2(x, dy, c, ctx.eps)
        return gx, gdy, None


class _RmsNorm(torch.autograd.Function):
    @staticmethod
    def forward(x, eps):
        return torch.ops.ebr_fused.block_rmsnorm(x, eps)

    @staticmethod
    def setup_context(ctx, inputs, output):
        x, eps = inputs
        ctx.save_for_backward(x)
        ctx.eps = eps

    @staticmethod
    def backward(ctx, dy):
        (x,) = ctx.saved_tensors
        return _RmsNormBwd.apply(x, dy, ctx.eps), None


# ---------------------------------------------------------------------------------------------------------------------
# SwiGLU
# ---------------------------------------------------------------------------------------------------------------------


@torch.library.custom_op("ebr_fused::block_swiglu", mutates_args=(), device_types="cuda")
def swiglu_op(gu: Tensor) -> Tensor:
    lib = hip_library()
    _half(gu)
    gu = _c(gu)
    rows, two_i = _rows(gu)
    y = gu.new_empty((*gu.shape[:-1], two_i // 2))
    if y.numel() == 0:
        return y
    with torch.cuda.device(gu.device):
        rc = lib.ebr_block_swiglu(_code(gu), rows, two_i // 2, gu.data_ptr(), y.data_ptr(), _stream(gu))
    _capi.check(rc, "ebr_block_swiglu")
    return y


@swiglu_op.register_fake
def _(gu):
    return gu.new_empty((*gu.shape[:-1], gu.shape[-1] // 2))


@torch.library.custom_op("ebr_fused::block_swiglu_bwd", mutates_args=(), device_types="cuda")
def swiglu_bwd_op(gu: Tensor, dy: Tensor) -> Tensor:
    lib = hip_library()
    _like(dy, (*gu.shape[:-1], _half(gu)), gu, "dy")
    gu, dy = _c(gu), _c(dy.to(gu.dtype))
    rows, two_i = _rows(gu)
    dgu = torch.empty_like(gu)
    if dgu.numel() == 0:
        return dgu
    with torch.cuda.device(gu.device):
        rc = lib.ebr_block_swiglu_bwd(_code(gu), rows, two_i // 2, gu.data_ptr(), dy.data_ptr(), dgu.data_ptr(),
                                      _stream(gu))
    _capi.check(rc, "ebr_block_swiglu_bwd")
    return dgu


@swiglu_bwd_op.register_fake
def _(gu, dy):
    return torch.empty_like(gu, memory_format=torch.contiguous_format)


@torch.library.custom_op("ebr_fused::block_swiglu_bwd2", mutates_args=(), device_types="cuda")
def swiglu_bwd2_op(gu: Tensor, dy: Tensor, c: Tensor) -> Tuple[Tensor, Tensor]:
    lib = hip_library()
    _like(dy, (*gu.shape[:-1], _half(gu)), gu, "dy")
    _like(c, gu.shape, gu, "c")
    gu, dy, c = _c(gu), _c(dy.to(gu.dtype)), _c(c.to(gu.dtype))
    rows, two_i = _rows(gu)
    ggu, gdy = torch.empty_like(gu), torch.empty_like(dy)
    if ggu.numel() == 0:
        return ggu, gdy
    with torch.cuda.device(gu.device):
        rc = lib.ebr_block_swiglu_bwd2(
            _code(gu), rows, two_i // 2, gu.data_ptr(), dy.data_ptr(), c.data_ptr(), ggu.data_ptr(), gdy.data_ptr(),
            _stream(gu),
        )  # fmt: skip
    _capi.check(rc, "ebr_block_swiglu_bwd2")
    return ggu, gdy


@swiglu_bwd2_op.register_fake
def _(gu, dy, c):
    return torch.empty_like(gu, memory_format=torch.contiguous_format), torch.empty_like(
        dy, memory_format=torch.contiguous_format
    )


class _SwiGLUBwd(torch.autograd.Function):
    @staticmethod
    def forward(gu, dy):
        return torch.ops.ebr_fused.block_swiglu_bwd(gu, dy)

    @staticmethod
    def setup_context(ctx, inputs, output):
        ctx.save_for_backward(*inputs)

    @staticmethod
    @once_differentiable
    def backward(ctx, c):
        gu, dy = ctx.saved_tensors
        return torch.ops.ebr_fused.block_swiglu_bwd2(gu, dy, c)


class _SwiGLU(torch.autograd.Function):
    @staticmethod
    def forward(gu):
        return torch.ops.ebr_fused.block_swiglu(gu)

    @staticmethod
    def setup_context(ctx, inputs, output):
        ctx.save_for_backward(inputs[0])

    @staticmethod
    def backward(ctx, dy):
        (gu,) = ctx.saved_tensors
        return _SwiGLUBwd.apply(gu, dy)


def rms_norm(x: Tensor, eps: float) -> Tensor:
    """Unit RMS over the last dim (statistics in fp32), differentiable twice."""
    return _RmsNorm.apply(x, eps)


def swiglu(gate_up: Tensor) -> Tensor:
    """silu(gate) * up of the two halves of the last dim, differentiable twice."""
    _half(gate_up)
    return _SwiGLU.apply(gate_up)


rms_norm = torch._dynamo.allow_in_graph(rms_norm)
swiglu = torch._dynamo.allow_in_graph(swiglu)

__all__ = ["rms_norm", "swiglu"]
