"""Fused latent-descent wrapper on gfx950: the pointwise work around every descent microstep
``z -> sphere(rms_norm(z) + noise - alpha dE/dz)`` as HIP kernels (``ebr_amd/csrc/ebr_descent.hip``, C ABI
``include/ebr_descent.h``). Drop-in for the reference's ``descent_wrapper_compile`` functions, which it compiles with
inductor (reference models/energy.py:225-261):

- ``noisy_point(z, noise, sigma, eps)``          reference energy.py:226-227  rms_norm(z) + noise * sigma
- ``noisy_point_replayed(z, noise, eps)``        reference energy.py:230-232  rms_norm(z) + noise
- ``step_and_project(v, grad, alpha, z, active, eps)``  reference energy.py:235-241  where(active, sphere(v - alpha grad), z)
- ``normalize(z, eps)``                          reference energy.py:287-288  rms_norm(z) (no noise)

Argument meaning is the reference's: ``sigma`` / ``alpha`` a Python float or a per-row [B, 1, 1] tensor in the data
dtype (the reference's caller casts them, energy.py:313, 330); ``active`` a [B, 1, 1] bool mask or None. The values
are rounded where the eager formulas round them.

Ops (``torch.ops.ebr_fused.*``, fresh contiguous outputs, HIP device only; a missing library raises):
``descent_noisy_point``, ``descent_noisy_point_bwd``, ``descent_step_project``, ``descent_step_project_bwd``.
Autograd: first order (``alpha`` and ``sigma`` are schedule constants of the reference and get gradients only through
the plain torch formula below); the backward is not itself differentiable, like the reference's inductor graphs
taken once.
"""

# No ``from __future__ import annotations``: custom_op schema inference needs real type objects.
from typing import Optional, Tuple, Union

import torch
from torch.autograd.function import once_differentiable

from ebr_amd import _capi
from ebr_amd.fused_attn.loader import hip_library
from ebr_amd.fused_attn.ops import _dtype_code, _stream

Tensor = torch.Tensor
Scalar = Union[float, Tensor]

RMS_NORM_EPS = 1e-5  # reference models/layers.py:12


def _contig(t: Tensor) -> Tensor:
    return t if t.is_contiguous() else t.contiguous()


def _ptr(t: Optional[Tensor]) -> int:
    return 0 if t is None or t.numel() == 0 else t.data_ptr()


def _check_board(t: Tensor, name: str) -> None:
    if t.dim() != 3:
        raise ValueError(f"descent wrapper: {name} must be [B, L, C], got {tuple(t.shape)}")


def _per_row(x: Scalar, rows: int, dtype: torch.dtype, device, name: str) -> Tensor:
    """fp32 [rows] values of a per-row scalar: a float as given (torch multiplies a scalar at fp32), a tensor rounded
    through ``dtype`` (the reference's caller has cast it)."""
    if not isinstance(x, Tensor):
        return torch.full((rows,), float(x), device=device, dtype=torch.float32)
    if x.requires_grad and torch.is_grad_enabled():
        raise NotImplementedError(f"descent wrapper: {name} is a schedule constant here (no gradient)")
    if x.dtype != dtype:
        raise TypeError(f"descent wrapper: {name} has dtype {x.dtype}, expected {dtype} (cast it as the caller does)")
    if x.numel() not in (1, rows) or any(s != 1 for s in x.shape[1:]):
        raise ValueError(f"descent wrapper: {name} must be a scalar or [B, 1, 1] per row, got {tuple(x.shape)}")
    return x.reshape(-1).expand(rows).to(device=device, dtype=torch.float32).contiguous()


def _like(t: Tensor, ref: Tensor, name: str) -> None:
    """An operand the kernels index like ``ref`` (the C ABI takes only ``ref``'s sizes)."""
    if t.shape != ref.shape or t.device != ref.device:
        raise ValueError(f"descent wrapper: {name} is {tuple(t.shape)} on {t.device}, expected {tuple(ref.shape)} on "
                         f"{ref.device}")


def _row_vec(t: Tensor, rows: int, dtype: torch.dtype, ref: Tensor, name: str) -> Tensor:
    """A per-row operand of the ops: ``rows`` elements of ``dtype`` on ``ref``'s device."""
    if t.numel() != rows or t.dtype != dtype or t.device != ref.device:
        raise ValueError(f"descent wrapper: {name} must be {rows} {dtype} values on {ref.device}, got "
                         f"{tuple(t.shape)} {t.dtype} on {t.device}")
    return _contig(t.reshape(rows))


def _mask(active: Optional[Tensor], rows: int, device) -> Optional[Tensor]:
    if active is None:
        return None
    if active.numel() != rows or any(s != 1 for s in active.shape[1:]):
        raise ValueError(f"descent wrapper: active must be [B, 1, 1], got {tuple(active.shape)}")
    return active.reshape(rows).to(device=device, dtype=torch.uint8).contiguous()


# ---------------------------------------------------------------------------------------------------------------------
# Ops
# ---------------------------------------------------------------------------------------------------------------------


@torch.library.custom_op("ebr_fused::descent_noisy_point", mutates_args=(), device_types="cuda")
def noisy_point_op(z: Tensor, noise: Optional[Tensor], sigma: Optional[Tensor], eps: float) -> Tensor:
    """v = rms_norm(z) (+ noise) (+ round(noise * sigma[b])); ``sigma`` fp32 [B] or None."""
    lib = hip_library()
    code = _dtype_code(z)
    _check_board(z, "z")
    z = _contig(z)
    B, L, C = z.shape
    if noise is not None:
        _like(noise, z, "noise")
        noise = _contig(noise.to(z.dtype))
    if sigma is not None:
        sigma = _row_vec(sigma, B, torch.float32, z, "sigma")
    v = torch.empty_like(z)
    if v.numel() == 0:
        return v
    with torch.cuda.device(z.device):
        rc = lib.ebr_descent_noisy_point(code, B, L, C, eps, z.data_ptr(), _ptr(noise), _ptr(sigma), v.data_ptr(),
                                         _stream(z))
    _capi.check(rc, "ebr_descent_noisy_point")
    return v


@noisy_point_op.register_fake
def _(z, noise, sigma, eps):
    return torch.empty_like(z, memory_format=torch.contiguous_format)


@torch.library.custom_op("ebr_fused::descent_noisy_point_bwd", mutates_args=(), device_types="cuda")
def noisy_point_bwd_op(z: Tensor, dv: Tensor, eps: float) -> Tensor:
    lib = hip_library()
    code = _dtype_code(z)
    _check_board(z, "z")
    _like(dv, z, "dv")
    z, dv = _contig(z), _contig(dv.to(z.dtype))
    B, L, C = z.shape
    dz = torch.empty_like(z)
    if dz.numel() == 0:
        return dz
    with torch.cuda.device(z.device):
        rc = lib.ebr_descent_noisy_point_bwd(code, B, L, C, eps, z.data_ptr(), dv.data_ptr(), dz.data_ptr(), _stream(z))
    _capi.check(rc, "ebr_descent_noisy_point_bwd")
    return dz


@noisy_point_bwd_op.register_fake
def _(z, dv, eps):
    return torch.empty_like(z, memory_format=torch.contiguous_format)


@torch.library.custom_op("ebr_fused::descent_step_project", mutates_args=(), device_types="cuda")
def step_project_op(v: Tensor, g: Tensor, alpha: Tensor, z: Optional[Tensor], active: Optional[Tensor],
                    eps: float) -> Tuple[Tensor, Tensor]:
    """(where(active, sphere(v - round(alpha g)), z), rms [B] fp32); ``alpha`` fp32 [B], ``active`` uint8 [B]."""
    lib = hip_library()
    code = _dtype_code(v)
    _check_board(v, "v")
    _like(g, v, "g")
    v, g = _contig(v), _contig(g.to(v.dtype))
    B = v.shape[0]
    if v.numel() == 0:
        return torch.empty_like(v), v.new_zeros((B,), dtype=torch.float32)
    N = v.numel() // B
    alpha = _row_vec(alpha, B, torch.float32, v, "alpha")
    if active is not None:
        if z is None:
            raise ValueError("descent wrapper: a row mask needs z (the rows it keeps)")
        _like(z, v, "z")
        active = _row_vec(active, B, torch.uint8, v, "active")
        z = _contig(z.to(v.dtype))
    out = torch.empty_like(v)
    rms = torch.empty((B,), device=v.device, dtype=torch.float32)
    with torch.cuda.device(v.device):
        rc = lib.ebr_descent_step_project(
            code, B, N, eps, v.data_ptr(), g.data_ptr(), alpha.data_ptr(), _ptr(z) if active is not None else 0,
            _ptr(active), out.data_ptr(), rms.data_ptr(), _stream(v),
        )  # fmt: skip
    _capi.check(rc, "ebr_descent_step_project")
    return out, rms


@step_project_op.register_fake
def _(v, g, alpha, z, active, eps):
    return torch.empty_like(v, memory_format=torch.contiguous_format), v.new_empty((v.shape[0],), dtype=torch.float32)


@torch.library.custom_op("ebr_fused::descent_step_project_bwd", mutates_args=(), device_types="cuda")
def step_project_bwd_op(v: Tensor, g: Tensor, alpha: Tensor, active: Optional[Tensor], rms: Tensor, dout: Tensor,
                        eps: float) -> Tuple[Tensor, Tensor, Tensor]:
    """(dv, dg, dz); dz is an empty tensor when ``active`` is None (every row moves, so it would be zero)."""
    lib = hip_library()
    code = _dtype_code(v)
    _check_board(v, "v")
    _like(g, v, "g")
    _like(dout, v, "dout")
    v, g, dout = _contig(v), _contig(g.to(v.dtype)), _contig(dout.to(v.dtype))
    B = v.shape[0]
    if v.numel() == 0:
        dz = torch.empty_like(v) if active is not None else v.new_empty((0,))
        return torch.empty_like(v), torch.empty_like(v), dz
    N = v.numel() // B
    alpha = _row_vec(alpha, B, torch.float32, v, "alpha")
    rms = _row_vec(rms, B, torch.float32, v, "rms")
    if active is not None:
        active = _row_vec(active, B, torch.uint8, v, "active")
    dv, dg = torch.empty_like(v), torch.empty_like(v)
    dz = torch.empty_like(v) if active is not None else v.new_empty((0,))
    with torch.cuda.device(v.device):
        rc = lib.ebr_descent_step_project_bwd(
            code, B, N, eps, v.data_ptr(), g.data_ptr(), alpha.data_ptr(), _ptr(active), rms.data_ptr(),
            dout.data_ptr(), dv.data_ptr(), dg.data_ptr(), _ptr(dz), _stream(v),
        )  # fmt: skip
    _capi.check(rc, "ebr_descent_step_project_bwd")
    return dv, dg, dz


@step_project_bwd_op.register_fake
def _(v, g, alpha, active, rms, dout, eps):
    like = torch.empty_like(v, memory_format=torch.contiguous_format)
    dz = torch.empty_like(like) if active is not None else v.new_empty((0,))
    return like, torch.empty_like(like), dz


# ---------------------------------------------------------------------------------------------------------------------
# Autograd
# ---------------------------------------------------------------------------------------------------------------------


class _NoisyPoint(torch.autograd.Function):
    @staticmethod
    def forward(z, noise, sigma32, sigma, eps):
        return torch.ops.ebr_fused.descent_noisy_point(z, noise, sigma32, eps)

    @staticmethod
    def setup_context(ctx, inputs, output):
        z, noise, sigma32, sigma, eps = inputs
        ctx.save_for_backward(z, sigma if isinstance(sigma, Tensor) else None)
        ctx.sigma = None if isinstance(sigma, Tensor) else sigma
        ctx.scaled = sigma32 is not None
        ctx.eps = eps

    @staticmethod
    @once_differentiable
    def backward(ctx, dv):
        z, sigma_t = ctx.saved_tensors
        dz = torch.ops.ebr_fused.descent_noisy_point_bwd(z, dv, ctx.eps) if ctx.needs_input_grad[0] else None
        dnoise = None
        if ctx.needs_input_grad[1]:  # the reference's noise is drawn without grad; the plain formula if it has one
            sig = sigma_t if sigma_t is not None else ctx.sigma
            dnoise = dv * sig if ctx.scaled else dv
        return dz, dnoise, None, None, None


class _StepProject(torch.autograd.Function):
    @staticmethod
    def forward(v, g, alpha32, z, active8, eps):
        return torch.ops.ebr_fused.descent_step_project(v, g, alpha32, z, active8, eps)

    @staticmethod
    def setup_context(ctx, inputs, output):
        v, g, alpha32, z, active8, eps = inputs
        out, rms = output
        ctx.mark_non_differentiable(rms)
        ctx.eps = eps
        ctx.masked = active8 is not None
        ctx.save_for_backward(v, g, alpha32, active8, rms)

    @staticmethod
    @once_differentiable
    def backward(ctx, dout, _drms):
        v, g, alpha32, active8, rms = ctx.saved_tensors
        if dout is None:
            return None, None, None, None, None, None
        dv, dg, dz = torch.ops.ebr_fused.descent_step_project_bwd(v, g, alpha32, active8, rms, dout, ctx.eps)
        return dv, dg, None, (dz if ctx.masked else None), None, None


# ---------------------------------------------------------------------------------------------------------------------
# Reference-shaped entry points
# ---------------------------------------------------------------------------------------------------------------------


def normalize(z: Tensor, eps: float = RMS_NORM_EPS) -> Tensor:
    """rms_norm over the last dim (reference EnergyDescent.normalize_descent_state, energy.py:287-288)."""
    _check_board(z, "z")
    return _NoisyPoint.apply(z, None, None, None, eps)


def noisy_point(z: Tensor, noise: Tensor, sigma: Scalar, eps: float = RMS_NORM_EPS) -> Tensor:
    """rms_norm(z) + noise * sigma (reference energy.py:226-227)."""
    _check_board(z, "z")
    if noise.shape != z.shape:
        raise ValueError(f"descent wrapper: noise {tuple(noise.shape)} != z {tuple(z.shape)}")
    s32 = _per_row(sigma, z.shape[0], z.dtype, z.device, "sigma")
    return _NoisyPoint.apply(z, noise.to(device=z.device, dtype=z.dtype), s32, sigma, eps)


def noisy_point_replayed(z: Tensor, noise: Tensor, eps: float = RMS_NORM_EPS) -> Tensor:
    """rms_norm(z) + noise (reference energy.py:230-232)."""
    _check_board(z, "z")
    if noise.shape != z.shape:
        raise ValueError(f"descent wrapper: noise {tuple(noise.shape)} != z {tuple(z.shape)}")
    return _NoisyPoint.apply(z, noise.to(device=z.device, dtype=z.dtype), None, None, eps)


def step_and_project(v: Tensor, grad: Tensor, alpha: Scalar, z: Tensor, active: Optional[Tensor],
                     eps: float = RMS_NORM_EPS) -> Tensor:
    """where(active, sphere(v - alpha * grad), z) (reference energy.py:235-241)."""
    _check_board(v, "v")
    if grad.shape != v.shape or z.shape != v.shape:
        raise ValueError(f"descent wrapper: grad {tuple(grad.shape)} / z {tuple(z.shape)} != v {tuple(v.shape)}")
    B = v.shape[0]
    a32 = _per_row(alpha, B, v.dtype, v.device, "alpha")
    act = _mask(active, B, v.device)
    out, _ = _StepProject.apply(v, grad, a32, z if act is not None else None, act, eps)
    return out


noisy_point = torch._dynamo.allow_in_graph(noisy_point)
noisy_point_replayed = torch._dynamo.allow_in_graph(noisy_point_replayed)
step_and_project = torch._dynamo.allow_in_graph(step_and_project)
normalize = torch._dynamo.allow_in_graph(normalize)

__all__ = ["RMS_NORM_EPS", "noisy_point", "noisy_point_replayed", "normalize", "step_and_project"]
