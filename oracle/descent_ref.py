"""CPU restatement of the latent-descent wrapper: the pointwise work around every descent microstep
``z -> sphere(rms_norm(z) + noise - alpha dE/dz)``.

TEST INFRASTRUCTURE ONLY (the checker of ``ebr_amd.descent``'s HIP kernels; never the implementation measured).

Forward functions restate the reference's eager formulas op by op, in the caller's dtype, so every rounding to the
tensor dtype happens where the reference's happens:
- ``rms_norm``               reference models/layers.py:37-42
- ``sphere``                 reference models/energy.py:219-222
- ``noisy_point``            reference models/energy.py:226-227 (and the eager branch :337-340)
- ``noisy_point_replayed``   reference models/energy.py:230-232 (and :335-336)
- ``step_and_project``       reference models/energy.py:235-241
The reference's backward is torch autograd through those formulas; ``vjp_noisy_point`` and ``vjp_step_and_project``
take it through the restatements. ``rms_norm_vjp`` and ``sphere_vjp`` are the closed forms of the two normalisations'
VJPs, used to pin autograd's in fp64.
"""

from __future__ import annotations

from typing import Optional, Union

import torch

RMS_NORM_EPS = 1e-5  # reference models/layers.py:12

Scalar = Union[float, torch.Tensor]


def rms_norm(x: torch.Tensor, eps: float = RMS_NORM_EPS) -> torch.Tensor:
    """Last-dim unit RMS computed in fp32 (fp64 stays fp64), returned in the input dtype."""
    dtype = x.dtype
    h = x.to(torch.promote_types(dtype, torch.float32))
    h = h * torch.rsqrt(h.square().mean(-1, keepdim=True) + eps)
    return h.to(dtype)


def sphere(z: torch.Tensor, eps: float = RMS_NORM_EPS) -> torch.Tensor:
    """Each row (dims 1 and 2, the whole board) rescaled to unit RMS, the RMS clamped below at ``eps``."""
    ct = torch.promote_types(z.dtype, torch.float32)
    rms = z.to(ct).square().mean(dim=(1, 2), keepdim=True).sqrt().clamp_min(eps)
    return (z.to(ct) / rms).to(z.dtype)


def noisy_point(z: torch.Tensor, noise: torch.Tensor, sigma: Scalar, eps: float = RMS_NORM_EPS) -> torch.Tensor:
    """rms_norm(z) + noise * sigma; a tensor ``sigma`` is [B, 1, 1] in z's dtype (the caller casts it)."""
    return rms_norm(z, eps) + noise * sigma


def noisy_point_replayed(z: torch.Tensor, noise: torch.Tensor, eps: float = RMS_NORM_EPS) -> torch.Tensor:
    v = rms_norm(z, eps)
    return v + noise.to(dtype=v.dtype)


def step_and_project(
    v: torch.Tensor, grad: torch.Tensor, alpha: Scalar, z: torch.Tensor, active: Optional[torch.Tensor],
    eps: float = RMS_NORM_EPS,
) -> torch.Tensor:
    """where(active, sphere(v - alpha * grad), z); ``alpha`` a float or a [B, 1, 1] tensor in v's dtype, ``active`` a
    [B, 1, 1] bool mask or None (every row moves)."""
    z_next = sphere(v - alpha * grad, eps)
    if active is not None:
        z_next = torch.where(active, z_next, z.to(dtype=z_next.dtype))
    return z_next


def vjp_noisy_point(z, noise, sigma, dv, eps: float = RMS_NORM_EPS) -> torch.Tensor:
    """dz of ``noisy_point`` (``sigma`` None: ``noisy_point_replayed``; ``noise`` None: plain rms_norm) by autograd."""
    x = z.detach().clone().requires_grad_(True)
    if noise is None:
        v = rms_norm(x, eps)
    elif sigma is None:
        v = noisy_point_replayed(x, noise, eps)
    else:
        v = noisy_point(x, noise, sigma, eps)
    (dz,) = torch.autograd.grad(v, x, dv)
    return dz


def vjp_step_and_project(v, grad, alpha, z, active, dout, eps: float = RMS_NORM_EPS):
    """(dv, dgrad, dz) of ``step_and_project`` by autograd; dz is None when ``active`` is None."""
    vv = v.detach().clone().requires_grad_(True)
    gg = grad.detach().clone().requires_grad_(True)
    zz = z.detach().clone().requires_grad_(True) if active is not None else z.detach()
    out = step_and_project(vv, gg, alpha, zz, active, eps)
    ins = (vv, gg, zz) if active is not None else (vv, gg)
    res = torch.autograd.grad(out, ins, dout, allow_unused=True)
    dz = res[2] if active is not None else None
    if dz is None and active is not None:
        dz = torch.zeros_like(z)
    return res[0], res[1], dz


def rms_norm_vjp(x: torch.Tensor, dy: torch.Tensor, eps: float = RMS_NORM_EPS) -> torch.Tensor:
    """Closed form: y = x r with r = (mean(x^2) + eps)^-1/2 gives dx = r dy - x r^3 mean(dy x) (fp64)."""
    x, dy = x.double(), dy.double()
    r = torch.rsqrt(x.square().mean(-1, keepdim=True) + eps)
    return r * dy - x * r**3 * (dy * x).mean(-1, keepdim=True)


def sphere_vjp(u: torch.Tensor, dy: torch.Tensor, eps: float = RMS_NORM_EPS) -> torch.Tensor:
    """Closed form: y = u / r with r = max(sqrt(mean(u^2)), eps) gives du = (dy - y mean(dy y)) / r where the clamp
    is inactive and dy / eps where it holds (fp64)."""
    u, dy = u.double(), dy.double()
    raw = u.square().mean(dim=(1, 2), keepdim=True).sqrt()
    r = raw.clamp_min(eps)
    y = u / r
    through = (dy - y * (dy * y).mean(dim=(1, 2), keepdim=True)) / r
    return torch.where(raw > eps, through, dy / eps)


def make_descent_inputs(B: int, L: int, C: int, dtype=torch.float32, seed: int = 0, device="cpu"):
    """z, noise, grad, per-row sigma and alpha [B, 1, 1] (fp32), a [B, 1, 1] mask with both values when B > 1."""
    g = torch.Generator().manual_seed(seed)
    z = (torch.randn(B, L, C, generator=g) * 1.7).to(dtype)
    noise = torch.randn(B, L, C, generator=g).to(dtype)
    grad = (torch.randn(B, L, C, generator=g) * 0.3).to(dtype)
    sigma = (0.05 + 0.2 * torch.rand(B, 1, 1, generator=g)).float()
    alpha = (0.05 + 0.1 * torch.rand(B, 1, 1, generator=g)).float()
    active = torch.rand(B, 1, 1, generator=g) < 0.6
    if B > 1:
        active[0], active[-1] = True, False
    return tuple(t.to(device) for t in (z, noise, grad, sigma, alpha, active))
