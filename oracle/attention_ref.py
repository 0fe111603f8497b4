"""Dense CPU restatement of the reference's eager attention path (test infrastructure only).

Follows, in the build's own code:
- ``models/fused_attn/reference.py:10-29``  dtype rules (fp32 compute, fp64 stays fp64; lse in the compute dtype),
  ``default_scale`` = D**-0.5, P recomputed from Q, K and the stored lse.
- ``models/fused_attn/reference.py:32-36``  attn_fwd: O = softmax(s Q K^T) V, natural-log row logsumexp.
- ``models/fused_attn/reference.py:39-58``  attn_bwd: Dr = rowsum(dO * O) from the STORED O, dS = P (dP - Dr).
- ``models/fused_attn/reference.py:61-91``  attn_bwd_bwd: the total derivative of <gQ,dQ> + <gK,dK> + <gV,dV>
  with respect to (Q, K, V, dO); ``dq`` is accepted and not read.
- ``models/attention.py:49-54``             math_attention: half types get an fp32 softmax, scale after the matmul.
- ``models/attention.py:156-161``           the max-abs-relative error metric ``rel``.
- ``models/fused_attn/ops.py:131-151``      which inputs get a second-order gradient (o and lse get none).

The bwd_bwd algebra is written in the S/P/dS/A/Bm/E/T notation (A = s(gQ K^T + Q gK^T), Bm = dO gV^T,
E = rowsum(P*A), T = rowsum(dS*A + P*Bm), dS2 = dS*A + P*Bm - E dS - T P, Pa = P*A - E P); it is equal to the
reference's ``gp``/``gs`` form (softmax Jacobian applied to the P-gradient), which ``tests/test_oracle.py`` checks
against torch autograd rather than against this file's own formulas.

Every function works on [B, H, L, D] tensors and can process the (b, h) slices in chunks (``chunk``) so that the
L x L temporaries of long sequences stay within host memory. Chunking changes no arithmetic: slices are independent.
"""

from __future__ import annotations

from typing import Callable, Optional, Sequence, Tuple

import torch

Tensor = torch.Tensor


# ---------------------------------------------------------------------------------------------------------------------
# dtype rules (reference.py:10-20)
# ---------------------------------------------------------------------------------------------------------------------


def compute_dtype(x: Tensor) -> torch.dtype:
    """fp64 stays fp64; everything else (fp32, bf16, fp16) computes in fp32."""
    return torch.float64 if x.dtype == torch.float64 else torch.float32


def default_scale(q: Tensor, scale: Optional[float] = None) -> float:
    return float(q.shape[-1] ** -0.5) if scale is None else float(scale)


def _chunked(fn: Callable[..., Tuple[Tensor, ...]], tensors: Sequence[Tensor], chunk: Optional[int]):
    """Apply ``fn`` to (b, h) slices of ``tensors`` (all shaped [B, H, ...]) ``chunk`` slices at a time."""
    B, H = tensors[0].shape[:2]
    if chunk is None or chunk >= B * H:
        return fn(*tensors)
    flat = [t.reshape(B * H, *t.shape[2:]) for t in tensors]
    outs = None
    for s in range(0, B * H, chunk):
        part = fn(*[t[s : s + chunk].unsqueeze(0) for t in flat])
        part = [p.squeeze(0) for p in part]
        if outs is None:
            outs = [torch.empty((B * H, *p.shape[1:]), dtype=p.dtype) for p in part]
        for o, p in zip(outs, part):
            o[s : s + chunk] = p
    return tuple(o.reshape(B, H, *o.shape[1:]) for o in outs)


def _scores(q: Tensor, k: Tensor, scale: float) -> Tensor:
    ct = compute_dtype(q)
    return torch.matmul(q.to(ct), k.to(ct).transpose(-1, -2)) * scale


# ---------------------------------------------------------------------------------------------------------------------
# The three ops (reference.py:32-91)
# ---------------------------------------------------------------------------------------------------------------------


def attn_fwd(q: Tensor, k: Tensor, v: Tensor, scale: float, chunk: Optional[int] = None) -> Tuple[Tensor, Tensor]:
    """(O, lse): O = softmax(s Q K^T) V in q.dtype, lse = natural-log row logsumexp in the compute dtype."""

    def run(q, k, v):
        ct = compute_dtype(q)
        s = _scores(q, k, scale)
        lse = torch.logsumexp(s, dim=-1)
        p = torch.exp(s - lse.unsqueeze(-1))
        o = torch.matmul(p, v.to(ct))
        return o.to(q.dtype), lse.to(ct)

    return _chunked(run, (q, k, v), chunk)


def _first_order(q, k, v, o, lse, do, scale):
    """P, dP, Dr and dS of one call; Dr uses the stored O (reference.py:44-45)."""
    ct = compute_dtype(q)
    s = _scores(q, k, scale)
    p = torch.exp(s - lse.to(ct).unsqueeze(-1))
    dof = do.to(ct)
    dp = torch.matmul(dof, v.to(ct).transpose(-1, -2))
    dr = (dof * o.to(ct)).sum(-1, keepdim=True)
    ds = p * (dp - dr)
    return p, dp, dr, ds


def attn_bwd(q, k, v, o, lse, do, scale: float, chunk: Optional[int] = None) -> Tuple[Tensor, Tensor, Tensor]:
    """(dQ, dK, dV) = gradient of <dO, O>, in the input dtype."""
    do = do.to(q.dtype)  # ops.py:84

    def run(q, k, v, o, lse, do):
        ct = compute_dtype(q)
        p, _, _, ds = _first_order(q, k, v, o, lse, do, scale)
        dq = torch.matmul(ds, k.to(ct)) * scale
        dk = torch.matmul(ds.transpose(-1, -2), q.to(ct)) * scale
        dv = torch.matmul(p.transpose(-1, -2), do.to(ct))
        return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype)

    return _chunked(run, (q, k, v, o, lse, do), chunk)


def attn_bwd_bwd(
    q, k, v, o, lse, do, dq, gq, gk, gv, scale: float, chunk: Optional[int] = None
) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """(hQ, hK, hV, hdO) = d/d(Q, K, V, dO) of <gQ, dQ> + <gK, dK> + <gV, dV>; ``dq`` is not read."""
    del dq

    def run(q, k, v, o, lse, do, gq, gk, gv):
        ct = compute_dtype(q)
        qf, kf, vf, dof = q.to(ct), k.to(ct), v.to(ct), do.to(ct)
        gqf, gkf, gvf = gq.to(ct), gk.to(ct), gv.to(ct)
        p, _, _, ds = _first_order(q, k, v, o, lse, do, scale)
        a = (torch.matmul(gqf, kf.transpose(-1, -2)) + torch.matmul(qf, gkf.transpose(-1, -2))) * scale
        bm = torch.matmul(dof, gvf.transpose(-1, -2))
        e = (p * a).sum(-1, keepdim=True)
        m1 = ds * a + p * bm
        t = m1.sum(-1, keepdim=True)
        ds2 = m1 - e * ds - t * p
        pa = p * a - e * p
        hq = (torch.matmul(ds2, kf) + torch.matmul(ds, gkf)) * scale
        hk = (torch.matmul(ds2.transpose(-1, -2), qf) + torch.matmul(ds.transpose(-1, -2), gqf)) * scale
        hv = torch.matmul(pa.transpose(-1, -2), dof)
        hdo = torch.matmul(pa, vf) + torch.matmul(p, gvf)
        return hq.to(q.dtype), hk.to(k.dtype), hv.to(v.dtype), hdo.to(do.dtype)

    do = do.to(q.dtype)
    return _chunked(run, (q, k, v, o, lse, do, gq.to(q.dtype), gk.to(q.dtype), gv.to(q.dtype)), chunk)


# ---------------------------------------------------------------------------------------------------------------------
# The eager path the fused ops replace (attention.py:49-54) and its autograd recipes
# ---------------------------------------------------------------------------------------------------------------------


def math_attention(q: Tensor, k: Tensor, v: Tensor) -> Tensor:
    """Plain softmax attention with scale D**-0.5 applied after the matmul; half types get an fp32 softmax."""
    out_dtype = q.dtype
    ct = torch.float32 if out_dtype in (torch.bfloat16, torch.float16) else out_dtype
    scores = torch.matmul(q.to(ct), k.to(ct).transpose(-1, -2)) * q.shape[-1] ** -0.5
    return torch.matmul(scores.softmax(dim=-1), v.to(ct)).to(out_dtype)


def autograd_bwd(q, k, v, do, attn: Callable[..., Tensor] = math_attention):
    """(dQ, dK, dV) of <dO, attn(q, k, v)> through torch autograd."""
    qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    out = attn(qq, kk, vv)
    return torch.autograd.grad(out, (qq, kk, vv), do.to(out.dtype))


def autograd_bwd_bwd(q, k, v, do, gq, gk, gv, attn: Callable[..., Tensor] = math_attention):
    """(hQ, hK, hV, hdO) through torch autograd: grad of sum(dQ*gQ + dK*gK + dV*gV) w.r.t. (q, k, v, dO), where
    dQ, dK, dV come from ``autograd.grad(..., create_graph=True)`` (the BASELINE config-0 recipe)."""
    qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    dd = do.detach().clone().to(q.dtype).requires_grad_(True)
    out = attn(qq, kk, vv)
    dq, dk, dv = torch.autograd.grad(out, (qq, kk, vv), dd, create_graph=True)
    phi = (dq * gq).sum() + (dk * gk).sum() + (dv * gv).sum()
    return torch.autograd.grad(phi, (qq, kk, vv, dd))


# ---------------------------------------------------------------------------------------------------------------------
# Inputs and the error metric
# ---------------------------------------------------------------------------------------------------------------------


def make_inputs(
    B: int, H: int, L: int, D: int, dtype: torch.dtype = torch.float32, seed: int = 0, qkv_scale: Optional[float] = None
):
    """Seeded inputs in the documented order: Q, K, V, dO, R1, R2, R3 ~ N(0, 1) from a CPU generator.

    ``qkv_scale`` multiplies Q, K and V (1/sqrt(64) = 0.125 for the bf16 BASELINE configs); all seven tensors are then
    cast to ``dtype``.
    """
    g = torch.Generator("cpu").manual_seed(seed)
    ts = [torch.randn((B, H, L, D), generator=g, dtype=torch.float32) for _ in range(7)]
    if qkv_scale is not None:
        for i in range(3):
            ts[i] = ts[i] * qkv_scale
    return tuple(t.to(dtype) for t in ts)


def rel_err(a: Tensor, ref: Tensor) -> float:
    """max|a - ref| / max|ref| (models/attention.py:156-161)."""
    a = a.detach().to("cpu", torch.float64)
    ref = ref.detach().to("cpu", torch.float64)
    return float((a - ref).abs().max() / ref.abs().max().clamp_min(1e-12))


__all__ = [
    "attn_bwd",
    "attn_bwd_bwd",
    "attn_fwd",
    "autograd_bwd",
    "autograd_bwd_bwd",
    "compute_dtype",
    "default_scale",
    "make_inputs",
    "math_attention",
    "rel_err",
]
