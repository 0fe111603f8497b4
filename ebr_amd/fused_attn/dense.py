"""Dense (materialised L x L) implementation of the three attention ops, in plain torch.

This is the path the ops take for tensors off the GPU and, on the GPU, only when ``EBR_FUSED_ATTN_IMPL=reference``
selects it explicitly (reference ``models/fused_attn/ops.py:65-121`` runs its dense functions on CPU tensors, and
``loader.py:21-23`` forces them with ``reference``). It is never chosen implicitly for a GPU tensor: there the HIP
kernels run or the call raises.

Semantics (reference ``models/fused_attn/reference.py:10-91``):
- arithmetic in fp32 for fp32 / bf16 / fp16 inputs and in fp64 for fp64 inputs; every output is rounded once to its
  input's dtype; lse is kept in that arithmetic dtype (fp32, or fp64 for fp64 inputs);
- the scores are the product Q K^T, then multiplied by ``scale``;
- the backward recomputes P from the given lse and takes rowsum(dO * O) from the given (stored) O;
- the backward of the backward does not read ``dq``.

The second-order outputs are written with the row statistics E = rowsum(P * A) and T = rowsum(dS * A + P * Bm),
where A = s (gQ K^T + Q gK^T) and Bm = dO gV^T: the score cotangent is dS2 = dS * (A - E) + P * (Bm - T) and the
value-side weight is Pa = P * (A - E). This is the softmax Jacobian applied to the cotangent of P, expanded.

Long sequences are processed a group of (b, h) slices at a time so that the L x L temporaries stay bounded; slices are
independent, so the grouping changes no value.
"""

from __future__ import annotations

from typing import Callable, Sequence, Tuple

import torch

Tensor = torch.Tensor

# Elements of one L x L fp32 temporary per group of slices (about 64 MB); several such temporaries are alive at once.
_GROUP_ELEMS = 1 << 24


def arithmetic_dtype(x: Tensor) -> torch.dtype:
    return torch.float64 if x.dtype == torch.float64 else torch.float32


def _per_group(fn: Callable[..., Tuple[Tensor, ...]], args: Sequence[Tensor], L: int) -> Tuple[Tensor, ...]:
    """Run ``fn`` over groups of (b, h) slices of ``args`` (each [B, H, ...]) and stitch the results together."""
    B, H = args[0].shape[:2]
    n = B * H
    per = max(1, _GROUP_ELEMS // max(1, L * L))
    if per >= n:
        return fn(*args)
    flat = [a.reshape(n, 1, *a.shape[2:]) for a in args]
    pieces = [fn(*(f[i : i + per] for f in flat)) for i in range(0, n, per)]
    return tuple(torch.cat(col, dim=0).reshape(B, H, *col[0].shape[2:]) for col in zip(*pieces))


class _Rows:
    """The per-call L x L quantities shared by the backward and the backward of the backward."""

    def __init__(self, q: Tensor, k: Tensor, v: Tensor, o: Tensor, lse: Tensor, do: Tensor, scale: float) -> None:
        at = arithmetic_dtype(q)
        self.at, self.scale = at, scale
        self.q, self.k, self.v, self.do = q.to(at), k.to(at), v.to(at), do.to(at)
        scores = torch.matmul(self.q, self.k.transpose(-1, -2)) * scale
        self.p = torch.exp(scores - lse.to(at)[..., None])
        self.dp = torch.matmul(self.do, self.v.transpose(-1, -2))
        dr = (self.do * o.to(at)).sum(dim=-1, keepdim=True)
        self.ds = self.p * (self.dp - dr)


def attn_fwd(q: Tensor, k: Tensor, v: Tensor, scale: float) -> Tuple[Tensor, Tensor]:
    def one(q, k, v):
        at = arithmetic_dtype(q)
        scores = torch.matmul(q.to(at), k.to(at).transpose(-1, -2)) * scale
        lse = torch.logsumexp(scores, dim=-1)
        o = torch.matmul(torch.exp(scores - lse[..., None]), v.to(at))
        return o.to(q.dtype), lse

    return _per_group(one, (q, k, v), q.shape[-2])


def attn_bwd(q: Tensor, k: Tensor, v: Tensor, o: Tensor, lse: Tensor, do: Tensor,
             scale: float) -> Tuple[Tensor, Tensor, Tensor]:
    def one(q, k, v, o, lse, do):
        r = _Rows(q, k, v, o, lse, do, scale)
        dq = torch.matmul(r.ds, r.k) * scale
        dk = torch.matmul(r.ds.transpose(-1, -2), r.q) * scale
        dv = torch.matmul(r.p.transpose(-1, -2), r.do)
        return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype)

    return _per_group(one, (q, k, v, o, lse, do), q.shape[-2])


def attn_bwd_bwd(q: Tensor, k: Tensor, v: Tensor, o: Tensor, lse: Tensor, do: Tensor, gq: Tensor, gk: Tensor,
                 gv: Tensor, scale: float) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    def one(q, k, v, o, lse, do, gq, gk, gv):
        r = _Rows(q, k, v, o, lse, do, scale)
        gqa, gka, gva = gq.to(r.at), gk.to(r.at), gv.to(r.at)
        a = (torch.matmul(gqa, r.k.transpose(-1, -2)) + torch.matmul(r.q, gka.transpose(-1, -2))) * scale
        bm = torch.matmul(r.do, gva.transpose(-1, -2))
        e = (r.p * a).sum(dim=-1, keepdim=True)
        t = (r.ds * a + r.p * bm).sum(dim=-1, keepdim=True)
        centred = a - e
        ds2 = r.ds * centred + r.p * (bm - t)
        pa = r.p * centred
        hq = (torch.matmul(ds2, r.k) + torch.matmul(r.ds, gka)) * scale
        hk = (torch.matmul(ds2.transpose(-1, -2), r.q) + torch.matmul(r.ds.transpose(-1, -2), gqa)) * scale
        hv = torch.matmul(pa.transpose(-1, -2), r.do)
        hdo = torch.matmul(pa, r.v) + torch.matmul(r.p, gva)
        return hq.to(q.dtype), hk.to(k.dtype), hv.to(v.dtype), hdo.to(do.dtype)

    return _per_group(one, (q, k, v, o, lse, do, gq, gk, gv), q.shape[-2])


__all__ = ["arithmetic_dtype", "attn_bwd", "attn_bwd_bwd", "attn_fwd"]
