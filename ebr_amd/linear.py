"""Linear layers of the energy network with their weight gradients taken as split-K GEMMs.

The energy network's projections (reference ``CastedLinear``, models/layers.py:45-57) see M = batch x tokens rows
(31,104 at the training shape) against 512 to 3,072 features. Their weight gradient ``dW = dY^T X`` reduces over
those M rows into a small [N, K] output, a shape the library's single-GEMM heuristics serve poorly (a few dozen
output tiles for 256 CUs): at the training shape it takes 120-200 us, against 40-125 us as S = 8 or 16 batched
partial products over M / S rows each, accumulated and returned in fp32 (``torch.bmm(..., out_dtype=float32)``),
then summed in fp32 and rounded once to the dtype. The result differs from the single GEMM only in the order of its
fp32 sums.

``linear(x, w)`` is ``F.linear(x, w)`` with that weight gradient, and with the input gradient ``dX = dY W`` as an
autograd Function of its own, whose weight gradient (``dY^T G`` for the cotangent G of dX, needed when training
differentiates a descent step's dE/dz) is split-K as well. Gradients the autograd engine will not use are not
computed (``torch._C._will_engine_execute_node``), as for torch's own linear: the descent's ``autograd.grad(E, z)``
asks for input gradients only. Under ``create_graph`` the weight gradients are taken with differentiable torch ops,
so higher-order derivatives stay exact.
"""

from typing import Optional

import torch
import torch.nn.functional as F

Tensor = torch.Tensor

SPLITS = (16, 8, 4, 2)
MIN_ROWS_PER_SPLIT = 1024
SPLIT8_OUTPUT = 1_500_000  # outputs of at least this many elements have tiles enough for 8 splits


def _splits(m: int, outputs: int) -> int:
    first = 8 if outputs >= SPLIT8_OUTPUT else 16
    for s in SPLITS:
        if s <= first and m % s == 0 and m // s >= MIN_ROWS_PER_SPLIT:
            return s
    return 1


def weight_grad(a: Tensor, b: Tensor) -> Tensor:
    """a^T b over the flattened leading dims: a [..., N], b [..., K] -> [N, K] in a's dtype, fp32 accumulation."""
    a2, b2 = a.reshape(-1, a.shape[-1]), b.reshape(-1, b.shape[-1])
    if torch.is_grad_enabled() and (a2.requires_grad or b2.requires_grad):
        return a2.t() @ b2  # recorded for higher-order derivatives
    m, n, k = a2.shape[0], a2.shape[1], b2.shape[1]
    s = _splits(m, n * k) if a2.is_cuda and a2.dtype in (torch.bfloat16, torch.float16) else 1
    if s == 1:
        return a2.t() @ b2
    a3 = a2.contiguous().view(s, m // s, n).transpose(1, 2)
    b3 = b2.contiguous().view(s, m // s, k)  # the right operand stays a contiguous (non-transposed) batch
    return torch.bmm(a3, b3, out_dtype=torch.float32).sum(0).to(a.dtype)


def _needed(ctx, i: int) -> bool:
    node = ctx.next_functions[i][0]
    if not ctx.needs_input_grad[i] or node is None:
        return False
    if node.name().endswith("AccumulateGrad"):  # a leaf: the engine cannot say under autograd.grad, so compute it
        return True
    return torch._C._will_engine_execute_node(node)


class _Dgrad(torch.autograd.Function):
    """dX = dY W (dY [..., N], W [N, K]) as a node of its own, for the weight gradient of its backward."""

    @staticmethod
    def forward(dy, w):
        return torch.matmul(dy, w)

    @staticmethod
    def setup_context(ctx, inputs, output):
        ctx.save_for_backward(*inputs)

    @staticmethod
    def backward(ctx, g):
        dy, w = ctx.saved_tensors
        gdy = gw = None
        if _needed(ctx, 0):
            gdy = _Linear.apply(g, w) if torch.is_grad_enabled() else F.linear(g, w)
        if _needed(ctx, 1):
            gw = weight_grad(dy, g)
        return gdy, gw


class _Linear(torch.autograd.Function):
    """Y = X W^T (X [..., K], W [N, K])."""

    @staticmethod
    def forward(x, w):
        return F.linear(x, w)

    @staticmethod
    def setup_context(ctx, inputs, output):
        ctx.save_for_backward(*inputs)

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        dx = dw = None
        if _needed(ctx, 0):
            dx = _Dgrad.apply(dy, w)
        if _needed(ctx, 1):
            dw = weight_grad(dy, x)
        return dx, dw


def linear(x: Tensor, w: Tensor, b: Optional[Tensor] = None) -> Tensor:
    """F.linear(x, w, b) with split-K weight gradients (the bias, if any, added by torch)."""
    y = _Linear.apply(x, w)
    return y if b is None else y + b


__all__ = ["linear", "weight_grad"]
