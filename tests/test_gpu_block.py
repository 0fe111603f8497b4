"""GPU parity of the fused energy-block kernels (``ebr_fused::block_*`` through the C ABI): rms_norm and the SwiGLU
activation, forward, backward and backward-of-backward, against torch autograd of the eager formulas
(``ebr_amd.layers.rms_norm``, ``F.silu(gate) * up``), plus fp64 gradcheck / gradgradcheck on the GPU and the energy
network's graded training step with the fused block against the eager one.

Bars: fp64 1e-10 (the second derivatives cancel terms of order 1, so their rounding differs at ~1e-12) and fp32 1e-5
relative (max|a - ref| / max|ref|); bf16 / fp16 2e-2 (the kernels round each output once where eager chains several
rounded kernels).
"""

import pytest
import torch
import torch.nn.functional as F

from ebr_amd import block
from ebr_amd import energy as en
from ebr_amd import layers

pytestmark = pytest.mark.gpu

EPS = 1e-5
TOL = {torch.float64: 1e-10, torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _rel(a, r):
    a, r = a.detach().double().cpu(), r.detach().double().cpu()
    return float((a - r).abs().max() / r.abs().max().clamp_min(1e-30))


def _eager_swiglu(gu):
    g, u = gu.chunk(2, dim=-1)
    return F.silu(g) * u


def _three_orders(fn, x, seed):
    """y, dL/dx (with create_graph) and d/dx <c, dL/dx> for L = <w, fn(x)>, plus the gradient w.r.t. w."""
    g = torch.Generator().manual_seed(seed)
    x = x.detach().clone().requires_grad_(True)
    y = fn(x)
    w = torch.randn(y.shape, generator=g).to(y).requires_grad_(True)
    c = torch.randn(x.shape, generator=g).to(x)
    (dx,) = torch.autograd.grad((y * w).sum(), x, create_graph=True)
    gx, gw = torch.autograd.grad((dx * c).sum(), (x, w))
    return y.detach(), dx.detach(), gx, gw


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16, torch.float16])
# widths cover the register-resident vector kernels (1 to 4 vectors per lane, a partial last vector, row counts that
# leave the last wave short) and the streaming fallback (odd widths, rows beyond 4 vectors per lane)
@pytest.mark.parametrize(
    "shape", [(3, 9, 64), (2, 81, 512), (5, 7, 13), (2, 1, 3), (3, 7, 1024), (1, 5, 1544), (2, 3, 2056), (1, 9, 520)]
)
def test_rms_norm_three_orders(cuda, dtype, shape):
    _say(f"rms_norm {shape} {dtype}")
    x = (torch.randn(shape, generator=torch.Generator().manual_seed(1)) * 1.5).to(cuda, dtype)
    got = _three_orders(lambda t: block.rms_norm(t, EPS), x, seed=2)
    if dtype == torch.float64:  # layers.rms_norm (as the reference's) computes in fp32; the kernel keeps fp64
        ref = _three_orders(lambda t: t * torch.rsqrt(t.square().mean(-1, keepdim=True) + EPS), x, seed=2)
    else:
        ref = _three_orders(lambda t: layers.rms_norm(t, EPS), x, seed=2)
    for name, a, r in zip(("y", "dx", "d2x", "dw"), got, ref):
        assert _rel(a, r) <= TOL[dtype], (name, _rel(a, r))


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16, torch.float16])
# I = 64 and 1536: vector kernel; I = 3: element kernel; I = 12: vector kernel for fp32 / fp64, element kernel for
# 16-bit (not a multiple of 8)
@pytest.mark.parametrize("shape", [(3, 9, 128), (2, 81, 3072), (4, 6), (5, 7, 24)])
def test_swiglu_three_orders(cuda, dtype, shape):
    _say(f"swiglu {shape} {dtype}")
    x = (torch.randn(shape, generator=torch.Generator().manual_seed(3)) * 2).to(cuda, dtype)
    got = _three_orders(block.swiglu, x, seed=4)
    ref = _three_orders(_eager_swiglu, x, seed=4)
    for name, a, r in zip(("y", "dx", "d2x", "dw"), got, ref):
        assert _rel(a, r) <= TOL[dtype], (name, _rel(a, r))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_misaligned_rows_take_the_element_kernels(cuda, dtype):
    """Tensors that start 2 or 4 bytes past a 16-byte boundary (contiguous, so no copy is made) give the same results
    as aligned copies of the same values."""
    _say(f"block misaligned {dtype}")
    g = torch.Generator().manual_seed(8)
    for width, fn in ((512, lambda t: block.rms_norm(t, EPS)), (256, block.swiglu)):
        n = 6 * width
        buf = torch.randn(n + 1, generator=g).to(cuda, dtype)
        x = buf[1:].view(6, width)
        assert x.is_contiguous() and x.data_ptr() % 16 != 0
        got = _three_orders(fn, x, seed=9)
        ref = _three_orders(fn, x.clone(), seed=9)
        for name, a, r in zip(("y", "dx", "d2x", "dw"), got, ref):
            assert _rel(a, r) <= TOL[dtype], (width, name, _rel(a, r))


def test_swiglu_64bit_offsets(cuda):
    """A gate / up tensor of more than 2^31 elements: the vector kernel's 64-bit index variant."""
    _say("swiglu 64-bit offsets")
    rows, inter = (1 << 20) + 1, 1024
    gen = torch.Generator(cuda).manual_seed(3)
    gu = torch.empty(rows, 2 * inter, device=cuda, dtype=torch.bfloat16).normal_(generator=gen)
    assert gu.numel() >= (1 << 31)
    y = block.swiglu(gu)
    ref = _eager_swiglu(gu)
    del gu
    assert _rel(y[-4:], ref[-4:]) <= TOL[torch.bfloat16]  # rows past the 2^31st element
    assert _rel(y, ref) <= TOL[torch.bfloat16]


def test_fp64_gradcheck_and_gradgradcheck(cuda):
    _say("block gradcheck")
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 3, 8, generator=g, dtype=torch.float64).to(cuda).requires_grad_(True)
    assert torch.autograd.gradcheck(lambda t: block.rms_norm(t, EPS), (x,))
    assert torch.autograd.gradgradcheck(lambda t: block.rms_norm(t, EPS), (x,))
    gu = torch.randn(2, 3, 10, generator=g, dtype=torch.float64).to(cuda).requires_grad_(True)
    assert torch.autograd.gradcheck(block.swiglu, (gu,))
    assert torch.autograd.gradgradcheck(block.swiglu, (gu,))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_train_step_fused_block_matches_eager(cuda, dtype):
    """The graded training step (second order through both blocks) with the fused block equals the eager one."""
    _say(f"train step fused block {dtype}")
    models = []
    for impl in ("fused", "eager"):
        cfg = en.EnergyConfig(hidden_size=64, num_heads=4, grid=(4, 4), block_impl=impl)
        models.append(en.build(cfg, cuda, seed=41))
    g = torch.Generator("cpu").manual_seed(42)
    B, L = 3, 16
    x = torch.randint(0, 11, (B, L), generator=g).to(cuda)
    z0 = torch.randn(B, L, 64, generator=g).to(cuda, dtype)
    tg = torch.randint(0, 11, (B, L), generator=g).to(cuda)
    losses = [float(en.train_step(m, d, x, z0, tg, steps=3)) for m, d in models]
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert abs(losses[0] - losses[1]) <= tol * max(1.0, abs(losses[1]))
    gtol = 1e-4 if dtype == torch.float32 else 1e-1
    (mf, _), (me, _) = models
    for (n, pf), (_, pe) in zip(mf.named_parameters(), me.named_parameters()):
        if pe.grad is not None:
            err = float((pf.grad.float() - pe.grad.float()).abs().max() / pe.grad.float().abs().max().clamp_min(1e-12))
            assert err <= gtol, (n, err)


def test_ops_reject_mismatched_operands_and_take_empty_inputs(cuda):
    """The C ABI takes only x's (or gu's) sizes, so every other operand is checked against them before a launch;
    empty tensors return empty results without one."""
    x = torch.randn(4, 64, device=cuda)
    with pytest.raises(ValueError):
        torch.ops.ebr_fused.block_rmsnorm_bwd(x, x[:3], EPS)
    with pytest.raises(ValueError):
        torch.ops.ebr_fused.block_rmsnorm_bwd2(x, x, x[:, :32], EPS)
    gu = torch.randn(4, 64, device=cuda)
    with pytest.raises(ValueError):
        torch.ops.ebr_fused.block_swiglu_bwd(gu, gu)  # dy must have the half width
    with pytest.raises(ValueError):
        torch.ops.ebr_fused.block_swiglu_bwd2(gu, gu[:, :32], gu[:2])
    with pytest.raises(ValueError):
        torch.ops.ebr_fused.block_swiglu(torch.randn(4, 7, device=cuda))
    e = torch.empty(0, 64, device=cuda)
    assert block.rms_norm(e, EPS).shape == (0, 64) and block.swiglu(e).shape == (0, 32)
    xe = e.clone().requires_grad_(True)
    (dx,) = torch.autograd.grad(block.rms_norm(xe, EPS).sum(), xe, create_graph=True)
    assert dx.shape == (0, 64)
