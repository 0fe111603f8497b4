"""GPU parity of the split-K linear (``ebr_amd.linear``): the weight gradient as batched fp32 partial products against
an fp32 product of the same bf16 / fp16 operands, at the energy network's training shapes; the linear's first and
second derivatives against ``F.linear`` at a size that takes the split path; and the graded training step with
``linear_impl="splitk"`` against the eager one.

Bars: the weight gradient within 1e-2 of the fp32 product, max-relative (one 16-bit rounding of an fp32 sum, as
torch's own single GEMM, which is held to the same bar); derivatives within 2e-2 max-relative of F.linear's.
"""

import pytest
import torch
import torch.nn.functional as F

from ebr_amd import energy as en
from ebr_amd import linear

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _rel(a, r):
    a, r = a.detach().double(), r.detach().double()
    return float((a - r).abs().max() / r.abs().max().clamp_min(1e-30))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,n,k", [(31104, 1536, 512), (31104, 512, 512), (31104, 3072, 512), (31104, 512, 1536),
                                   (16384, 96, 40), (5000, 64, 64)])
def test_weight_grad_matches_fp32_product(cuda, dtype, m, n, k):
    _say(f"weight_grad m={m} n={n} k={k} {dtype}")
    g = torch.Generator(cuda).manual_seed(m + n + k)
    a = torch.randn(m, n, device=cuda, generator=g).to(dtype)
    b = torch.randn(m, k, device=cuda, generator=g).to(dtype)
    got = linear.weight_grad(a, b)
    ref = a.float().t() @ b.float()
    assert got.dtype == dtype and got.shape == (n, k)
    assert _rel(got, ref) <= 1e-2
    assert _rel(a.t() @ b, ref) <= 1e-2  # torch's single GEMM meets the same bar


def test_weight_grad_takes_three_dim_operands(cuda):
    g = torch.Generator(cuda).manual_seed(1)
    a = torch.randn(48, 81, 256, device=cuda, generator=g).to(torch.bfloat16)
    b = torch.randn(48, 81, 128, device=cuda, generator=g).to(torch.bfloat16)
    assert linear._splits(48 * 81, 256 * 128) > 1
    assert _rel(linear.weight_grad(a, b), a.reshape(-1, 256).float().t() @ b.reshape(-1, 128).float()) <= 1e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_linear_two_orders_match_f_linear(cuda, dtype):
    _say(f"linear two orders {dtype}")
    g = torch.Generator(cuda).manual_seed(2)
    x0 = torch.randn(64, 256, 128, device=cuda, generator=g).to(dtype)
    w0 = (torch.randn(128, 128, device=cuda, generator=g) / 12).to(dtype)
    u = torch.randn(64, 256, 128, device=cuda, generator=g).to(dtype)
    outs = []
    for fn in (linear.linear, F.linear):
        x, w = x0.clone().requires_grad_(True), w0.clone().requires_grad_(True)
        wc = w * 1  # a non-leaf weight, as the model's cast parameter
        y = fn(torch.tanh(fn(x, wc)), wc)
        (dx,) = torch.autograd.grad((y * u).sum(), x, create_graph=True)
        (dx.float().square().sum() + y.float().square().sum()).backward()
        outs.append([y, dx, x.grad, w.grad])
    for name, a, r in zip(("y", "dx", "gx", "gw"), *outs):
        assert _rel(a, r) <= (1e-5 if dtype == torch.float32 else 2e-2), (name, _rel(a, r))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_train_step_splitk_matches_eager(cuda, dtype):
    _say(f"train step splitk {dtype}")
    runs = []
    g = torch.Generator("cpu").manual_seed(6)
    B, L = 128, 16  # 2048 token rows: two splits of the minimum size
    x = torch.randint(0, 11, (B, L), generator=g).to(cuda)
    z0 = torch.randn(B, L, 64, generator=g).to(cuda, dtype)
    tg = torch.randint(0, 11, (B, L), generator=g).to(cuda)
    for impl in ("splitk", "eager"):
        cfg = en.EnergyConfig(hidden_size=64, num_heads=4, grid=(4, 4), linear_impl=impl, block_impl="fused")
        model, dec = en.build(cfg, cuda, seed=7)
        loss = float(en.train_step(model, dec, x, z0, tg, steps=3))
        runs.append((loss, {n: p.grad.float().clone() for n, p in model.named_parameters() if p.grad is not None}))
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert abs(runs[0][0] - runs[1][0]) <= tol * max(1.0, abs(runs[1][0]))
    gtol = 1e-4 if dtype == torch.float32 else 1e-1
    for n, r in runs[1][1].items():
        assert _rel(runs[0][1][n], r) <= gtol, (n, _rel(runs[0][1][n], r))
