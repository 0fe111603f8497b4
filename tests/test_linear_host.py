"""The split-K linear (``ebr_amd.linear``) on the CPU: its autograd structure against ``F.linear`` (values, first,
second and third derivatives in fp64, gradcheck / gradgradcheck), that the descent's ``autograd.grad(E, z)`` takes no
weight gradient while the training backward takes them all, and a graded training step with ``linear_impl="splitk"``
equal to the eager one. The split-K product itself needs ``bmm(out_dtype=float32)``, a GPU kernel; its parity is in
``tests/test_gpu_linear.py``."""

import pytest
import torch
import torch.nn.functional as F

from ebr_amd import energy as en
from ebr_amd import layers, linear

F64 = torch.float64


def _derivs(fn, x, w, seed):
    g = torch.Generator().manual_seed(seed)
    x = x.detach().clone().requires_grad_(True)
    w = w.detach().clone().requires_grad_(True)
    y = fn(torch.tanh(fn(x, w)), w)  # nonlinear, so that every order depends on x and w
    u = torch.randn(y.shape, generator=g, dtype=F64)
    dx, dw = torch.autograd.grad((y * u).sum(), (x, w), create_graph=True)
    c1, c2 = torch.randn(dx.shape, generator=g, dtype=F64), torch.randn(dw.shape, generator=g, dtype=F64)
    hx, hw = torch.autograd.grad((dx * c1).sum() + (dw * c2).sum(), (x, w), create_graph=True)
    (tx,) = torch.autograd.grad((hx * hx).sum() + (hw * hw).sum(), x)
    return [t.detach() for t in (y, dx, dw, hx, hw, tx)]


def test_linear_values_and_three_orders_equal_f_linear():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 5, 7, generator=g, dtype=F64)
    w = torch.randn(7, 7, generator=g, dtype=F64) / 3
    got = _derivs(linear.linear, x, w, seed=1)
    ref = _derivs(F.linear, x, w, seed=1)
    for a, r in zip(got, ref):
        assert torch.allclose(a, r, rtol=1e-12, atol=1e-12)


def test_linear_gradcheck_and_gradgradcheck():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 3, 4, generator=g, dtype=F64, requires_grad=True)
    w = torch.randn(5, 4, generator=g, dtype=F64, requires_grad=True)
    b = torch.randn(5, generator=g, dtype=F64, requires_grad=True)
    assert torch.autograd.gradcheck(linear.linear, (x, w, b))
    assert torch.autograd.gradgradcheck(linear.linear, (x, w, b))


def test_descent_takes_no_weight_gradient(monkeypatch):
    """autograd.grad(E, z, create_graph=True) asks for dE/dz only: no weight gradient is computed then; the training
    backward through that graph computes every weight gradient, equal to F.linear's."""
    calls = []
    real = linear.weight_grad

    def counting(a, b):
        calls.append(torch.is_grad_enabled())
        return real(a, b)

    monkeypatch.setattr(linear, "weight_grad", counting)
    g = torch.Generator().manual_seed(3)
    w_ref = torch.randn(6, 6, generator=g, dtype=F64, requires_grad=True)
    z0 = torch.randn(4, 6, generator=g, dtype=F64)
    grads = []
    for fn in (linear.linear, F.linear):
        w = w_ref.detach().clone().requires_grad_(True)
        z = z0.clone().requires_grad_(True)
        wc = w.clone()  # as the model's weight: a cast of the fp32 parameter, not the leaf itself
        e = torch.tanh(fn(torch.tanh(fn(z, wc)), wc)).sum()
        (dz,) = torch.autograd.grad(e, z, create_graph=True)
        if fn is linear.linear:
            assert calls == []
        z1 = z - 0.1 * dz
        (fn(z1, wc) ** 2).sum().backward()
        grads.append(w.grad)
    assert len(calls) >= 4 and not any(calls)  # the training backward, without a graph
    assert torch.allclose(grads[0], grads[1], rtol=1e-12, atol=1e-12)


def test_train_step_splitk_matches_eager():
    kw = dict(hidden_size=32, num_heads=2, num_layers=2, grid=(3, 3), attn_backend="math", attn_nograd_backend="math")
    g = torch.Generator().manual_seed(4)
    B, L = 2, 9
    x = torch.randint(0, 11, (B, L), generator=g)
    z0 = torch.randn(B, L, 32, generator=g)
    tg = torch.randint(0, 11, (B, L), generator=g)
    runs = []
    for impl in ("splitk", "eager"):
        model, dec = en.build(en.EnergyConfig(linear_impl=impl, **kw), torch.device("cpu"), seed=5)
        loss = en.train_step(model, dec, x, z0, tg, steps=3)
        runs.append((float(loss), {n: p.grad.clone() for n, p in model.named_parameters() if p.grad is not None}))
    assert abs(runs[0][0] - runs[1][0]) <= 1e-6 * max(1.0, abs(runs[1][0]))
    assert runs[0][1].keys() == runs[1][1].keys() and len(runs[0][1]) > 0
    for n in runs[1][1]:
        assert torch.allclose(runs[0][1][n], runs[1][1][n], rtol=1e-4, atol=1e-6), n


def test_linear_impl_is_checked():
    with pytest.raises(ValueError):
        layers.CastedLinear(4, 4, bias=False, impl="fast")
    with pytest.raises(ValueError):
        en.build(en.EnergyConfig(hidden_size=32, num_heads=2, grid=(3, 3), linear_impl="fast"), torch.device("cpu"))
    assert linear._splits(31104, 1536 * 512) == 16 and linear._splits(31104, 3072 * 512) == 8
    assert linear._splits(1000, 64) == 1  # too few rows to split
