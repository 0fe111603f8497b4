"""GPU parity of the fused descent wrapper (``ebr_fused::descent_*``, HIP kernels through the C ABI) against the CPU
oracle ``oracle.descent_ref``, and of the harness's reference microstep with the fused wrapper against the eager one.

Tolerances: the kernels compute in fp32 and round to the dtype where the eager formula rounds, but their sums run in
another order than torch's and 1/sqrt is a correctly rounded division of a correctly rounded root where the oracle
uses torch.rsqrt, so a result next to a rounding boundary can land one unit in the last place (ulp) away. The bar:
fp32 within 1e-5 relative; bf16 / fp16 within one ulp of the dtype at the result's own magnitude plus one at the
row's RMS scale, with at most 1% of elements differing at all.
"""

import pytest
import torch

import oracle
from ebr_amd import _capi
from ebr_amd import descent
from ebr_amd import energy as en

pytestmark = pytest.mark.gpu

EPS = oracle.RMS_NORM_EPS
DTYPES = [torch.float32, torch.bfloat16, torch.float16]
# 16-bit rows of 576 .. 65536 elements take the register-resident step kernels with 1, 2, 4, 6 and 8 vectors per
# thread (the backward streams above 6); (1, 900, 512), fp32 rows above 32768 and the narrow shapes stream.
SHAPES = [(3, 81, 512), (2, 9, 64), (4, 100, 128), (2, 64, 512), (2, 128, 512), (1, 900, 512), (2, 7, 20), (1, 1, 4),
          (2, 5, 3)]


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _close(a, r, what=""):
    """The bar stated in the module docstring."""
    a = a.detach().cpu()
    assert a.shape == r.shape and a.dtype == r.dtype, (what, a.shape, r.shape, a.dtype, r.dtype)
    ad, rd = a.double(), r.double()
    scale = float(rd.square().mean().sqrt()) if r.numel() else 0.0
    diff = (ad - rd).abs()
    if r.dtype == torch.float32:
        ok = diff <= 1e-5 * (rd.abs() + scale)
    else:
        e = torch.finfo(r.dtype).eps
        ok = diff <= e * (rd.abs() + scale)
        frac = float((diff > 0).double().mean()) if r.numel() else 0.0
        assert frac <= 0.01, f"{what}: {frac:.4f} of elements differ"
    assert bool(ok.all()), f"{what}: max diff {float(diff.max()):.3e} (scale {scale:.3e})"


def _inputs(B, L, C, dtype, seed):
    z, noise, grad, sigma, alpha, active = oracle.make_descent_inputs(B, L, C, dtype=dtype, seed=seed)
    return z, noise, grad, sigma.to(dtype), alpha.to(dtype), active


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,L,C", SHAPES)
def test_noisy_point_matches_oracle(cuda, dtype, B, L, C):
    _say(f"noisy_point B={B} L={L} C={C} {dtype}")
    z, noise, _, sigma, _, _ = _inputs(B, L, C, dtype, seed=B * 7 + C)
    zc, nc = z.to(cuda), noise.to(cuda)
    _close(descent.normalize(zc), oracle.rms_norm(z, EPS), "normalize")
    _close(descent.noisy_point_replayed(zc, nc), oracle.noisy_point_replayed(z, noise, EPS), "replayed")
    _close(descent.noisy_point(zc, nc, sigma.to(cuda)), oracle.noisy_point(z, noise, sigma, EPS), "sigma tensor")
    _close(descent.noisy_point(zc, nc, 0.37), oracle.noisy_point(z, noise, 0.37, EPS), "sigma float")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,L,C", SHAPES)
def test_noisy_point_backward_matches_oracle(cuda, dtype, B, L, C):
    _say(f"noisy_point_bwd B={B} L={L} C={C} {dtype}")
    z, _, grad, _, _, _ = _inputs(B, L, C, dtype, seed=B + C)
    dz = torch.ops.ebr_fused.descent_noisy_point_bwd(z.to(cuda), grad.to(cuda), EPS)
    _close(dz, oracle.vjp_noisy_point(z, None, None, grad, EPS), "dz")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,L,C", SHAPES)
@pytest.mark.parametrize("masked", [False, True])
def test_step_and_project_matches_oracle(cuda, dtype, B, L, C, masked):
    _say(f"step_project B={B} L={L} C={C} {dtype} masked={masked}")
    z, noise, grad, sigma, alpha, active = _inputs(B, L, C, dtype, seed=B * 3 + L)
    act = active if masked else None
    v = oracle.noisy_point(z, noise, sigma, EPS)
    for a in (alpha, 0.05):
        out = descent.step_and_project(v.to(cuda), grad.to(cuda), a.to(cuda) if torch.is_tensor(a) else a, z.to(cuda),
                                       None if act is None else act.to(cuda))
        ref = oracle.step_and_project(v, grad, a, z, act, EPS)
        _close(out, ref, f"out alpha={'tensor' if torch.is_tensor(a) else a}")
        if act is not None:  # rows that do not move are z, bit for bit
            keep = ~act.view(-1)
            assert torch.equal(out.cpu()[keep], z[keep])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,L,C", SHAPES)
@pytest.mark.parametrize("masked", [False, True])
def test_step_and_project_backward_matches_oracle(cuda, dtype, B, L, C, masked):
    _say(f"step_project_bwd B={B} L={L} C={C} {dtype} masked={masked}")
    z, noise, grad, sigma, alpha, active = _inputs(B, L, C, dtype, seed=B * 5 + C)
    act = active if masked else None
    v = oracle.noisy_point(z, noise, sigma, EPS)
    dout = torch.randn(z.shape, generator=torch.Generator().manual_seed(C)).to(dtype)
    rdv, rdg, rdz = oracle.vjp_step_and_project(v, grad, alpha, z, act, dout, EPS)
    a32 = alpha.reshape(-1).float().to(cuda)
    act8 = None if act is None else act.reshape(-1).to(torch.uint8).to(cuda)
    vc, gc = v.to(cuda), grad.to(cuda)
    _, rms = torch.ops.ebr_fused.descent_step_project(vc, gc, a32, z.to(cuda), act8, EPS)
    dv, dg, dz = torch.ops.ebr_fused.descent_step_project_bwd(vc, gc, a32, act8, rms, dout.to(cuda), EPS)
    _close(dv, rdv, "dv")
    _close(dg, rdg, "dg")
    if act is None:
        assert dz.numel() == 0
    else:
        assert torch.equal(dz.cpu(), rdz)  # dout on rows that keep z, zero elsewhere: exact


@pytest.mark.parametrize("B,L,C", [(3, 9, 32), (3, 81, 512)])
def test_projection_clamp_and_rms(cuda, B, L, C):
    """A row whose RMS is below eps divides by eps in both directions; the kernel's rms output is the clamped
    board RMS (fp32: a register-resident and a streamed row)."""
    _say(f"step_project clamp B={B} L={L} C={C}")
    z, noise, grad, sigma, alpha, _ = _inputs(B, L, C, torch.float32, seed=11)
    v = oracle.noisy_point(z, noise, sigma, EPS)
    v[1] *= 1e-7
    grad[1] *= 1e-7
    a32 = alpha.reshape(-1).float().to(cuda)
    out, rms = torch.ops.ebr_fused.descent_step_project(v.to(cuda), grad.to(cuda), a32, None, None, EPS)
    _close(out, oracle.step_and_project(v, grad, alpha, z, None, EPS), "out")
    u = (v - alpha * grad).double()
    ref_rms = u.square().mean(dim=(1, 2)).sqrt().clamp_min(EPS)
    assert torch.allclose(rms.cpu().double(), ref_rms, rtol=1e-6) and float(rms[1]) == pytest.approx(EPS)
    dout = torch.randn(z.shape, generator=torch.Generator().manual_seed(12))
    dv, dg, _ = torch.ops.ebr_fused.descent_step_project_bwd(v.to(cuda), grad.to(cuda), a32, None, rms, dout.to(cuda),
                                                             EPS)
    rdv, rdg, _ = oracle.vjp_step_and_project(v, grad, alpha, z, None, dout, EPS)
    _close(dv, rdv, "dv")
    _close(dg, rdg, "dg")


def test_unaligned_views_take_narrow_accesses(cuda):
    """Views starting one element into their buffers (only scalar accesses aligned): results do not change."""
    _say("descent unaligned")
    B, L, C = 2, 9, 64
    dtype = torch.bfloat16
    z, noise, grad, sigma, alpha, active = _inputs(B, L, C, dtype, seed=13)

    def shifted(t):
        buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=cuda)
        buf[1:] = t.reshape(-1).to(cuda)
        return buf[1:].view(t.shape)

    zc, nc, gc = shifted(z), shifted(noise), shifted(grad)
    assert zc.data_ptr() % 4 != 0
    _close(descent.noisy_point(zc, nc, sigma.to(cuda)), oracle.noisy_point(z, noise, sigma, EPS), "noisy")
    v = oracle.noisy_point(z, noise, sigma, EPS)
    _close(descent.step_and_project(shifted(v), gc, alpha.to(cuda), zc, active.to(cuda)),
           oracle.step_and_project(v, grad, alpha, z, active, EPS), "step")


def test_autograd_through_both_wrappers(cuda):
    """First-order gradients of a loss through noisy_point -> step_and_project, with respect to z and the energy
    gradient, match autograd through the oracle (fp32)."""
    _say("descent autograd")
    B, L, C = 3, 16, 48
    z, noise, grad, sigma, alpha, active = _inputs(B, L, C, torch.float32, seed=14)
    w = torch.randn(z.shape, generator=torch.Generator().manual_seed(15))

    def run(noisy, step, dev):
        zz = z.to(dev).requires_grad_(True)
        gg = grad.to(dev).requires_grad_(True)
        v = noisy(zz, noise.to(dev), sigma.to(dev))
        out = step(v, gg, alpha.to(dev), zz, active.to(dev))
        return torch.autograd.grad((out * w.to(dev)).sum(), (zz, gg))

    got = run(descent.noisy_point, descent.step_and_project, cuda)
    ref = run(lambda a, b, c: oracle.noisy_point(a, b, c, EPS),
              lambda a, b, c, d, e: oracle.step_and_project(a, b, c, d, e, EPS), "cpu")
    for name, a, r in zip(("dz", "dgrad"), got, ref):
        _close(a, r, name)


def test_config3_shape_properties(cuda):
    """The training step's shape ([384, 81, 512], bf16): moved rows have unit RMS, kept rows are z exactly, and the
    output matches the oracle."""
    _say("descent config-3 shape")
    B, L, C = 384, 81, 512
    z, noise, grad, sigma, alpha, active = _inputs(B, L, C, torch.bfloat16, seed=16)
    zc, nc, gc = z.to(cuda), noise.to(cuda), grad.to(cuda)
    v = descent.noisy_point(zc, nc, sigma.to(cuda))
    out = descent.step_and_project(v, gc, alpha.to(cuda), zc, active.to(cuda))
    a = active.view(-1).to(cuda)
    rms = out.float().square().mean(dim=(1, 2)).sqrt()
    assert float((rms[a] - 1).abs().max()) < 4e-3
    assert torch.equal(out[~a], zc[~a])
    rv = oracle.noisy_point(z, noise, sigma, EPS)
    _close(v, rv, "v")
    _close(out, oracle.step_and_project(rv, grad, alpha, z, active, EPS), "out")


def test_c_abi_errors(cuda):
    """Unsupported dtype code, empty shape and NULL pointers come back as error codes, before any launch."""
    lib = _capi.load()
    t = torch.zeros(2, 3, 8, device=cuda)
    p = t.data_ptr()
    assert lib.ebr_descent_noisy_point(7, 2, 3, 8, EPS, p, None, None, p, None) == 1
    assert lib.ebr_descent_noisy_point(0, 0, 3, 8, EPS, p, None, None, p, None) == 2
    assert lib.ebr_descent_noisy_point(0, 2, 3, 8, EPS, None, None, None, p, None) == 4
    assert lib.ebr_descent_step_project(0, 2, 24, EPS, p, p, p, None, p, p, p, None) == 4  # a mask without z
    with pytest.raises(TypeError):
        descent.normalize(torch.zeros(2, 3, 8, device=cuda, dtype=torch.float64))


def test_ops_reject_mismatched_operands_and_take_empty_inputs(cuda):
    """The C ABI takes only the board's sizes, so every other operand of the raw ops is checked against them before a
    launch; an empty batch returns empty results without one."""
    z = torch.randn(2, 3, 8, device=cuda)
    row = torch.ones(2, device=cuda)
    ops = torch.ops.ebr_fused
    with pytest.raises(ValueError):
        ops.descent_noisy_point(z, z[:1], None, EPS)
    with pytest.raises(ValueError):
        ops.descent_noisy_point(z, z, torch.ones(3, device=cuda), EPS)  # sigma per row: 2 values
    with pytest.raises(ValueError):
        ops.descent_noisy_point_bwd(z, z[:, :2], EPS)
    with pytest.raises(ValueError):
        ops.descent_step_project(z, z, torch.ones(1, device=cuda), None, None, EPS)
    with pytest.raises(ValueError):
        ops.descent_step_project(z, z, row, z, torch.ones(2, device=cuda), EPS)  # the mask must be uint8
    with pytest.raises(ValueError):
        ops.descent_step_project(z, z, row, None, torch.ones(2, device=cuda, dtype=torch.uint8), EPS)
    with pytest.raises(ValueError):
        ops.descent_step_project_bwd(z, z, row, None, torch.ones(5, device=cuda), z, EPS)  # rms per row
    e = torch.empty(0, 3, 8, device=cuda)
    assert ops.descent_noisy_point(e, None, None, EPS).shape == e.shape
    out, rms = ops.descent_step_project(e, e, torch.empty(0, device=cuda), None, None, EPS)
    assert out.shape == e.shape and rms.shape == (0,)


def _energy_models(cuda):
    """Two copies of one small energy network (fp32 parameters; activations follow the latent's dtype)."""
    cfg = en.EnergyConfig(hidden_size=64, num_heads=4, grid=(4, 4))
    return [en.build(cfg, cuda, seed=21) for _ in range(2)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_train_step_fused_wrapper_matches_eager(cuda, dtype):
    """The reference microstep in a graded training step (noise drawn with per-row sigma, per-row alpha, a row mask)
    with the fused wrapper gives the eager wrapper's loss and parameter gradients."""
    _say(f"train step fused vs eager wrapper {dtype}")
    (mf, df), (me, de) = _energy_models(cuda)
    g = torch.Generator("cpu").manual_seed(22)
    B, L, steps = 4, 16, 3
    x = torch.randint(0, 11, (B, L), generator=g).to(cuda)
    z0 = torch.randn(B, L, 64, generator=g).to(cuda, dtype)
    tg = torch.randint(0, 11, (B, L), generator=g).to(cuda)
    sigma = torch.full((B, 1, 1), 0.1, device=cuda, dtype=dtype)
    alpha = (0.05 + 0.1 * torch.rand(B, 1, 1, generator=g)).to(cuda, dtype)
    active = [torch.tensor([True, False, True, True], device=cuda).view(-1, 1, 1)] * steps
    losses = []
    for (m, d), wrapper in (((mf, df), "fused"), ((me, de), "eager")):
        torch.manual_seed(23)  # the same noise draws in both runs
        losses.append(float(en.train_step(m, d, x, z0, tg, steps=steps, alpha=alpha, wrapper=wrapper, sigma=sigma,
                                          active=active)))
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert abs(losses[0] - losses[1]) <= tol * max(1.0, abs(losses[1]))
    gtol = 1e-4 if dtype == torch.float32 else 5e-2
    for (n, pf), (_, pe) in zip(mf.named_parameters(), me.named_parameters()):
        if pe.grad is not None:
            err = float((pf.grad.float() - pe.grad.float()).abs().max() / pe.grad.float().abs().max().clamp_min(1e-12))
            assert err <= gtol, (n, err)


def test_nograd_descent_fused_wrapper_matches_eager(cuda):
    """Non-graded descent with replayed noise (the explore / eval tier): fused and eager wrappers agree (fp32)."""
    _say("no-grad descent fused vs eager wrapper")
    (mf, _), _ = _energy_models(cuda)
    g = torch.Generator("cpu").manual_seed(24)
    B, L, steps = 3, 16, 4
    x = torch.randint(0, 11, (B, L), generator=g).to(cuda)
    z0 = torch.randn(B, L, 64, generator=g).to(cuda)
    noises = [0.1 * torch.randn(B, L, 64, generator=g).to(cuda) for _ in range(steps)]
    xe = mf.puzzle_embedding(x, z0.dtype).detach()
    out = [en.descend(mf, z0, xe, steps, 0.1, create_graph=False, wrapper=w, noises=noises).detach()
           for w in ("fused", "eager")]
    assert float((out[0] - out[1]).abs().max()) <= 1e-5 * float(out[1].abs().max())


def test_wrapper_functions_under_torch_compile(cuda):
    """The reference compiles its wrapper functions (energy.py:249-261); the fused ones trace as opaque nodes under
    torch.compile (aot_eager, no Triton) and give the eager kernels' results, forward and first-order backward."""
    _say("descent under torch.compile")
    torch._dynamo.reset()
    B, L, C = 3, 16, 64
    z, noise, grad, sigma, alpha, active = _inputs(B, L, C, torch.float32, seed=31)
    zc, nc, gc = z.to(cuda), noise.to(cuda), grad.to(cuda)
    sc, ac, mc = sigma.to(cuda), alpha.to(cuda), active.to(cuda)

    def microstep(zz, gg):
        v = descent.noisy_point(zz, nc, sc)
        return descent.step_and_project(v, gg, ac, zz, mc)

    compiled = torch.compile(microstep, backend="aot_eager", fullgraph=True)
    w = torch.randn(z.shape, generator=torch.Generator().manual_seed(32)).to(cuda)
    outs = []
    for fn in (microstep, compiled):
        zz, gg = zc.clone().requires_grad_(True), gc.clone().requires_grad_(True)
        out = fn(zz, gg)
        outs.append((out.detach(), *torch.autograd.grad((out * w).sum(), (zz, gg))))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
