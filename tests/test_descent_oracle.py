"""CPU checks that pin the descent-wrapper oracle (``oracle.descent_ref``) against library routines, closed forms and
invariants rather than a retyped formula; the harness's eager wrapper against it; and the argument checks of
``ebr_amd.descent`` (which run before any kernel)."""

import pytest
import torch
import torch.nn.functional as F

import oracle
from ebr_amd import energy as en
from ebr_amd import layers

EPS = oracle.RMS_NORM_EPS


def _rows_rms(t):
    return t.double().square().mean(dim=(1, 2)).sqrt()


def test_rms_norm_is_torch_rms_norm():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 7, 48, generator=g, dtype=torch.float64) * 2.5
    assert torch.allclose(oracle.rms_norm(x, EPS), F.rms_norm(x, (48,), eps=EPS), rtol=1e-13, atol=0)
    # the closed form of the output's mean square: m / (m + eps)
    x = torch.randn(2, 5, 32, generator=g, dtype=torch.float64) * 3e-3  # m ~ 1e-5: eps matters
    m = x.square().mean(-1)
    assert torch.allclose(oracle.rms_norm(x, EPS).square().mean(-1), m / (m + EPS), rtol=1e-12)


def test_rms_norm_planted_mistake_is_caught():
    """Dropping eps changes the closed-form mean square where the input is small."""
    x = torch.randn(2, 5, 32, generator=torch.Generator().manual_seed(1), dtype=torch.float64) * 3e-3
    m = x.square().mean(-1)
    no_eps = x * torch.rsqrt(x.square().mean(-1, keepdim=True))
    assert not torch.allclose(no_eps.square().mean(-1), m / (m + EPS), rtol=1e-3)


def test_sphere_is_the_scaled_l2_normalisation():
    g = torch.Generator().manual_seed(2)
    u = torch.randn(4, 9, 16, generator=g, dtype=torch.float64)
    n = u[0].numel()
    norm = torch.linalg.vector_norm(u.flatten(1), dim=1).view(-1, 1, 1)
    assert torch.allclose(oracle.sphere(u, EPS), u * n**0.5 / norm, rtol=1e-13)
    assert torch.allclose(_rows_rms(oracle.sphere(u, EPS)), torch.ones(4, dtype=torch.float64), rtol=1e-13)
    assert torch.allclose(oracle.sphere(7.5 * u, EPS), oracle.sphere(u, EPS), rtol=1e-13)  # scale invariance
    tiny = u * 1e-7  # RMS below eps: the clamp divides by eps
    assert torch.allclose(oracle.sphere(tiny, EPS), tiny / EPS, rtol=1e-13)
    # normalising each token instead of the board is a plausible mistake; it fails the board-norm identity
    wrong = u / u.square().mean(-1, keepdim=True).sqrt()
    assert not torch.allclose(wrong, u * n**0.5 / norm, rtol=1e-3)


def test_noisy_point_is_affine_in_the_noise():
    z, noise, _, sigma, _, _ = oracle.make_descent_inputs(3, 8, 32, dtype=torch.float64, seed=3)
    base = oracle.rms_norm(z, EPS)
    assert torch.allclose(oracle.noisy_point(z, noise, sigma, EPS) - base, noise * sigma, atol=1e-14)
    assert torch.allclose(oracle.noisy_point(z, noise, 0.3, EPS) - base, 0.3 * noise, atol=1e-14)
    assert torch.equal(oracle.noisy_point_replayed(z, noise, EPS), base + noise)


def test_step_and_project_invariants():
    z, _, grad, _, alpha, active = oracle.make_descent_inputs(5, 9, 16, dtype=torch.float64, seed=4)
    v = oracle.rms_norm(z, EPS)
    out = oracle.step_and_project(v, grad, alpha, z, active, EPS)
    keep = ~active.view(-1)
    assert torch.equal(out[keep], z[keep])  # rows that do not move keep z exactly
    moved = _rows_rms(out)[active.view(-1)]
    assert torch.allclose(moved, torch.ones_like(moved), rtol=1e-13)
    assert torch.allclose(oracle.step_and_project(v, grad, 0.0, z, None, EPS), oracle.sphere(v, EPS), rtol=1e-14)
    # the step direction: v - alpha g projected back equals the L2-normalised difference
    u = v - alpha * grad
    norm = torch.linalg.vector_norm(u.flatten(1), dim=1).view(-1, 1, 1)
    ref = u * u[0].numel() ** 0.5 / norm
    assert torch.allclose(out[~keep], ref[~keep], rtol=1e-13)


def test_vjps_match_the_closed_forms():
    z, noise, grad, sigma, alpha, active = oracle.make_descent_inputs(4, 6, 24, dtype=torch.float64, seed=5)
    dy = torch.randn(z.shape, generator=torch.Generator().manual_seed(6), dtype=torch.float64)
    for nz, sg in ((None, None), (noise, None), (noise, sigma)):
        assert torch.allclose(oracle.vjp_noisy_point(z, nz, sg, dy, EPS), oracle.rms_norm_vjp(z, dy, EPS), rtol=1e-11)
    v = oracle.rms_norm(z, EPS)
    dv, dg, dz = oracle.vjp_step_and_project(v, grad, alpha, z, active, dy, EPS)
    a = active.view(-1)
    du = oracle.sphere_vjp(v - alpha * grad, dy, EPS)
    assert torch.allclose(dv[a], du[a], rtol=1e-11, atol=1e-14)
    assert torch.allclose(dg, -alpha * dv, rtol=1e-14)
    assert torch.equal(dv[~a], torch.zeros_like(dv[~a]))
    assert torch.equal(dz[~a], dy[~a]) and torch.equal(dz[a], torch.zeros_like(dz[a]))
    # the clamped branch: RMS below eps
    tiny = v * 1e-7
    dv2, _, dz2 = oracle.vjp_step_and_project(tiny, grad * 0, 0.1, z, None, dy, EPS)
    assert dz2 is None and torch.allclose(dv2, dy / EPS, rtol=1e-13)


def test_autograd_of_the_oracle_passes_gradcheck():
    z, noise, grad, sigma, alpha, active = oracle.make_descent_inputs(2, 3, 5, dtype=torch.float64, seed=7)
    zz = z.clone().requires_grad_(True)
    assert torch.autograd.gradcheck(lambda t: oracle.noisy_point(t, noise, sigma, EPS), (zz,))
    v = oracle.rms_norm(z, EPS).requires_grad_(True)
    gg = grad.clone().requires_grad_(True)
    assert torch.autograd.gradcheck(lambda a, b: oracle.step_and_project(a, b, alpha, z, active, EPS), (v, gg))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_harness_eager_wrapper_equals_the_oracle(dtype):
    z, noise, grad, sigma, alpha, active = oracle.make_descent_inputs(3, 9, 32, dtype=dtype, seed=8)
    s, a = sigma.to(dtype), alpha.to(dtype)
    assert torch.equal(layers.rms_norm(z, EPS), oracle.rms_norm(z, EPS))
    assert torch.equal(en._eager_noisy_point(z, noise, s, EPS), oracle.noisy_point(z, noise, s, EPS))
    assert torch.equal(en._eager_noisy_point(z, noise, None, EPS), oracle.noisy_point_replayed(z, noise, EPS))
    v = oracle.noisy_point(z, noise, s, EPS)
    assert torch.equal(en._eager_step_and_project(v, grad, a, z, active, EPS),
                       oracle.step_and_project(v, grad, a, z, active, EPS))
    assert torch.equal(en.sphere(v, EPS), oracle.sphere(v, EPS))


def test_descent_argument_checks():
    from ebr_amd import descent

    z = torch.zeros(2, 3, 8)
    with pytest.raises(ValueError):
        descent.normalize(torch.zeros(6, 8))  # not [B, L, C]
    with pytest.raises(ValueError):
        descent.noisy_point(z, torch.zeros(2, 3, 4), 0.1)  # noise shape
    with pytest.raises(TypeError):
        descent.noisy_point(z, z, torch.full((2, 1, 1), 0.1, dtype=torch.float64))  # sigma not in z's dtype
    with pytest.raises(ValueError):
        descent.step_and_project(z, z, torch.full((2, 3, 1), 0.1), z, None)  # alpha not per row
    with pytest.raises(ValueError):
        descent.step_and_project(z, z, 0.1, z, torch.ones(2, 3, 1, dtype=torch.bool))  # mask not per row
    with pytest.raises(NotImplementedError):
        descent.step_and_project(z, z, torch.full((2, 1, 1), 0.1, requires_grad=True), z, None)


def test_harness_eager_wrapper_gradient_equals_the_oracle():
    """In bf16 the reference's sphere reads its input through two casts, so autograd rounds the gradient's two terms
    separately; the harness's eager wrapper does the same (bit-exact), and a single-cast sphere would not."""
    z, noise, grad, sigma, alpha, active = oracle.make_descent_inputs(3, 9, 64, dtype=torch.bfloat16, seed=9)
    a = alpha.to(torch.bfloat16)
    v = oracle.noisy_point(z, noise, sigma.to(torch.bfloat16), EPS)
    dout = torch.randn(z.shape, generator=torch.Generator().manual_seed(10)).to(torch.bfloat16)
    rdv, rdg, rdz = oracle.vjp_step_and_project(v, grad, a, z, active, dout, EPS)
    vv, gg, zz = (t.clone().requires_grad_(True) for t in (v, grad, z))
    out = en._eager_step_and_project(vv, gg, a, zz, active, EPS)
    dv, dg, dz = torch.autograd.grad(out, (vv, gg, zz), dout)
    assert torch.equal(dv, rdv) and torch.equal(dg, rdg) and torch.equal(dz, rdz)

    def single_cast_sphere(t):
        tf = t.float()
        return (tf / tf.square().mean(dim=(1, 2), keepdim=True).sqrt().clamp_min(EPS)).to(t.dtype)

    uu = (v - a * grad).clone().requires_grad_(True)
    (d1,) = torch.autograd.grad(single_cast_sphere(uu), uu, dout)
    (d2,) = torch.autograd.grad(oracle.sphere(uu, EPS), uu, dout)
    assert not torch.equal(d1, d2)
