"""Host-side boundary on the CPU: the ebr_fused custom ops, their fakes, the autograd Functions, fused_attention, the
implementation selector and the second-order self-test (reference models/fused_attn/ops.py, loader.py and
models/attention.py:89-173).

The shipped ops have a HIP kernel only. These tests register a test-local CPU kernel for them that wraps the CPU
oracle (with a switch that plants a mistake), so the wiring can be exercised without a GPU. The CPU kernel never ships:
it exists only inside this test module.
"""

import os

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import oracle
from ebr_amd import attention as att
from ebr_amd.fused_attn import loader, ops

F64 = torch.float64
PLANT = {"bwd_bwd_scale": 1.0, "detach": False, "calls": []}


def _cpu_fwd(q, k, v, scale):
    PLANT["calls"].append("fwd")
    o, lse = oracle.attn_fwd(q, k, v, scale)
    return o.contiguous(), lse.to(ops.lse_dtype_for(q)).contiguous()


def _cpu_bwd(q, k, v, o, lse, do, scale):
    PLANT["calls"].append("bwd")
    dq, dk, dv = oracle.attn_bwd(q, k, v, o, lse, do, scale)
    return dq.contiguous(), dk.contiguous(), dv.contiguous()


def _cpu_bwd_bwd(q, k, v, o, lse, do, dq, gq, gk, gv, scale):
    PLANT["calls"].append(("bwd_bwd", gq.stride(), gk.stride(), gv.stride()))
    hq, hk, hv, hdo = oracle.attn_bwd_bwd(q, k, v, o, lse, do, dq, gq, gk, gv, scale)
    f = PLANT["bwd_bwd_scale"]
    return (hq * f).contiguous(), hk.contiguous(), hv.contiguous(), hdo.contiguous()


_REGISTERED = False


@pytest.fixture(scope="module", autouse=True)
def cpu_kernels():
    global _REGISTERED
    if not _REGISTERED:
        ops.attn_fwd.register_kernel("cpu")(_cpu_fwd)
        ops.attn_bwd.register_kernel("cpu")(_cpu_bwd)
        ops.attn_bwd_bwd.register_kernel("cpu")(_cpu_bwd_bwd)
        _REGISTERED = True
    yield


@pytest.fixture(autouse=True)
def reset_plant():
    PLANT.update(bwd_bwd_scale=1.0, detach=False, calls=[])
    yield
    PLANT.update(bwd_bwd_scale=1.0, detach=False, calls=[])


def _inputs(B=2, H=2, L=9, D=8, dtype=F64, seed=0):
    return oracle.make_inputs(B, H, L, D, dtype=dtype, seed=seed, qkv_scale=0.6)


def test_fused_attention_matches_eager_to_second_order():
    q, k, v, do, gq, gk, gv = _inputs()
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    dd = do.clone().requires_grad_(True)
    o = ops.fused_attention(qq, kk, vv)
    assert torch.allclose(o, oracle.math_attention(q, k, v), atol=1e-12)
    dq, dk, dv = torch.autograd.grad(o, (qq, kk, vv), dd, create_graph=True)
    phi = (dq * gq).sum() + (dk * gk).sum() + (dv * gv).sum()
    got = torch.autograd.grad(phi, (qq, kk, vv, dd))
    want = oracle.autograd_bwd_bwd(q, k, v, do, gq, gk, gv)
    for g_, w_ in zip(got, want):
        assert torch.allclose(g_, w_, atol=1e-11)
    first = oracle.autograd_bwd(q, k, v, do)
    for g_, w_ in zip((dq, dk, dv), first):
        assert torch.allclose(g_, w_, atol=1e-11)


def test_none_cotangents_become_expanded_zero_rows():
    q, k, v, do, gq, gk, gv = _inputs(seed=1)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    o = ops.fused_attention(qq, kk, vv)
    dq, dk, dv = torch.autograd.grad(o, (qq, kk, vv), do, create_graph=True)
    PLANT["calls"].clear()
    hq, hk = torch.autograd.grad((dq * gq).sum(), (qq, kk))  # gk, gv are None in the bwd node's backward
    bb = [c for c in PLANT["calls"] if isinstance(c, tuple)]
    assert len(bb) == 1
    _, sq, sk, sv = bb[0]
    assert sk == (0, 0, 0, 1) and sv == (0, 0, 0, 1)  # one zero row expanded, no L x D memory
    z = torch.zeros_like(q)
    want = oracle.autograd_bwd_bwd(q, k, v, do, gq, z, z)
    assert torch.allclose(hq, want[0], atol=1e-11) and torch.allclose(hk, want[1], atol=1e-11)


def test_call_sequence_of_a_graded_microstep():
    """fwd x1; first backward x1 (create_graph); outer backward: bwd_bwd x1 and attn_bwd once more (ops.py:131-185)."""
    q, k, v, do, gq, gk, gv = _inputs(seed=2)
    x = q.clone().requires_grad_(True)
    w = torch.randn(8, 8, dtype=F64, requires_grad=True)
    PLANT["calls"].clear()
    o = ops.fused_attention(x @ w, k, v)
    (g,) = torch.autograd.grad(o.sum(), x, create_graph=True)
    (g * gq).sum().backward()
    names = [c if isinstance(c, str) else c[0] for c in PLANT["calls"]]
    assert names.count("fwd") == 1 and names.count("bwd") == 2 and names.count("bwd_bwd") == 1
    assert w.grad is not None


def test_lse_not_differentiable_and_outputs_fresh():
    q, k, v, *_ = _inputs(seed=3)
    o, lse = ops._FusedAttn.apply(q.clone().requires_grad_(True), k, v, 0.3)
    assert o.requires_grad and not lse.requires_grad
    assert o.is_contiguous() and lse.dtype == F64


def test_torch_func_grad_then_autograd():
    """The reference's compiled-energy pattern (models/energy.py:371-434): dE/dz through torch.func.grad, then the
    second derivative through torch.autograd.grad on its result."""
    q, k, v, *_ = _inputs(seed=4)

    def probe(attn):
        z = q.clone().requires_grad_(True)
        g = torch.func.grad(lambda zz: attn(zz, k, v).pow(2).sum())(z)
        (hz,) = torch.autograd.grad((g * v).sum(), z)
        return g.detach(), hz

    g, hz = probe(ops.fused_attention)
    g_ref, hz_ref = probe(lambda a, b, c: oracle.math_attention(a, b, c))
    assert torch.allclose(g, g_ref, atol=1e-11) and torch.allclose(hz, hz_ref, atol=1e-10)


def test_torch_compile_aot_eager():
    q, k, v, do, *_ = _inputs(seed=5)

    def f(q, k, v):
        return ops.fused_attention(q, k, v) * 2.0

    cf = torch.compile(f, backend="aot_eager", fullgraph=True)
    qq = q.clone().requires_grad_(True)
    out = cf(qq, k, v)
    (gq,) = torch.autograd.grad(out, qq, do)
    want = oracle.autograd_bwd(q, k, v, 2.0 * do)[0]
    assert torch.allclose(out, 2.0 * oracle.math_attention(q, k, v), atol=1e-12)
    assert torch.allclose(gq, want, atol=1e-11)


def test_fakes_match_contract():
    with FakeTensorMode():
        q = torch.empty(2, 3, 81, 64, dtype=torch.bfloat16).transpose(1, 2).transpose(1, 2)
        o, lse = ops.attn_fwd(q, q, q, 0.125)
        assert o.shape == q.shape and o.is_contiguous() and o.dtype == torch.bfloat16
        assert lse.shape == (2, 3, 81) and lse.dtype == torch.float32
        dq, dk, dv = ops.attn_bwd(q, q, q, o, lse, q, 0.125)
        assert all(t.shape == q.shape and t.is_contiguous() for t in (dq, dk, dv))
        hs = ops.attn_bwd_bwd(q, q, q, o, lse, q, dq, q, q, q, 0.125)
        assert len(hs) == 4 and all(t.shape == q.shape for t in hs)


def test_argument_errors():
    q = torch.zeros(1, 2, 3, 8)
    with pytest.raises(ValueError):
        ops._check(q, q[:, :, :2], q)
    with pytest.raises(ValueError):
        ops._check(q, q.double(), q)
    with pytest.raises(ValueError):
        ops._check(q[0], q[0], q[0])
    with pytest.raises(TypeError):
        ops._dtype_code(q.to(torch.int32))
    assert ops._dtype_code(q.double()) == 3  # fp64 has kernels of its own
    ops._check_like(q, o=q, lse=q[..., 0], do=q)
    with pytest.raises(ValueError):
        ops._check_like(q, o=q[:, :1])  # o is read by q's sizes
    with pytest.raises(ValueError):
        ops._check_like(q, lse=q)  # lse is [B, H, N]
    with pytest.raises(ValueError):
        ops._check_like(q, gk=q[..., :4])
    assert ops.default_scale(q, None) == 8**-0.5 and ops.default_scale(q, 0.3) == 0.3


def test_rows_keeps_aligned_views_and_copies_others():
    x = torch.zeros(2, 5, 3, 4, 64, dtype=torch.bfloat16)  # [B, L, 3, H, D] projection
    q = x[:, :, 0].transpose(1, 2)
    assert ops._rows(q) is q
    odd = torch.zeros(2, 3, 5, 65, dtype=torch.bfloat16)[..., :64]  # row stride 65 elements: not 16-byte aligned
    assert ops._rows(odd) is not odd and ops._rows(odd).is_contiguous()
    odd64 = torch.zeros(2, 3, 5, 65, dtype=torch.float64)[..., :64]  # fp64 needs element alignment only
    assert ops._rows(odd64) is odd64


def test_loader_modes(monkeypatch):
    monkeypatch.setenv("EBR_FUSED_ATTN_IMPL", "reference")
    with pytest.raises(RuntimeError, match="no dense"):
        loader.hip_library()
    monkeypatch.setenv("EBR_FUSED_ATTN_IMPL", "bogus")
    with pytest.raises(ValueError):
        loader.mode()
    monkeypatch.setenv("EBR_FUSED_ATTN_IMPL", "triton")
    assert loader.mode() == "triton"
    from ebr_amd import _capi

    monkeypatch.setattr(_capi, "_LIB", None)
    monkeypatch.setattr(_capi, "LIB_PATH", _capi.LIB_PATH.with_name("missing_lib.so"))
    monkeypatch.setenv("EBR_FUSED_ATTN_IMPL", "auto")
    with pytest.raises(RuntimeError, match="unavailable"):
        loader.hip_library()
    assert ops.implementation("cpu") == "none"
    assert ops.implementation("cuda") == "none"


def test_verify_second_order_passes_and_catches_planted_mistake():
    backend = att.get_backend("fused")
    att.verify_second_order(backend, device=torch.device("cpu"))
    PLANT["bwd_bwd_scale"] = 0.9  # hQ off by 10%
    with pytest.raises(att.SecondOrderUnsafeError, match="does NOT carry second order"):
        att.verify_second_order(backend, device=torch.device("cpu"))


def test_verify_second_order_rejects_backend_without_second_derivative():
    def detached(q, k, v):
        o = oracle.math_attention(q, k, v)
        return o.detach() + (q - q.detach()).sum() * 0  # first order is wrong too: caught either way

    bad = att.AttentionBackend("bad", detached, True)
    with pytest.raises(att.SecondOrderUnsafeError):
        att.verify_second_order(bad, device=torch.device("cpu"))


def test_self_test_priming_keeps_the_global_rng_and_seeding_reaches_every_layer():
    """prime_attention_self_test runs each layer's self-test once under a forked RNG (the caller's next draw is
    unchanged); seed_attention_self_test sets the seed the pending self-tests will use."""
    from ebr_amd import energy as en

    cfg = en.EnergyConfig(hidden_size=32, num_heads=2, num_layers=2, grid=(3, 3), attn_backend="math",
                          attn_nograd_backend="math")
    model, _ = en.build(cfg, torch.device("cpu"), seed=1)
    layers = [m for m in model.modules() if isinstance(m, att.EnergyAttention)]
    assert len(layers) == 2
    att.seed_attention_self_test(model, 1234)
    assert all(m.self_test_seed == 1234 for m in layers)
    torch.manual_seed(7)
    expected = torch.rand(3)
    torch.manual_seed(7)
    att.prime_attention_self_test(model)
    assert all(m._verified for m in layers)
    assert torch.equal(torch.rand(3), expected)


def test_backend_registry_and_tier_flag():
    assert set(att.ATTENTION_BACKENDS) == {"math", "sdpa_auto", "fused"}
    assert att.get_backend("fused").second_order and not att.get_backend("sdpa_auto").second_order
    with pytest.raises(ValueError):
        att.get_backend("nope")
    assert not att.second_order_required()
    with att.second_order_window(True):
        assert att.second_order_required()
        with att.second_order_window(False):
            assert not att.second_order_required()
        assert att.second_order_required()
    assert not att.second_order_required()
    with pytest.raises(att.SecondOrderUnsafeError):
        att.EnergyAttention(64, 16, 4, backend="sdpa_auto", nograd_backend="sdpa_auto")


def test_energy_attention_fused_equals_math_on_cpu():
    torch.manual_seed(0)
    m_fused = att.EnergyAttention(32, 8, 4, backend="fused", nograd_backend="math").double()
    m_math = att.EnergyAttention(32, 8, 4, backend="math", nograd_backend="math").double()
    m_math.load_state_dict(m_fused.state_dict())
    x = torch.randn(2, 9, 32, dtype=F64, requires_grad=True)
    with att.second_order_window(True):
        y1 = m_fused(None, x)
        y2 = m_math(None, x)
    assert torch.allclose(y1, y2, atol=1e-12)
    assert m_fused._verified
    (g1,) = torch.autograd.grad(y1.pow(2).sum(), x, create_graph=True)
    (g2,) = torch.autograd.grad(y2.pow(2).sum(), x, create_graph=True)
    h1 = torch.autograd.grad(g1.sum(), list(m_fused.parameters()))
    h2 = torch.autograd.grad(g2.sum(), list(m_math.parameters()))
    for a, b in zip(h1, h2):
        assert torch.allclose(a, b, atol=1e-10)


def test_hip_ops_have_no_cpu_kernel_in_the_package():
    """The package registers the ops for the HIP device only; this module's CPU kernel is a test double."""
    import inspect

    src = inspect.getsource(ops)
    assert 'device_types="cuda"' in src and "oracle" not in src
    assert os.path.basename(ops.__file__) == "ops.py"
