"""Host-side boundary on the CPU: the ebr_fused custom ops, their fakes, the autograd Functions, fused_attention, the
implementation selector and the second-order self-test (reference models/fused_attn/ops.py, loader.py and
models/attention.py:89-173).

On CPU tensors the ops run the package's dense path (``ebr_amd/fused_attn/dense.py``), as the reference's ops run its
dense functions there (ops.py:68-70); every value is compared with the CPU oracle or with torch autograd. Calls are
counted by wrapping the dense functions; the one planted mistake lives in a test-only attention backend built from
the oracle.
"""

import os

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import oracle
from ebr_amd import attention as att
from ebr_amd.fused_attn import dense, loader, ops

F64 = torch.float64


@pytest.fixture
def calls(monkeypatch):
    """Records every dense call the ops make (name and, for bwd_bwd, the cotangents' strides)."""
    seen = []

    def wrap(name, fn, strides=False):
        def run(*args):
            seen.append((name, tuple(a.stride() for a in args[6:9])) if strides else name)
            return fn(*args)

        return run

    monkeypatch.setattr(dense, "attn_fwd", wrap("fwd", dense.attn_fwd))
    monkeypatch.setattr(dense, "attn_bwd", wrap("bwd", dense.attn_bwd))
    monkeypatch.setattr(dense, "attn_bwd_bwd", wrap("bwd_bwd", dense.attn_bwd_bwd, strides=True))
    return seen


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


def test_none_cotangents_become_expanded_zero_rows(calls):
    q, k, v, do, gq, gk, gv = _inputs(seed=1)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    o = ops.fused_attention(qq, kk, vv)
    dq, dk, dv = torch.autograd.grad(o, (qq, kk, vv), do, create_graph=True)
    calls.clear()
    hq, hk = torch.autograd.grad((dq * gq).sum(), (qq, kk))  # gk, gv are None in the bwd node's backward
    bb = [c for c in calls if isinstance(c, tuple)]
    assert len(bb) == 1
    _, (sq, sk, sv) = bb[0]
    assert sk == (0, 0, 0, 1) and sv == (0, 0, 0, 1)  # one zero row expanded, no L x D memory
    z = torch.zeros_like(q)
    want = oracle.autograd_bwd_bwd(q, k, v, do, gq, z, z)
    assert torch.allclose(hq, want[0], atol=1e-11) and torch.allclose(hk, want[1], atol=1e-11)


def test_call_sequence_of_a_graded_microstep(calls):
    """fwd x1; first backward x1 (create_graph); outer backward: bwd_bwd x1 and attn_bwd once more (ops.py:131-185)."""
    q, k, v, do, gq, gk, gv = _inputs(seed=2)
    x = q.clone().requires_grad_(True)
    w = torch.randn(8, 8, dtype=F64, requires_grad=True)
    calls.clear()
    o = ops.fused_attention(x @ w, k, v)
    (g,) = torch.autograd.grad(o.sum(), x, create_graph=True)
    (g * gq).sum().backward()
    names = [c if isinstance(c, str) else c[0] for c in calls]
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


def test_launcher_argument_errors():
    """The launcher layer checks its arguments as reference triton_kernels._cfg does (TypeError for a dtype without
    kernels, ValueError for a tensor that is not 4-D or an unknown input_precision), and takes GPU tensors only; all
    of it before any launch."""
    from ebr_amd.fused_attn import kernels

    q = torch.zeros(1, 2, 3, 8)
    with pytest.raises(TypeError):
        kernels.attn_fwd(q.to(torch.int32), q, q, 0.5)
    with pytest.raises(ValueError):
        kernels.attn_fwd(q[0], q[0], q[0], 0.5)
    with pytest.raises(ValueError, match="input_precision"):
        kernels.attn_bwd(q, q, q, q, q[..., 0], q, 0.5, input_precision="fp16")
    for prec in kernels.PRECISIONS + (None,):
        with pytest.raises(ValueError, match="GPU tensors"):  # every name the reference accepts passes the check
            kernels.attn_bwd_bwd(q, q, q, q, q[..., 0], q, None, None, None, None, 0.5, input_precision=prec)


def test_plan_override_keys_and_values(monkeypatch):
    """PLAN_OVERRIDE takes the reference's keys and values (triton_kernels.py:610-615): block-shape tuples are
    accepted and select nothing, the modes 'single' and 'two' map onto this library's one-launch and streamed
    families, 'atomic' raises; this library's family names work on the three selecting keys. Anything else raises
    ValueError before any other check or launch."""
    from ebr_amd import _capi
    from ebr_amd.fused_attn import kernels

    q = torch.zeros(1, 2, 3, 8)
    monkeypatch.setattr(kernels, "PLAN_OVERRIDE", {"bob_tile": (16, 16, 4, 1)})
    with pytest.raises(ValueError, match="not a plan key"):
        kernels.attn_fwd(q, q, q, 0.5)
    for bad in ({"bob_row": (16, 16, 4)}, {"bwd_col": "long"}, {"fwd": "two"}, {"bob_mode": (64, 32, 4, 3)},
                {"bwd_dq": (16, 16, 4, 0)}, {"bwd_mode": "fast"}):
        monkeypatch.setattr(kernels, "PLAN_OVERRIDE", bad)
        with pytest.raises(ValueError, match="names no kernel family"):
            kernels.attn_bwd(q, q, q, q, q[..., 0], q, 0.5)
    monkeypatch.setattr(kernels, "PLAN_OVERRIDE", {"bwd_mode": "atomic"})
    with pytest.raises(ValueError, match="atomic"):
        kernels.attn_bwd(q, q, q, q, q[..., 0], q, 0.5)
    monkeypatch.setattr(kernels, "PLAN_OVERRIDE", {"fwd": "long", "bwd_mode": "resident", "bob_mode": "auto"})
    assert (kernels._plan("fwd"), kernels._plan("bwd_mode"), kernels._plan("bob_mode")) == (4, 2, 0)
    # the reference's own default plans for bf16 at N = 81 (triton_kernels.py:641-652) and at N = 900
    ref81 = dict(fwd=(64, 32, 4, 3), bwd_mode="single", bwd_single=(32, 128, 4, 1), bwd_col=(64, 64, 4, 3),
                 bwd_dq=(64, 32, 4, 3), bob_mode="single", bob_single=(16, 128, 4, 1), bob_row=(64, 32, 4, 3),
                 bob_col=(64, 64, 4, 2))
    monkeypatch.setattr(kernels, "PLAN_OVERRIDE", ref81)
    assert [kernels._plan(k, 81) for k in ("fwd", "bwd_mode", "bob_mode")] == [_capi.PLAN_AUTO] * 3
    with pytest.raises(ValueError, match="one-launch"):
        kernels._plan("bob_mode", 900)
    monkeypatch.setattr(kernels, "PLAN_OVERRIDE", dict(ref81, fwd=(64, 64, 4, 3), bwd_mode="two", bob_mode="two"))
    assert [kernels._plan(k, 900) for k in ("fwd", "bwd_mode", "bob_mode")] == [_capi.PLAN_AUTO] * 3
    assert [kernels._plan(k, 81) for k in ("bwd_mode", "bob_mode")] == [_capi.PLAN_GENERIC] * 2
    # above D = 128 every shape takes the two streamed launches: "two" is the library's choice, "single" has no plan
    assert [kernels._plan(k, 81, 256) for k in ("bwd_mode", "bob_mode")] == [_capi.PLAN_AUTO] * 2
    monkeypatch.setattr(kernels, "PLAN_OVERRIDE", ref81)
    with pytest.raises(ValueError, match="one-launch"):
        kernels._plan("bwd_mode", 81, 192)
    with pytest.raises(ValueError, match="GPU tensors"):  # a valid dictionary reaches the usual checks
        kernels.attn_fwd(q, q, q, 0.5)


def test_rows_keeps_aligned_views_and_copies_others():
    x = torch.zeros(2, 5, 3, 4, 64, dtype=torch.bfloat16)  # [B, L, 3, H, D] projection
    q = x[:, :, 0].transpose(1, 2)
    assert ops._rows(q) is q
    odd = torch.zeros(2, 3, 5, 65, dtype=torch.bfloat16)[..., :64]  # row stride 65 elements: not 16-byte aligned
    assert ops._rows(odd) is not odd and ops._rows(odd).is_contiguous()
    odd64 = torch.zeros(2, 3, 5, 65, dtype=torch.float64)[..., :64]  # fp64 needs element alignment only
    assert ops._rows(odd64) is odd64


def test_loader_modes_and_routing(monkeypatch):
    monkeypatch.setenv("EBR_FUSED_ATTN_IMPL", "bogus")
    with pytest.raises(ValueError):
        loader.mode()
    for m in ("auto", "hip", "triton"):
        monkeypatch.setenv("EBR_FUSED_ATTN_IMPL", m)
        assert ops.route("cpu") == "reference" and ops.route("cuda") == "hip"
    monkeypatch.setenv("EBR_FUSED_ATTN_IMPL", "reference")
    assert ops.route("cpu") == "reference" and ops.route("cuda") == "reference"
    assert ops.implementation("cuda") == "reference"
    from ebr_amd import _capi

    monkeypatch.setattr(_capi, "_LIB", None)
    monkeypatch.setattr(_capi, "LIB_PATH", _capi.LIB_PATH.with_name("missing_lib.so"))
    monkeypatch.setenv("EBR_FUSED_ATTN_IMPL", "auto")
    with pytest.raises(RuntimeError, match="unavailable"):
        loader.hip_library()
    assert ops.implementation("cpu") == "reference"
    assert ops.implementation("cuda") == "unavailable"  # a GPU call would raise, never fall back


def test_cpu_tensors_run_the_dense_path_and_equal_the_oracle():
    """fused_attention's ops on CPU tensors (reference ops.py:68-70) against the oracle, in every dtype, with views."""
    for dt, tol in ((F64, 1e-13), (torch.float32, 1e-6), (torch.bfloat16, 1e-2), (torch.float16, 2e-3)):
        q, k, v, do, gq, gk, gv = oracle.make_inputs(2, 3, 21, 24, dtype=dt, seed=11, qkv_scale=0.5)
        qv = torch.cat([q, q], dim=-1)[..., :24]  # a strided view
        s = 24**-0.5
        o, lse = ops.attn_fwd(qv, k, v, s)
        assert lse.dtype == ops.lse_dtype_for(q) and o.dtype == dt and o.is_contiguous()
        ref_o, ref_lse = oracle.attn_fwd(q, k, v, s)
        assert oracle.rel_err(o, ref_o) <= tol and oracle.rel_err(lse, ref_lse) <= tol
        d = ops.attn_bwd(qv, k, v, o, lse, do, s)
        for got, ref in zip(d, oracle.attn_bwd(q, k, v, o, lse, do, s)):
            assert got.dtype == dt and oracle.rel_err(got, ref) <= tol
        h = ops.attn_bwd_bwd(qv, k, v, o, lse, do, d[0], gq, gk, gv, s)
        for got, ref in zip(h, oracle.attn_bwd_bwd(q, k, v, o, lse, do, None, gq, gk, gv, s)):
            assert got.dtype == dt and oracle.rel_err(got, ref) <= tol


def test_dense_path_groups_long_sequences_without_changing_values(monkeypatch):
    q, k, v, do, gq, gk, gv = _inputs(B=2, H=3, L=33, D=8, seed=12)
    s = 0.4
    whole = [ops.attn_fwd(q, k, v, s)]
    monkeypatch.setattr(dense, "_GROUP_ELEMS", 33 * 33 * 2)  # two (b, h) slices per group: 3 groups
    grouped = [ops.attn_fwd(q, k, v, s)]
    for a, b in zip(whole[0], grouped[0]):
        assert torch.equal(a, b)
    o, lse = whole[0]
    h = ops.attn_bwd_bwd(q, k, v, o, lse, do, do, gq, gk, gv, s)
    for got, ref in zip(h, oracle.attn_bwd_bwd(q, k, v, o, lse, do, None, gq, gk, gv, s)):
        assert oracle.rel_err(got, ref) <= 1e-13


def test_kernel_head_dims_pad_to_the_row_vector():
    assert ops.kernel_head_dim(torch.bfloat16, 64) == 64 and ops.kernel_head_dim(torch.bfloat16, 20) == 24
    assert ops.kernel_head_dim(torch.float16, 1) == 8 and ops.kernel_head_dim(torch.float32, 36) == 36
    assert ops.kernel_head_dim(torch.float32, 37) == 40 and ops.kernel_head_dim(F64, 37) == 37
    assert ops.kernel_head_dim(torch.bfloat16, 121) == 128
    assert ops.kernel_head_dim(torch.bfloat16, 129) == 136 and ops.kernel_head_dim(torch.float32, 255) == 256
    with pytest.raises(ValueError):
        ops.kernel_head_dim(torch.bfloat16, 257)
    assert ops.kernel_head_dim(F64, 129) == 129
    with pytest.raises(ValueError):
        ops.kernel_head_dim(F64, 257)


def test_zero_head_columns_change_nothing():
    """The padding identity the GPU path relies on, on the oracle: zero columns appended to q, k, v, dO and the
    cotangents leave every score unchanged and give zero output columns."""
    q, k, v, do, gq, gk, gv = _inputs(B=1, H=2, L=7, D=5, seed=13)
    s = 5**-0.5
    pad = lambda t: torch.nn.functional.pad(t, (0, 3))  # noqa: E731
    o, lse = oracle.attn_fwd(q, k, v, s)
    op, lsep = oracle.attn_fwd(pad(q), pad(k), pad(v), s)
    assert torch.allclose(op[..., :5], o, atol=1e-15) and op[..., 5:].abs().max() == 0
    assert torch.allclose(lsep, lse, atol=1e-15)
    h = oracle.attn_bwd_bwd(q, k, v, o, lse, do, None, gq, gk, gv, s)
    hp = oracle.attn_bwd_bwd(*(pad(t) for t in (q, k, v)), pad(o), lse, pad(do), None,
                             *(pad(t) for t in (gq, gk, gv)), s)
    for a, b in zip(h, hp):
        assert torch.allclose(b[..., :5], a, atol=1e-14) and b[..., 5:].abs().max() == 0


class _PlantedBwd(torch.autograd.Function):
    """Oracle first derivative whose own derivative has hQ 10% too small: a backend with a planted mistake."""

    @staticmethod
    def forward(ctx, q, k, v, o, lse, do):
        ctx.save_for_backward(q, k, v, o, lse, do)
        return oracle.attn_bwd(q, k, v, o, lse, do, q.shape[-1] ** -0.5)

    @staticmethod
    def backward(ctx, gq, gk, gv):
        q, k, v, o, lse, do = ctx.saved_tensors
        z = torch.zeros_like(q)
        gq, gk, gv = (z if g is None else g for g in (gq, gk, gv))
        hq, hk, hv, hdo = oracle.attn_bwd_bwd(q, k, v, o, lse, do, None, gq, gk, gv, q.shape[-1] ** -0.5)
        return 0.9 * hq, hk, hv, None, None, hdo


class _PlantedAttn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v):
        o, lse = oracle.attn_fwd(q, k, v, q.shape[-1] ** -0.5)
        ctx.save_for_backward(q, k, v, o, lse)
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        return _PlantedBwd.apply(q, k, v, o, lse, do)


def test_verify_second_order_passes_and_catches_planted_mistake():
    att.verify_second_order(att.get_backend("fused"), device=torch.device("cpu"))
    planted = att.AttentionBackend("planted", _PlantedAttn.apply, True)
    with pytest.raises(att.SecondOrderUnsafeError, match="d2E/dz2"):
        att.verify_second_order(planted, device=torch.device("cpu"))


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


def test_package_does_not_import_the_oracle():
    """The dense path is the package's own code; the oracle stays test infrastructure."""
    import inspect

    for mod in (ops, dense, loader, att):
        assert "oracle" not in inspect.getsource(mod).replace("oracle/", "")
    assert os.path.basename(ops.__file__) == "ops.py"
