"""GPU parity of the fused 2D-RoPE split and merge (``ebr_fused::rope_split`` / ``rope_merge``, HIP kernels through the
C ABI) against the CPU oracle ``oracle.rope_ref``.

Both kernels compute in fp32 with the same separately rounded products and sums as the dense formula and round once
to the dtype, so the outputs are bit-identical to the oracle's for fp32, bf16 and fp16.
"""

import pytest
import torch

import oracle
from ebr_amd import energy as en
from ebr_amd.fused_attn import ops  # noqa: F401
from ebr_amd.fused_attn import rope_split as rs

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _tables(D, N):
    h, w = oracle.grid_shape(N)
    return oracle.rotary_tables(D, h, w)


def _say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,N,H,D", [(2, 81, 8, 64), (3, 100, 4, 32), (1, 1, 2, 16), (2, 30, 3, 12), (2, 9, 2, 128), (1, 20, 1, 4)])
@pytest.mark.parametrize("with_qscale", [False, True])
def test_split_and_merge_match_oracle_exactly(cuda, dtype, B, N, H, D, with_qscale):
    _say(f"rope B={B} N={N} H={H} D={D} {dtype} qscale={with_qscale}")
    qkv, (gq, gk, gv) = oracle.make_rope_inputs(B, N, H, D, dtype=dtype, seed=N + D)
    cos, sin = _tables(D, N)
    qs = torch.linspace(0.5, 1.5, H) if with_qscale else torch.zeros(0)
    q, k, v = torch.ops.ebr_fused.rope_split(qkv.to(cuda), cos.to(cuda), sin.to(cuda), qs.to(cuda), H)
    rq, rk, rv = oracle.ref_split(qkv, cos, sin, H, qs if with_qscale else None)
    for name, a, r in (("q", q, rq), ("k", k, rk), ("v", v, rv)):
        assert a.shape == r.shape and a.dtype == r.dtype and a.is_contiguous()
        assert torch.equal(a.cpu(), r), f"split {name}: max diff {(a.cpu().double() - r.double()).abs().max()}"
    g = torch.ops.ebr_fused.rope_merge(gq.to(cuda), gk.to(cuda), gv.to(cuda), cos.to(cuda), sin.to(cuda), qs.to(cuda))
    rg = oracle.ref_merge(gq, gk, gv, cos, sin, qs if with_qscale else None)
    assert g.shape == rg.shape and torch.equal(g.cpu(), rg), f"merge: max diff {(g.cpu().double() - rg.double()).abs().max()}"


def test_strided_inputs(cuda):
    """qkv with a padded row (stride(1) > 3*H*D) and odd batch stride, cotangents as transposed [B, N, H, D] views."""
    B, N, H, D = 2, 81, 4, 64
    _say("rope strided")
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(4)
    buf = torch.randn(B, N, 3 * H * D + 40, generator=g).to(dtype)
    qkv = buf[:, :, 8 : 8 + 3 * H * D]  # 16-byte offset row starts, row stride 3*H*D + 40
    cos, sin = _tables(D, N)
    q, k, v = torch.ops.ebr_fused.rope_split(qkv.to(cuda), cos.to(cuda), sin.to(cuda), torch.zeros(0, device=cuda), H)
    rq, rk, rv = oracle.ref_split(qkv.contiguous(), cos, sin, H)
    assert torch.equal(q.cpu(), rq) and torch.equal(k.cpu(), rk) and torch.equal(v.cpu(), rv)
    gq, gk, gv = (torch.randn(B, N, H, D, generator=g).to(dtype) for _ in range(3))
    views = [t.to(cuda).transpose(1, 2) for t in (gq, gk, gv)]
    assert not views[0].is_contiguous()
    out = torch.ops.ebr_fused.rope_merge(*views, cos.to(cuda), sin.to(cuda), torch.zeros(0, device=cuda))
    ref = oracle.ref_merge(*(t.transpose(1, 2) for t in (gq, gk, gv)), cos, sin)
    assert torch.equal(out.cpu(), ref)


def test_odd_alignment_takes_narrow_vectors(cuda):
    """A qkv view starting 2 bytes into its buffer: only 1-element accesses are aligned, and results do not change."""
    B, N, H, D = 1, 16, 2, 32
    _say("rope 2-byte aligned")
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(8)
    buf = torch.randn(B, N * (3 * H * D) + 1, generator=g).to(dtype).to(cuda)
    qkv = buf[:, 1:].reshape(B, N, 3 * H * D)
    cos, sin = _tables(D, N)
    q, k, v = torch.ops.ebr_fused.rope_split(qkv, cos.to(cuda), sin.to(cuda), torch.zeros(0, device=cuda), H)
    rq, rk, rv = oracle.ref_split(qkv.cpu(), cos, sin, H)
    assert torch.equal(q.cpu(), rq) and torch.equal(k.cpu(), rk) and torch.equal(v.cpu(), rv)


def test_autograd_first_and_second_order(cuda):
    """rope_split through autograd (its backward is the merge, the merge's backward the split), to second order,
    against autograd through the dense oracle in fp32."""
    B, N, H, D = 2, 25, 2, 16
    _say("rope autograd")
    qkv, (gq, gk, gv) = oracle.make_rope_inputs(B, N, H, D, dtype=torch.float32, seed=9)
    cos, sin = _tables(D, N)

    def run(split, x, c, s, w):
        # quadratic in the outputs, so the first derivative depends on x and the second goes through the merge's
        # backward (the split)
        x = x.clone().requires_grad_(True)
        q, k, v = split(x, c, s)
        loss = (q * q * w[0]).sum() + (k * w[1]).sum() + (v * v * w[2]).sum()
        (g1,) = torch.autograd.grad(loss, x, create_graph=True)
        (g2,) = torch.autograd.grad((g1 * w[3]).sum(), x)
        return g1.detach(), g2

    u = torch.randn(qkv.shape, generator=torch.Generator().manual_seed(10))
    w = (gq, gk, gv, u)
    g1, g2 = run(lambda x, c, s: rs.rope_split(x, c, s, H), qkv.to(cuda), cos.to(cuda), sin.to(cuda),
                 tuple(t.to(cuda) for t in w))
    r1, r2 = run(lambda x, c, s: oracle.ref_split(x, c, s, H), qkv, cos, sin, w)
    assert torch.allclose(g1.cpu(), r1, atol=1e-6, rtol=1e-6)
    assert torch.allclose(g2.cpu(), r2, atol=1e-6, rtol=1e-6)


def test_missing_cotangents(cuda):
    """Only q is used downstream: the backward reads stride-0 zero rows for k and v."""
    B, N, H, D = 1, 9, 2, 16
    qkv, (gq, _, _) = oracle.make_rope_inputs(B, N, H, D, dtype=torch.float32, seed=2)
    cos, sin = _tables(D, N)
    x = qkv.to(cuda).requires_grad_(True)
    q, k, v = rs.rope_split(x, cos.to(cuda), sin.to(cuda), H)
    (g,) = torch.autograd.grad((q * gq.to(cuda)).sum(), x)
    ref = oracle.ref_merge(gq, torch.zeros_like(gq), torch.zeros_like(gq), cos, sin)
    assert torch.allclose(g.cpu(), ref, atol=1e-6)


def test_energy_fused_rope_matches_broadcast(cuda):
    """The energy network with rope_impl = "fused" gives the same energy and graded training step as with the
    broadcast RoPE (fp32), and the no-grad tier with the kernel-applied temperature the same descent."""
    _say("energy fused rope")
    models = []
    for impl in ("fused", "broadcast"):
        cfg = en.EnergyConfig(hidden_size=64, num_heads=4, grid=(4, 4), rope_impl=impl)
        models.append(en.build(cfg, cuda, seed=12))
    g = torch.Generator("cpu").manual_seed(13)
    B, L = 3, 16
    x = torch.randint(0, 11, (B, L), generator=g).to(cuda)
    z0 = torch.randn(B, L, 64, generator=g).to(cuda)
    tg = torch.randint(0, 11, (B, L), generator=g).to(cuda)
    with torch.no_grad():
        for m, _ in models:
            m.layers[0].self_attn.log_logit_scale.copy_(torch.tensor([0.1, -0.2, 0.3, 0.0]))
    losses = [float(en.train_step(m, d, x, z0, tg, steps=2)) for m, d in models]
    assert abs(losses[0] - losses[1]) <= 1e-5 * max(1.0, abs(losses[1]))
    (mf, _), (mb, _) = models
    for (n, pf), (_, pb) in zip(mf.named_parameters(), mb.named_parameters()):
        if pb.grad is not None:
            err = float((pf.grad - pb.grad).abs().max() / pb.grad.abs().max().clamp_min(1e-12))
            assert err <= 1e-4, (n, err)
    xe = mf.puzzle_embedding(x, z0.dtype).detach()
    vf = en.descend(mf, z0, xe, 3, 0.1, create_graph=False).detach()
    vb = en.descend(mb, z0, xe, 3, 0.1, create_graph=False).detach()
    assert float((vf - vb).abs().max()) <= 1e-4 * float(vb.abs().max())


def test_raw_ops_check_operands(cuda):
    """The C ABI takes only the sizes of qkv (split) or dq (merge); the raw ops check every other operand first."""
    cos = torch.zeros(9, 16, device=cuda)
    qkv = torch.zeros(2, 9, 96, device=cuda, dtype=torch.bfloat16)
    none = torch.zeros(0, device=cuda)
    with pytest.raises(ValueError):
        torch.ops.ebr_fused.rope_split(qkv, cos[:8], cos[:8], none, 2)
    with pytest.raises(ValueError):
        torch.ops.ebr_fused.rope_split(qkv, cos, cos, torch.ones(5, device=cuda), 2)
    dq = torch.zeros(2, 2, 9, 16, device=cuda, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        torch.ops.ebr_fused.rope_merge(dq, dq[:, :1], dq, cos, cos, none)
    with pytest.raises(ValueError):
        torch.ops.ebr_fused.rope_merge(dq, dq, dq, cos[:, :8], cos[:, :8], none)


def test_fp64_on_the_gpu_runs_the_dense_functions_to_second_order(cuda):
    """fp64 GPU tensors (gradcheck) go to the dense functions, which the reference's kernel check does too
    (rope_split.py:18-19): values equal the oracle's, and gradcheck / gradgradcheck pass on the device."""
    _say("rope fp64 on the GPU: dense path, gradcheck and gradgradcheck")
    qkv, (gq, gk, gv) = oracle.make_rope_inputs(1, 6, 2, 8, dtype=torch.float64, seed=6)
    cos, sin = (t.double() for t in _tables(8, 6))
    got = rs.rope_split(qkv.to(cuda), cos.to(cuda), sin.to(cuda), 2)
    want = oracle.ref_split(qkv, cos, sin, 2)
    assert all(torch.allclose(a.cpu(), b, rtol=0, atol=1e-15) for a, b in zip(got, want))
    m = torch.ops.ebr_fused.rope_merge(gq.to(cuda), gk.to(cuda), gv.to(cuda), cos.to(cuda), sin.to(cuda),
                                       torch.zeros(0, device=cuda))
    assert torch.allclose(m.cpu(), oracle.ref_merge(gq, gk, gv, cos, sin), rtol=0, atol=1e-15)
    x = qkv.to(cuda).requires_grad_(True)
    c, s = cos.to(cuda), sin.to(cuda)

    def f(x):
        q, k, v = rs.rope_split(x, c, s, 2)
        return (q * k).sum(-1) + v.pow(2).sum(-1)

    assert torch.autograd.gradcheck(f, (x,))
    assert torch.autograd.gradgradcheck(f, (x,))
