"""CPU checks that pin the RoPE split/merge oracle (``oracle.rope_ref``) without retyping its formulas, plus the
argument checks of ``ebr_amd.fused_attn.rope_split.rope_split`` (which run before any kernel)."""

import pytest
import torch

import oracle
from ebr_amd import layers


def _tables(d, n, dtype=torch.float64):
    h, w = oracle.grid_shape(n)
    cos, sin = oracle.rotary_tables(d, h, w)
    return cos.to(dtype), sin.to(dtype), (h, w)


def test_quarter_swap_is_the_index_permutation():
    x = torch.arange(2 * 3 * 16, dtype=torch.float64).reshape(2, 3, 16)
    q = 4
    perm = [((d // q) ^ 1) * q + d % q for d in range(16)]
    assert torch.equal(oracle.quarter_swap(x), x[..., perm])
    assert torch.equal(layers.quarter_swap(x), x[..., perm])
    assert torch.equal(oracle.quarter_swap(oracle.quarter_swap(x)), x)


def test_tables_match_the_layers_table():
    for d, (h, w) in [(64, (9, 9)), (16, (3, 5)), (128, (10, 10))]:
        cos, sin = oracle.rotary_tables(d, h, w)
        t = layers.RotaryTable2D(d, h, w)()
        assert torch.allclose(cos, t.cos, atol=1e-6) and torch.allclose(sin, t.sin, atol=1e-6)


@pytest.mark.parametrize("B,N,H,D", [(2, 81, 3, 64), (1, 12, 2, 16), (3, 100, 1, 32)])
def test_split_is_the_broadcast_2d_rope(B, N, H, D):
    """The fused form x cos + quarter_swap(x) sin on the full tables equals rotate_half on each half with the row /
    column tables (the textbook 2D RoPE of ebr_amd.layers.apply_rope), for q and k; v passes through."""
    g = torch.Generator().manual_seed(N)
    qkv = torch.randn((B, N, 3 * H * D), generator=g, dtype=torch.float64)
    cos, sin, (hh, ww) = _tables(D, N)
    q, k, v = oracle.ref_split(qkv, cos, sin, H)
    x = qkv.reshape(B, N, 3, H, D)
    emb = layers.RotaryEmbedding2D(D, hh, ww)
    cs = tuple(tuple(t.double() for t in pair) for pair in emb())
    q_ref, k_ref = layers.apply_rope(cs, x[:, :, 0], x[:, :, 1])
    assert torch.allclose(q, q_ref.transpose(1, 2), atol=1e-12)
    assert torch.allclose(k, k_ref.transpose(1, 2), atol=1e-12)
    assert torch.equal(v, x[:, :, 2].transpose(1, 2))
    assert q.is_contiguous() and k.is_contiguous() and v.is_contiguous()


def test_split_preserves_each_rotated_pair_norm():
    B, N, H, D = 2, 25, 2, 32
    g = torch.Generator().manual_seed(3)
    qkv = torch.randn((B, N, 3 * H * D), generator=g, dtype=torch.float64)
    cos, sin, _ = _tables(D, N)
    q, _, _ = oracle.ref_split(qkv, cos, sin, H)
    x = qkv.reshape(B, N, 3, H, D)[:, :, 0].transpose(1, 2)
    Q = D // 4
    for lo in (0, 2 * Q):  # pairs (d, d + Q) inside each half
        a, b = slice(lo, lo + Q), slice(lo + Q, lo + 2 * Q)
        assert torch.allclose(q[..., a] ** 2 + q[..., b] ** 2, x[..., a] ** 2 + x[..., b] ** 2, atol=1e-12)


@pytest.mark.parametrize("with_qscale", [False, True])
def test_merge_is_the_adjoint_of_split(with_qscale):
    B, N, H, D = 2, 20, 3, 16
    qkv, (gq, gk, gv) = oracle.make_rope_inputs(B, N, H, D, dtype=torch.float64, seed=5)
    cos, sin, _ = _tables(D, N)
    qs = torch.tensor([0.5, 1.25, 2.0], dtype=torch.float64) if with_qscale else None
    q, k, v = oracle.ref_split(qkv, cos, sin, H, qs)
    lhs = (q * gq).sum() + (k * gk).sum() + (v * gv).sum()
    rhs = (qkv * oracle.ref_merge(gq, gk, gv, cos, sin, qs)).sum()
    assert torch.allclose(lhs, rhs, rtol=1e-12)


def test_merge_is_autograds_vjp_of_split():
    B, N, H, D = 1, 9, 2, 8
    qkv, (gq, gk, gv) = oracle.make_rope_inputs(B, N, H, D, dtype=torch.float64, seed=6)
    cos, sin, _ = _tables(D, N)
    x = qkv.clone().requires_grad_(True)
    q, k, v = oracle.ref_split(x, cos, sin, H)
    (vjp,) = torch.autograd.grad((q * gq).sum() + (k * gk).sum() + (v * gv).sum(), x)
    assert torch.allclose(vjp, oracle.ref_merge(gq, gk, gv, cos, sin), atol=1e-12)


def test_planted_mistake_is_caught():
    """An unsigned sin table (rotate_half's sign dropped) no longer equals the broadcast RoPE."""
    B, N, H, D = 1, 16, 1, 16
    g = torch.Generator().manual_seed(1)
    qkv = torch.randn((B, N, 3 * H * D), generator=g, dtype=torch.float64)
    cos, sin, (hh, ww) = _tables(D, N)
    q_bad, _, _ = oracle.ref_split(qkv, cos, sin.abs(), H)
    x = qkv.reshape(B, N, 3, H, D)
    cs = tuple(tuple(t.double() for t in pair) for pair in layers.RotaryEmbedding2D(D, hh, ww)())
    q_ref, _ = layers.apply_rope(cs, x[:, :, 0], x[:, :, 1])
    assert not torch.allclose(q_bad, q_ref.transpose(1, 2), atol=1e-6)


def test_temperature_rounds_twice_in_bf16():
    B, N, H, D = 2, 9, 2, 16
    qkv, _ = oracle.make_rope_inputs(B, N, H, D, dtype=torch.bfloat16, seed=7)
    cos, sin, _ = _tables(D, N, torch.float32)
    qs = torch.tensor([1.3, 0.7])
    q1, _, _ = oracle.ref_split(qkv, cos, sin, H)
    q2, _, _ = oracle.ref_split(qkv, cos, sin, H, qs)
    assert torch.equal(q2, (q1.float() * qs.view(1, -1, 1, 1)).to(torch.bfloat16))


def test_rope_split_argument_checks():
    from ebr_amd.fused_attn.rope_split import rope_split

    cos = torch.zeros(9, 16)
    with pytest.raises(ValueError):
        rope_split(torch.zeros(2, 9, 47), cos, cos, 1)  # last dim not a multiple of 3 * heads
    with pytest.raises(ValueError):
        rope_split(torch.zeros(2, 9, 3 * 18), torch.zeros(9, 18), torch.zeros(9, 18), 1)  # D % 4
    with pytest.raises(ValueError):
        rope_split(torch.zeros(2, 9, 48), torch.zeros(8, 16), torch.zeros(8, 16), 1)  # table rows != N
    with pytest.raises(ValueError):
        rope_split(torch.zeros(2, 9, 96), cos, cos, 2, torch.ones(3))  # qscale: one value per head
