"""The fused 2D-RoPE split / merge ops on CPU tensors: the package's dense path (the reference runs its dense
functions there, models/fused_attn/rope_split.py:71-101) against the CPU oracle, bit for bit, and the autograd pair
(split and merge are each other's backward) checked by fp64 gradcheck and gradgradcheck."""

import torch

import oracle
from ebr_amd.fused_attn.rope_split import rope_split


def _tables(n, d):
    h, w = oracle.grid_shape(n)
    return oracle.rotary_tables(d, h, w)


def test_dense_split_and_merge_equal_the_oracle_bitwise():
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        qkv, gs = oracle.make_rope_inputs(2, 12, 3, 16, dtype=dt, seed=3)
        cos, sin = _tables(12, 16)
        qs = torch.tensor([1.25, 0.5, 2.0]).to(dt)
        for scale in (None, qs):
            got = torch.ops.ebr_fused.rope_split(qkv, cos, sin, qs if scale is not None else torch.zeros(0), 3)
            want = oracle.ref_split(qkv, cos, sin, 3, scale)
            assert all(torch.equal(a, b) for a, b in zip(got, want)), dt
            m = torch.ops.ebr_fused.rope_merge(*gs, cos, sin, qs if scale is not None else torch.zeros(0))
            assert torch.equal(m, oracle.ref_merge(*gs, cos, sin, scale)), dt


def test_split_merge_autograd_to_second_order_fp64():
    qkv, _ = oracle.make_rope_inputs(1, 6, 2, 8, dtype=torch.float64, seed=4)
    cos, sin = _tables(6, 8)
    cos, sin = cos.double(), sin.double()
    x = qkv.clone().requires_grad_(True)

    def f(x):
        q, k, v = rope_split(x, cos, sin, 2)
        return (q * k).sum(-1) + v.pow(2).sum(-1)

    assert torch.autograd.gradcheck(f, (x,))
    assert torch.autograd.gradgradcheck(f, (x,))


def test_unused_outputs_get_no_materialised_cotangent():
    qkv, _ = oracle.make_rope_inputs(1, 6, 2, 8, dtype=torch.float64, seed=5)
    cos, sin = _tables(6, 8)
    x = qkv.clone().requires_grad_(True)
    q, k, v = rope_split(x, cos.double(), sin.double(), 2)
    (g,) = torch.autograd.grad(q.sum(), x)  # k and v unused
    want = oracle.ref_merge(torch.ones_like(q), torch.zeros_like(k), torch.zeros_like(v), cos.double(), sin.double())
    assert torch.allclose(g, want, atol=1e-14)
