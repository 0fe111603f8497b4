"""GPU parity of the fp64 kernels (ebr_fused ops on float64 inputs) against the CPU oracle in fp64, the golden
fixtures, and torch's gradcheck / gradgradcheck through ``fused_attention`` on the GPU (the reference tests its fp64
path the same way).

The ops round the scale to fp32 once, as the reference's launchers do (triton_kernels.py:689-693: "the fp64
gradcheck path sees the same fp32-rounded scale"), so the oracle is given that rounded scale. Bar: the reference's
max-relative error max|a - ref| / max|ref| <= 1e-12 for every output.
"""

import os

import numpy as np
import pytest
import torch

import oracle
from ebr_amd.fused_attn import fused_attention, ops  # noqa: F401

pytestmark = pytest.mark.gpu

F64 = torch.float64
TOL = 1e-12
NAMES = ["o", "lse", "dq", "dk", "dv", "hq", "hk", "hv", "hdo"]


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _s32(scale):
    return float(torch.tensor(scale, dtype=torch.float32))


def _run_gpu(ins, scale, dev):
    q, k, v, do, gq, gk, gv = (x.to(dev) for x in ins)
    o, lse = torch.ops.ebr_fused.attn_fwd(q, k, v, scale)
    dq, dk, dv = torch.ops.ebr_fused.attn_bwd(q, k, v, o, lse, do, scale)
    hq, hk, hv, hdo = torch.ops.ebr_fused.attn_bwd_bwd(q, k, v, o, lse, do, dq, gq, gk, gv, scale)
    torch.cuda.synchronize()
    return [x.cpu() for x in (o, lse, dq, dk, dv, hq, hk, hv, hdo)]


def _run_oracle(ins, scale):
    q, k, v, do, gq, gk, gv = ins
    o, lse = oracle.attn_fwd(q, k, v, scale)
    dq, dk, dv = oracle.attn_bwd(q, k, v, o, lse, do, scale)
    hq, hk, hv, hdo = oracle.attn_bwd_bwd(q, k, v, o, lse, do, dq, gq, gk, gv, scale)
    return [o, lse, dq, dk, dv, hq, hk, hv, hdo]


def _compare(got, ref, label, L):
    for n, g, r in zip(NAMES, got, ref):
        assert g.dtype == F64, (label, n, g.dtype)
        if L == 1 and n in ("dq", "dk", "hq", "hk", "hv"):  # exactly zero with one key
            assert float(g.abs().max()) <= TOL * float(ref[NAMES.index("dv")].abs().max()), (label, n)
            continue
        e = oracle.rel_err(g, r)
        assert e <= TOL, f"{label}: {n} rel err {e:.3e}"


@pytest.mark.parametrize(
    "B,H,L,D",
    [(2, 3, 1, 8), (2, 2, 5, 3), (1, 2, 17, 64), (2, 2, 40, 128), (1, 1, 81, 7), (2, 1, 129, 16), (1, 2, 200, 64),
     (1, 1, 9, 1), (1, 1, 33, 100), (1, 2, 17, 136), (2, 1, 40, 200), (1, 1, 70, 256)],
)
def test_fp64_matches_oracle(cuda, B, H, L, D):
    _say(f"fp64 B={B} H={H} L={L} D={D}")
    ins = oracle.make_inputs(B, H, L, D, dtype=F64, seed=L + D)
    scale = _s32(D**-0.5)
    _compare(_run_gpu(ins, scale, cuda), _run_oracle(ins, scale), f"B={B} H={H} L={L} D={D}", L)


def test_fp64_strided_views_and_zero_rows(cuda):
    """q, k, v as views of a fused [B, L, 3, H, D] projection (no copies at fp64's 8-byte rule), cotangents as one
    expanded zero row and a transposed view."""
    _say("fp64 strided")
    B, H, L, D = 2, 3, 21, 5
    g = torch.Generator().manual_seed(3)
    qkv = torch.randn(B, L, 3, H, D, generator=g, dtype=F64)
    q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
    do = torch.randn(B, L, H, D, generator=g, dtype=F64).transpose(1, 2)
    gq = torch.randn(B, H, L, D, generator=g, dtype=F64)
    zero = torch.zeros(D, dtype=F64).expand(B, H, L, D)
    scale = _s32(D**-0.5)
    ins = (q, k, v, do, gq, zero, zero)
    qd = qkv.to(cuda)
    views = [qd[:, :, i].transpose(1, 2) for i in range(3)]
    assert not views[0].is_contiguous() and ops._rows(views[0]).data_ptr() == views[0].data_ptr()
    dev_ins = (*views, do.to(cuda), gq.to(cuda), zero.to(cuda), zero.to(cuda))
    o, lse = torch.ops.ebr_fused.attn_fwd(*dev_ins[:3], scale)
    d = torch.ops.ebr_fused.attn_bwd(*dev_ins[:3], o, lse, dev_ins[3], scale)
    h = torch.ops.ebr_fused.attn_bwd_bwd(*dev_ins[:3], o, lse, dev_ins[3], d[0], *dev_ins[4:], scale)
    got = [x.cpu() for x in (o, lse, *d, *h)]
    _compare(got, _run_oracle([x.contiguous() for x in ins], scale), "strided", L)


def test_fp64_matches_golden(cuda):
    """The committed fixtures (fp64 outputs from fp32-valued inputs) whose scale is exact in fp32."""
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "attn_small.npz"))
    n = 0
    for ci in range(int(z["ncases"][0])):
        s = float(z[f"c{ci}_scale"][0])
        if _s32(s) != s:
            continue
        get = lambda name: torch.from_numpy(z[f"c{ci}_{name}"]).double()  # noqa: E731
        ins = [get(x) for x in ("q", "k", "v", "do", "gq", "gk", "gv")]
        _say(f"fp64 golden c{ci}")
        got = _run_gpu(ins, s, cuda)
        _compare(got, [get(x) for x in NAMES], f"golden c{ci}", int(z[f"c{ci}_shape"][2]))
        n += 1
    assert n >= 3


@pytest.mark.parametrize("shape", [(1, 2, 6, 4), (1, 1, 3, 136)])  # 136: the 8-row kernels of D > 128
def test_fp64_gradcheck_and_gradgradcheck(cuda, shape):
    """torch.autograd.gradcheck / gradgradcheck of fused_attention on the GPU: the forward, its backward (attn_bwd)
    and the double backward (attn_bwd_bwd) against finite differences of the op itself."""
    _say(f"fp64 gradcheck {shape}")
    g = torch.Generator().manual_seed(11)
    q, k, v = (torch.randn(*shape, generator=g, dtype=F64).to(cuda).requires_grad_(True) for _ in range(3))

    def f(a, b, c):
        return fused_attention(a, b, c, scale=0.5)

    assert torch.autograd.gradcheck(f, (q, k, v), eps=1e-6, atol=1e-8, rtol=1e-6)
    assert torch.autograd.gradgradcheck(f, (q, k, v), eps=1e-6, atol=1e-7, rtol=1e-5)


def test_fp64_lse_dtype_and_fakes(cuda):
    q = torch.randn(1, 1, 4, 8, dtype=F64, device=cuda)
    o, lse = torch.ops.ebr_fused.attn_fwd(q, q, q, 0.25)
    assert o.dtype == F64 and lse.dtype == F64 and lse.shape == (1, 1, 4)
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode() as mode:
        fq = mode.from_tensor(q)
        fo, flse = torch.ops.ebr_fused.attn_fwd(fq, fq, fq, 0.25)
        assert flse.dtype == F64
