"""GPU parity: the gfx950 kernels (through the C ABI, via the ebr_fused ops) against the CPU oracle.

Bars: max|a - ref| / max|ref| <= 1e-5 for fp32 and <= 2e-2 for bf16/fp16, for O, lse, dQ, dK,
dV and hQ, hK, hV, hdO, on identical seeded inputs. Slices (b, h) are independent, so at the full BASELINE sizes a
random sample of slices is checked against the oracle run on exactly those slices.
"""

import math

import pytest
import torch

import oracle
from ebr_amd.fused_attn import ops  # noqa: F401  (registers torch.ops.ebr_fused.*)

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def _say(msg: str) -> None:
    print(f"[case] {msg}", flush=True)


def _inputs(B, H, L, D, dtype, seed=0):
    scale = 0.125 if dtype != torch.float32 else None
    return oracle.make_inputs(B, H, L, D, dtype=dtype, seed=seed, qkv_scale=scale)


def _hip_all(q, k, v, do, gq, gk, gv, scale, dev):
    """All three ops on the GPU; returns CPU tensors (o, lse, dq, dk, dv, hq, hk, hv, hdo)."""
    t = [x.to(dev) for x in (q, k, v, do, gq, gk, gv)]
    qd, kd, vd, dod, gqd, gkd, gvd = t
    o, lse = torch.ops.ebr_fused.attn_fwd(qd, kd, vd, scale)
    dq, dk, dv = torch.ops.ebr_fused.attn_bwd(qd, kd, vd, o, lse, dod, scale)
    hq, hk, hv, hdo = torch.ops.ebr_fused.attn_bwd_bwd(qd, kd, vd, o, lse, dod, dq, gqd, gkd, gvd, scale)
    torch.cuda.synchronize()
    return [x.cpu() for x in (o, lse, dq, dk, dv, hq, hk, hv, hdo)]


def _oracle_all(q, k, v, do, gq, gk, gv, scale, o=None, lse=None, chunk=None):
    """Oracle outputs. bwd and bwd_bwd consume the given (o, lse) when provided (the GPU forward's), so each phase
    is checked on its own inputs, as the reference's ops are."""
    o_ref, lse_ref = oracle.attn_fwd(q, k, v, scale, chunk=chunk)
    o_in = o_ref if o is None else o
    lse_in = lse_ref if lse is None else lse
    dq, dk, dv = oracle.attn_bwd(q, k, v, o_in, lse_in, do, scale, chunk=chunk)
    hq, hk, hv, hdo = oracle.attn_bwd_bwd(q, k, v, o_in, lse_in, do, dq, gq, gk, gv, scale, chunk=chunk)
    return [o_ref, lse_ref, dq, dk, dv, hq, hk, hv, hdo]


NAMES = ["o", "lse", "dq", "dk", "dv", "hq", "hk", "hv", "hdo"]


def _compare(got, ref, dtype, label, tol=None):
    tol = TOL[dtype] if tol is None else tol
    errs = {n: oracle.rel_err(g, r) for n, g, r in zip(NAMES, got, ref)}
    for n, g in zip(NAMES, got):
        assert torch.isfinite(g.float()).all(), f"{label}: non-finite {n}"
    bad = {n: e for n, e in errs.items() if not (e <= tol)}
    print(f"{label}: " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    assert not bad, f"{label}: over tolerance {tol}: {bad}"
    return errs


def _case(B, H, L, D, dtype, dev, seed=0, tol=None):
    label = f"B={B} H={H} L={L} D={D} {str(dtype).split('.')[-1]} seed={seed}"
    _say(label)
    q, k, v, do, gq, gk, gv = _inputs(B, H, L, D, dtype, seed)
    scale = D**-0.5
    got = _hip_all(q, k, v, do, gq, gk, gv, scale, dev)
    ref = _oracle_all(q, k, v, do, gq, gk, gv, scale, o=got[0], lse=got[1])
    if L == 1:
        # Known answer: with one key P = 1, so O = V, dV = dO, hdO = gV, and dQ, dK, hQ, hK, hV are exactly 0; their
        # reference values are rounding noise, so they are checked against the size of the non-zero outputs.
        tol_ = TOL[dtype] if tol is None else tol
        zero = {"dq", "dk", "hq", "hk", "hv"}
        big = max(float(got[NAMES.index(n)].abs().max()) for n in ("dv", "hdo"))
        for n, g_ in zip(NAMES, got):
            if n in zero:
                assert float(g_.abs().max()) <= tol_ * big, f"{label}: {n} not ~0"
        keep = [i for i, n in enumerate(NAMES) if n not in zero]
        got = [got[i] if i in keep else torch.zeros(1) for i in range(len(NAMES))]
        ref = [ref[i] if i in keep else torch.zeros(1) for i in range(len(NAMES))]
        assert torch.equal(got[0].float(), v.float()), "L=1: O must equal V"
    return _compare(got, ref, dtype, label, tol)


# ---------------------------------------------------------------------------------------------------------------------
# Shape sweep: one-workgroup kernels (L <= 128) and two-launch kernels (L > 128), every head dim, every dtype.
# ---------------------------------------------------------------------------------------------------------------------


@pytest.mark.parametrize("L", [1, 7, 16, 17, 31, 32, 33, 64, 81, 100, 127, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_small_L(cuda, L, dtype):
    _case(2, 3, L, 64, dtype, cuda, seed=L)


@pytest.mark.parametrize("L", [129, 200, 256, 333])  # 256: no short stage, the first full stage finds m = -inf
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_long_L(cuda, L, dtype):
    _case(2, 2, L, 64, dtype, cuda, seed=L)


# The long kernels run the last 64-row stage of a slice 16 rows at a time, as far as L: 1, 2, 3 and 4 live tiles
# (L mod 64 = 22, 33, 49, 63), at every head dim the 16-bit long kernels are built for.
@pytest.mark.parametrize("L", [150, 161, 177, 191])
@pytest.mark.parametrize("D", [32, 64, 128])
def test_long_last_stage_tiles(cuda, L, D):
    _case(2, 2, L, D, torch.bfloat16, cuda, seed=L + D)


@pytest.mark.parametrize("D", [16, 32, 48, 128])
@pytest.mark.parametrize("L", [45, 150])
def test_head_dims_fp32(cuda, D, L):
    _case(2, 2, L, D, torch.float32, cuda, seed=D + L)


@pytest.mark.parametrize("D", [32, 40, 128])
@pytest.mark.parametrize("L", [45, 150])
def test_head_dims_bf16(cuda, D, L):
    _case(2, 2, L, D, torch.bfloat16, cuda, seed=D + L)


@pytest.mark.parametrize("L", [81, 200])
def test_fp16(cuda, L):
    _case(2, 2, L, 64, torch.float16, cuda, seed=5)


# Head dims above 128 (the reference pads any D to a power of two, triton_kernels.py:587-589): the streamed two-launch
# kernels at 256-wide rows, for every L; fp32 reads its seq-contraction operands from the natural rows there. 136 and
# 130 / 132 are padded to 256-wide rows with zero columns; L = 1 checks the known answer, 17 a ragged single chunk,
# 100 several row blocks, 150 a ragged last chunk.
@pytest.mark.parametrize("L", [1, 17, 100, 150])
@pytest.mark.parametrize("D,dtype", [(256, torch.bfloat16), (192, torch.float16), (136, torch.bfloat16),
                                     (256, torch.float32), (132, torch.float32)])
def test_wide_head_dims(cuda, L, D, dtype):
    _case(2, 2, L, D, dtype, cuda, seed=D + L)


@pytest.mark.parametrize("D,dtype", [(130, torch.bfloat16), (256, torch.bfloat16), (252, torch.float32)])
def test_wide_head_dims_strided(cuda, D, dtype):
    """Views of a fused [B, L, 3, H, D] projection on the GPU (row stride 3 H D, not contiguous); 130 and 252 are
    also padded by the ops."""
    _say(f"wide D={D} {str(dtype).split('.')[-1]} strided views")
    B, H, L = 2, 2, 70
    g = torch.Generator("cpu").manual_seed(D)
    qkv = (torch.randn(B, L, 3, H, D, generator=g) * 0.125).to(dtype)
    do, gq, gk, gv = (torch.randn(B, H, L, D, generator=g).to(dtype) for _ in range(4))
    qkv_d = qkv.to(cuda)
    q, k, v = (qkv_d[:, :, i].transpose(1, 2) for i in range(3))
    assert not q.is_contiguous()
    dod, gqd, gkd, gvd = (t.to(cuda) for t in (do, gq, gk, gv))
    scale = D**-0.5
    o, lse = torch.ops.ebr_fused.attn_fwd(q, k, v, scale)
    dq, dk, dv = torch.ops.ebr_fused.attn_bwd(q, k, v, o, lse, dod, scale)
    hs = torch.ops.ebr_fused.attn_bwd_bwd(q, k, v, o, lse, dod, dq, gqd, gkd, gvd, scale)
    got = [x.cpu() for x in (o, lse, dq, dk, dv, *hs)]
    qc, kc, vc = (qkv[:, :, i].transpose(1, 2).contiguous() for i in range(3))
    ref = _oracle_all(qc, kc, vc, do, gq, gk, gv, scale, o=got[0], lse=got[1])
    _compare(got, ref, dtype, f"wide D={D} strided")


# ---------------------------------------------------------------------------------------------------------------------
# BASELINE configurations
# ---------------------------------------------------------------------------------------------------------------------


def test_config0_nqueens_fp32_full(cuda):
    """Config 0: fp32 B=32 H=8 L=64 D=64, Q/K/V/dO/R ~ N(0,1) seed 0, every slice, 1e-5."""
    _case(32, 8, 64, 64, torch.float32, cuda, seed=0)


def _sampled(B, H, L, D, dtype, dev, nsample, seed=0):
    label = f"sampled B={B} H={H} L={L} D={D} {str(dtype).split('.')[-1]}"
    _say(label)
    q, k, v, do, gq, gk, gv = _inputs(B, H, L, D, dtype, seed)
    scale = D**-0.5
    got = _hip_all(q, k, v, do, gq, gk, gv, scale, dev)
    g = torch.Generator().manual_seed(1234)
    idx = torch.randperm(B * H, generator=g)[:nsample]

    def pick(t):
        return t.reshape(B * H, *t.shape[2:])[idx].unsqueeze(0)

    sub = [pick(t) for t in (q, k, v, do, gq, gk, gv)]
    got_s = [pick(t) for t in got]
    ref = _oracle_all(*sub, scale, o=got_s[0], lse=got_s[1])
    return _compare(got_s, ref, dtype, label)


def test_config1_sudoku_bf16_full_size(cuda):
    """Config 1: bf16 B=768 H=8 L=81 D=64 at full size; 128 random slices checked."""
    _sampled(768, 8, 81, 64, torch.bfloat16, cuda, 128)


@pytest.mark.parametrize("L", [28, 45, 64, 100])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_multi_solution_head_dim_128_full_size(cuda, L, dtype):
    """The multi-solution recipes' shapes: hidden 512 over 4 heads (D = 128), global batch 768, L = 28 / 45 (graph
    colouring 8 / 10), 64 / 100 (N-Queens 8 / 10); 16 random slices checked."""
    _sampled(768, 4, L, 128, dtype, cuda, 16, seed=L)


def test_config2_maze_bf16_full_size(cuda):
    """Config 2: bf16 B=64 H=8 L=900 D=64 at full size; 12 random slices checked."""
    _sampled(64, 8, 900, 64, torch.bfloat16, cuda, 12)


@pytest.mark.parametrize(
    "B,H,L,D,dtype",
    [
        (64, 8, 333, 32, torch.bfloat16),
        (48, 8, 517, 64, torch.float16),
        (64, 8, 177, 64, torch.bfloat16),
        (64, 8, 161, 128, torch.bfloat16),
        (48, 8, 240, 64, torch.bfloat16),
        (64, 8, 340, 128, torch.float16),
        (16, 8, 1024, 64, torch.bfloat16),
    ],
)
def test_long_wide_grids_ragged_L(cuda, B, H, L, D, dtype):
    """Grids large enough for the wide long-sequence workgroups (7 compute waves; 10 in the bwd_bwd row kernel, with
    its own 160-row blocking), L not a multiple of any block or stage (last stages of 1 to 4 live 16-row tiles); 8
    random slices checked. At L = 240, 340 and 1024 the last 112-row block holds one live 16-row strip (after a
    short stage of 48, 20 or no rows)."""
    _sampled(B, H, L, D, dtype, cuda, 8, seed=L)


@pytest.mark.parametrize("B,H,L", [(1, 2, 2500), (8, 8, 2500)])
def test_long_sequences_many_stages(cuda, B, H, L):
    """L = 2500 (40 stages of 64 rows, the last 4 rows short; 23 row blocks of 112, or 16 of the bwd_bwd row kernel's
    160 rows, none of them a multiple): the small-grid (4 waves) and wide (7 and 10 waves) long-sequence workgroups;
    2 random slices checked."""
    _sampled(B, H, L, 64, torch.bfloat16, cuda, 2, seed=L)


def test_config4_shape_bf16(cuda):
    """Config 4's attention shape (L=100) on a reduced batch; all slices checked."""
    _case(40, 8, 100, 64, torch.bfloat16, cuda, seed=4)


# ---------------------------------------------------------------------------------------------------------------------
# Strided inputs, stride-0 cotangents, the autograd path
# ---------------------------------------------------------------------------------------------------------------------


@pytest.mark.parametrize(
    "B,L,D",
    [(3, 81, 64), (3, 200, 64), (3, 45, 128), (3, 70, 128), (70, 100, 128)],
)
def test_strided_views(cuda, B, L, D):
    """q, k, v as transposed views of one [B, L, 3, H, D] projection (non-contiguous B/H/L strides); at D = 128 the
    persistent backward kernels (k_bwd_pipe, k_bwd_pp) and the half-chunk backward of the backward, B = 70 giving more
    slices than the persistent grid."""
    H = 4
    _say(f"strided qkv views B={B} L={L} D={D}")
    g = torch.Generator().manual_seed(7)
    qkv = (torch.randn(B, L, 3, H, D, generator=g) * 0.125).to(torch.bfloat16)
    do = torch.randn(B, H, L, D, generator=g).to(torch.bfloat16)
    gq, gk, gv = (torch.randn(B, H, L, D, generator=g).to(torch.bfloat16) for _ in range(3))
    qkv_d = qkv.to(cuda)
    q, k, v = (qkv_d[:, :, i].transpose(1, 2) for i in range(3))
    assert not q.is_contiguous()
    scale = D**-0.5
    o, lse = torch.ops.ebr_fused.attn_fwd(q, k, v, scale)
    dq, dk, dv = torch.ops.ebr_fused.attn_bwd(q, k, v, o, lse, do.to(cuda), scale)
    hq, hk, hv, hdo = torch.ops.ebr_fused.attn_bwd_bwd(
        q, k, v, o, lse, do.to(cuda), dq, gq.to(cuda), gk.to(cuda), gv.to(cuda), scale
    )
    got = [x.cpu() for x in (o, lse, dq, dk, dv, hq, hk, hv, hdo)]
    qc, kc, vc = (qkv[:, :, i].transpose(1, 2).contiguous() for i in range(3))
    ref = _oracle_all(qc, kc, vc, do, gq, gk, gv, scale, o=got[0], lse=got[1])
    _compare(got, ref, torch.bfloat16, f"strided B={B} L={L} D={D}")


@pytest.mark.parametrize("B,H,L,D", [(32, 4, 900, 64), (96, 4, 333, 128)])
def test_strided_views_long_wide_grids(cuda, B, H, L, D):
    """Every input a non-contiguous view at the long-sequence shapes with the wide (7-wave) workgroups: q, k, v
    slices of one [B, L, 3, H, D] projection, dO and the cotangents transposed [B, L, H, D] tensors; 6 random
    slices checked against the oracle on contiguous copies."""
    _say(f"strided long views B={B} H={H} L={L} D={D}")
    g = torch.Generator().manual_seed(L)
    qkv = (torch.randn(B, L, 3, H, D, generator=g) * 0.125).to(torch.bfloat16)
    rest = [torch.randn(B, L, H, D, generator=g).to(torch.bfloat16) for _ in range(4)]
    qkv_d = qkv.to(cuda)
    q, k, v = (qkv_d[:, :, i].transpose(1, 2) for i in range(3))
    do, gq, gk, gv = (t.to(cuda).transpose(1, 2) for t in rest)
    assert not (q.is_contiguous() or do.is_contiguous() or gk.is_contiguous())
    scale = D**-0.5
    o, lse = torch.ops.ebr_fused.attn_fwd(q, k, v, scale)
    dq, dk, dv = torch.ops.ebr_fused.attn_bwd(q, k, v, o, lse, do, scale)
    hq, hk, hv, hdo = torch.ops.ebr_fused.attn_bwd_bwd(q, k, v, o, lse, do, dq, gq, gk, gv, scale)
    torch.cuda.synchronize()
    idx = torch.randperm(B * H, generator=g)[:6]

    def pick(t):
        return t.reshape(B * H, *t.shape[2:])[idx].unsqueeze(0)

    got = [pick(x.cpu()) for x in (o, lse, dq, dk, dv, hq, hk, hv, hdo)]
    ins = [qkv[:, :, i].transpose(1, 2).contiguous() for i in range(3)] + [t.transpose(1, 2).contiguous() for t in rest]
    qs, ks, vs, dos, gqs, gks, gvs = (pick(t) for t in ins)
    ref = _oracle_all(qs, ks, vs, dos, gqs, gks, gvs, scale, o=got[0], lse=got[1])
    _compare(got, ref, torch.bfloat16, f"strided long B={B} H={H} L={L} D={D}")


def test_wide_row_stride(cuda):
    """Views whose row stride exceeds 16 KiB (a [B, L, 3, H, D] projection with H = 48): the persistent backward of
    the backward cannot hold that stride in a structured buffer descriptor and takes the one-slice kernel."""
    B, H, L, D = 1, 48, 81, 64
    _say("row stride > 16 KiB")
    g = torch.Generator().manual_seed(11)
    qkv = (torch.randn(B, L, 3, H, D, generator=g) * 0.125).to(torch.bfloat16)
    do, gq, gk, gv = (torch.randn(B, H, L, D, generator=g).to(torch.bfloat16) for _ in range(4))
    qkv_d = qkv.to(cuda)
    q, k, v = (qkv_d[:, :, i].transpose(1, 2) for i in range(3))
    assert q.stride(2) * q.element_size() > 16383
    scale = D**-0.5
    o, lse = torch.ops.ebr_fused.attn_fwd(q, k, v, scale)
    dq, dk, dv = torch.ops.ebr_fused.attn_bwd(q, k, v, o, lse, do.to(cuda), scale)
    hq, hk, hv, hdo = torch.ops.ebr_fused.attn_bwd_bwd(
        q, k, v, o, lse, do.to(cuda), dq, gq.to(cuda), gk.to(cuda), gv.to(cuda), scale
    )
    got = [x.cpu() for x in (o, lse, dq, dk, dv, hq, hk, hv, hdo)]
    qc, kc, vc = (qkv[:, :, i].transpose(1, 2).contiguous() for i in range(3))
    ref = _oracle_all(qc, kc, vc, do, gq, gk, gv, scale, o=got[0], lse=got[1])
    _compare(got, ref, torch.bfloat16, "row stride > 16 KiB")


# (B, H, L, D): more slices than the persistent kernels' grid (one workgroup per CU times the workgroups a CU holds),
# with a remainder, for one to four 32-key chunks and every head dim the persistent kernels take: at D = 128 the
# backward (one and two chunks; three, and four up to L = 112, with one region of each kind; L = 113 past that) and
# the backward of the backward (with four loader waves at two chunks); at D = 32 and 64 with four chunks the backward
# (tiles at D = 32, recomputed P and dS at D = 64).
@pytest.mark.parametrize(
    "B,H,L,D",
    [(75, 4, 81, 64), (130, 8, 20, 64), (70, 8, 50, 32), (90, 6, 96, 32), (101, 6, 100, 32), (99, 6, 113, 64),
     (140, 4, 28, 128), (130, 4, 45, 128), (129, 4, 64, 128), (70, 4, 70, 128), (67, 4, 100, 128),
     (65, 4, 112, 128), (66, 4, 113, 128)],
)
def test_persistent_many_slices(cuda, B, H, L, D):
    _case(B, H, L, D, torch.bfloat16, cuda, seed=L + D)


@pytest.mark.parametrize("L", [81, 200])
def test_zero_cotangent_rows(cuda, L):
    """gq = gk = 0 as stride-0 expanded rows: hV = 0 and hdO = P gV exactly as the dense formula gives."""
    B, H, D = 2, 2, 64
    dtype = torch.float32
    _say(f"stride-0 cotangents L={L}")
    q, k, v, do, _, _, gv = _inputs(B, H, L, D, dtype, 3)
    scale = D**-0.5
    z = torch.zeros(D, dtype=dtype).expand(B, H, L, D)
    dev = cuda
    qd, kd, vd, dod = (t.to(dev) for t in (q, k, v, do))
    zd = torch.zeros(D, device=dev, dtype=dtype).expand(B, H, L, D)
    o, lse = torch.ops.ebr_fused.attn_fwd(qd, kd, vd, scale)
    dq, _, _ = torch.ops.ebr_fused.attn_bwd(qd, kd, vd, o, lse, dod, scale)
    hq, hk, hv, hdo = torch.ops.ebr_fused.attn_bwd_bwd(qd, kd, vd, o, lse, dod, dq, zd, zd, gv.to(dev), scale)
    ref = oracle.attn_bwd_bwd(q, k, v, o.cpu(), lse.cpu(), do, None, z, z, gv, scale)
    assert hv.abs().max().item() == 0.0
    for n, g_, r in zip(["hq", "hk", "hv", "hdo"], (hq, hk, hv, hdo), ref):
        if n != "hv":
            assert oracle.rel_err(g_.cpu(), r) <= 1e-5, n


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_autograd_double_backward(cuda, dtype):
    """fused_attention + autograd.grad(create_graph) + second grad, against autograd on the eager math attention."""
    from ebr_amd.fused_attn import fused_attention

    B, H, L, D = 2, 4, 81, 64
    _say(f"autograd double backward {dtype}")
    q, k, v, do, r1, r2, r3 = _inputs(B, H, L, D, dtype, 11)
    ref = oracle.autograd_bwd_bwd(q, k, v, do, r1, r2, r3)
    ref_first = oracle.autograd_bwd(q, k, v, do)
    qd, kd, vd = (t.to(cuda).requires_grad_(True) for t in (q, k, v))
    dod = do.to(cuda).requires_grad_(True)
    out = fused_attention(qd, kd, vd)
    dq, dk, dv = torch.autograd.grad(out, (qd, kd, vd), dod, create_graph=True)
    phi = (dq * r1.to(cuda)).sum() + (dk * r2.to(cuda)).sum() + (dv * r3.to(cuda)).sum()
    hq, hk, hv, hdo = torch.autograd.grad(phi, (qd, kd, vd, dod))
    tol = TOL[dtype]
    for n, g_, r in zip(["dq", "dk", "dv"], (dq, dk, dv), ref_first):
        assert oracle.rel_err(g_.detach().cpu(), r) <= tol, n
    for n, g_, r in zip(["hq", "hk", "hv", "hdo"], (hq, hk, hv, hdo), ref):
        e = oracle.rel_err(g_.cpu(), r)
        print(f"  {n} rel={e:.2e}", flush=True)
        assert e <= tol, n


def test_verify_second_order_fused(cuda):
    """The reference's runtime gate (b=2, seq=32, heads=2, head_dim=16, fp32, rtol 5e-2) passes on the HIP backend."""
    from ebr_amd.attention import get_backend, verify_second_order

    _say("verify_second_order(fused)")
    verify_second_order(get_backend("fused"), device=cuda)


@pytest.mark.parametrize("B,H,L,D,dtype", [(4, 4, 150, 64, torch.bfloat16), (8, 4, 81, 64, torch.bfloat16),
                                           (2, 2, 100, 256, torch.bfloat16), (2, 2, 60, 256, torch.float32),
                                           (2, 2, 100, 128, torch.float16)])
def test_outputs_do_not_depend_on_stale_memory(cuda, B, H, L, D, dtype):
    """Two calls with the same inputs after a caching-allocator churn give bit-identical results (no reads of
    uninitialised memory, no run-to-run nondeterminism): long, persistent, resident and wide-row kernels."""
    _say(f"determinism B={B} H={H} L={L} D={D} {dtype}")
    q, k, v, do, gq, gk, gv = _inputs(B, H, L, D, dtype, 21)
    scale = D**-0.5
    a = _hip_all(q, k, v, do, gq, gk, gv, scale, cuda)
    junk = torch.full((64 << 20,), float("nan"), device=cuda)
    del junk
    b = _hip_all(q, k, v, do, gq, gk, gv, scale, cuda)
    for n, x, y in zip(NAMES, a, b):
        assert torch.equal(x, y), n


@pytest.mark.parametrize("D", [20, 36, 72, 100])
@pytest.mark.parametrize("L", [45, 150])
def test_padded_head_dims_bf16(cuda, D, L):
    """Head dims the kernels do not take natively are zero-padded to the next multiple of 8 and cut back (reference
    triton_kernels.py:587-589 pads the same way): exact, so the usual bar holds."""
    _case(2, 3, L, D, torch.bfloat16, cuda, seed=D * L)


@pytest.mark.parametrize("D,dtype", [(6, torch.float32), (30, torch.float32), (20, torch.float16), (3, torch.bfloat16)])
def test_padded_head_dims_other_dtypes(cuda, D, dtype):
    _case(2, 2, 33, D, dtype, cuda, seed=D)


def test_reference_mode_runs_dense_on_gpu_tensors(cuda, monkeypatch):
    """EBR_FUSED_ATTN_IMPL=reference selects the dense torch path for GPU tensors too (reference loader.py:21-23)."""
    from ebr_amd.fused_attn import dense

    _say("EBR_FUSED_ATTN_IMPL=reference on GPU tensors")
    monkeypatch.setenv("EBR_FUSED_ATTN_IMPL", "reference")
    assert ops.implementation("cuda") == "reference"
    used = []
    monkeypatch.setattr(dense, "attn_fwd", lambda *a, f=dense.attn_fwd: used.append(1) or f(*a))
    q, k, v, do, gq, gk, gv = _inputs(2, 2, 40, 64, torch.bfloat16, 9)
    got = _hip_all(q, k, v, do, gq, gk, gv, 0.125, cuda)
    assert used, "the dense path did not run"
    ref = _oracle_all(q, k, v, do, gq, gk, gv, 0.125, o=got[0], lse=got[1])
    _compare(got, ref, torch.bfloat16, "reference mode")


def test_empty_batch(cuda):
    _say("empty batch")
    q = torch.randn(0, 2, 16, 64, device=cuda, dtype=torch.bfloat16)
    o, lse = torch.ops.ebr_fused.attn_fwd(q, q, q, 0.125)
    dq, dk, dv = torch.ops.ebr_fused.attn_bwd(q, q, q, o, lse, q, 0.125)
    hs = torch.ops.ebr_fused.attn_bwd_bwd(q, q, q, o, lse, q, dq, q, q, q, 0.125)
    assert o.shape == q.shape and lse.shape == (0, 2, 16) and all(t.shape == q.shape for t in (dq, dk, dv, *hs))


def test_bad_arguments_raise(cuda):
    _say("argument errors")
    q = torch.randn(2, 2, 16, 64, device=cuda)
    with pytest.raises(ValueError):
        torch.ops.ebr_fused.attn_fwd(q, q[:, :, :8], q, 0.125)
    with pytest.raises(ValueError):
        torch.ops.ebr_fused.attn_fwd(q, q.half(), q, 0.125)
    with pytest.raises(TypeError):
        torch.ops.ebr_fused.attn_fwd(q.to(torch.int32), q.to(torch.int32), q.to(torch.int32), 0.125)
    with pytest.raises(ValueError):  # D > 256: no kernels that wide
        x = torch.randn(1, 1, 4, 264, device=cuda)
        torch.ops.ebr_fused.attn_fwd(x, x, x, 0.1)
    with pytest.raises(ValueError):  # fp64 kernels: D <= 256 too
        x = torch.randn(1, 1, 4, 260, device=cuda, dtype=torch.float64)
        torch.ops.ebr_fused.attn_fwd(x, x, x, 0.1)
    with pytest.raises(ValueError):  # rows but no head dim
        x = torch.randn(1, 1, 4, 0, device=cuda)
        torch.ops.ebr_fused.attn_fwd(x, x, x, 0.1)
    assert math.isfinite(1.0)


# ---------------------------------------------------------------------------------------------------------------------
# Launcher keywords (reference triton_kernels.py:15-17, 566-591)
# ---------------------------------------------------------------------------------------------------------------------


@pytest.mark.parametrize("L", [81, 200])
def test_launcher_lowp_dots(cuda, L):
    """``kernels.attn_*`` on bf16 inputs. lowp_dots=True (the default) is the ops' path, bit for bit. lowp_dots=False
    keeps the derived tiles in fp32: each output is then the oracle's fp32 result on the same bf16 values, rounded
    once to bf16, so it lies within one bf16 step (2^-7 of the largest output) of the oracle, well inside the 2e-2
    bar of the 16-bit tiles; lse is fp32 and within the fp32 bar."""
    from ebr_amd.fused_attn import kernels

    B, H, D = 2, 2, 64
    _say(f"launcher lowp_dots L={L}")
    q, k, v, do, gq, gk, gv = _inputs(B, H, L, D, torch.bfloat16, seed=L)
    scale = D**-0.5
    qd, kd, vd, dod, gqd, gkd, gvd = (x.to(cuda) for x in (q, k, v, do, gq, gk, gv))

    def run(**kw):
        o, lse = kernels.attn_fwd(qd, kd, vd, scale, **kw)
        dq, dk, dv = kernels.attn_bwd(qd, kd, vd, o, lse, dod, scale, **kw)
        hs = kernels.attn_bwd_bwd(qd, kd, vd, o, lse, dod, dq, gqd, gkd, gvd, scale, **kw)
        torch.cuda.synchronize()
        return [x.cpu() for x in (o, lse, dq, dk, dv, *hs)]

    ops_path = _hip_all(q, k, v, do, gq, gk, gv, scale, cuda)
    for a, b in zip(run(), ops_path):
        assert torch.equal(a, b)
    wide = run(lowp_dots=False)
    assert all(t.dtype == (torch.float32 if n == "lse" else torch.bfloat16) for n, t in zip(NAMES, wide))
    ref = _oracle_all(q, k, v, do, gq, gk, gv, scale, o=wide[0], lse=wide[1])
    errs = {n: oracle.rel_err(g, r) for n, g, r in zip(NAMES, wide, ref)}
    print(f"lowp_dots=False L={L}: " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    assert errs["lse"] <= TOL[torch.float32] and all(e <= 2.0**-7 for n, e in errs.items() if n != "lse"), errs


def test_launcher_input_precision_fp32(cuda):
    """Every input_precision the reference accepts runs the same IEEE fp32 dots on gfx950: identical outputs."""
    from ebr_amd.fused_attn import kernels

    _say("launcher input_precision fp32")
    q, k, v, do, gq, gk, gv = (x.to(cuda) for x in _inputs(2, 2, 64, 64, torch.float32, seed=5))
    outs = []
    for prec in kernels.PRECISIONS:
        o, lse = kernels.attn_fwd(q, k, v, 0.125, input_precision=prec)
        dq, dk, dv = kernels.attn_bwd(q, k, v, o, lse, do, 0.125, input_precision=prec)
        hs = kernels.attn_bwd_bwd(q, k, v, o, lse, do, dq, gq, None, gv, 0.125, input_precision=prec)
        outs.append([x.cpu() for x in (o, lse, dq, dk, dv, *hs)])
    for other in outs[1:]:
        assert all(torch.equal(a, b) for a, b in zip(outs[0], other))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rising", [True, False])
def test_long_forward_moving_maximum(cuda, dtype, rising):
    """The long forward takes a stage's exponentials against the running reference point and redoes the stage with
    the row maximum only when a row's sum of them leaves the operand type's safe range (2^32 for bf16, 2^15 for
    fp16). It takes the short stage (keys 320..332 here) first, then keys 0..319 in 64-key stages. Keys scaled by a
    ramp in that order make the stage maxima rise ~35 log2 units per stage, past that bound every time (rising), or
    sit in the first stage taken (falling); every output still matches the oracle."""
    B, H, L, D = 1, 2, 333, 64
    _say(f"long forward moving maximum {str(dtype).split('.')[-1]} rising={rising}")
    q, k, v, do, gq, gk, gv = _inputs(B, H, L, D, torch.float32, seed=7)
    ramp = torch.linspace(0.0, 1.0, L)
    ramp[320:] = 0.0  # the short stage, taken first
    if not rising:
        ramp = 1.0 - ramp
    k = k * (1.0 + 59.0 * ramp)[None, None, :, None]  # score spread 1 -> 60
    q, k, v, do, gq, gk, gv = (t.to(dtype) for t in (q, k, v, do, gq, gk, gv))
    scale = D**-0.5
    got = _hip_all(q, k, v, do, gq, gk, gv, scale, cuda)
    ref = _oracle_all(q, k, v, do, gq, gk, gv, scale, o=got[0], lse=got[1])
    _compare(got, ref, dtype, f"moving maximum rising={rising}")


@pytest.mark.parametrize("scale", [-0.2, 0.0, 0.37])
@pytest.mark.parametrize("L,dtype", [(81, torch.bfloat16), (200, torch.bfloat16), (900, torch.float16),
                                     (81, torch.float32), (150, torch.float32)])
def test_any_scale(cuda, L, dtype, scale):
    """The scale is any float, as in the reference's ops: negative (the row maximum of the scaled scores is then
    the scale times the row minimum), zero (uniform P) or large; every kernel family matches the oracle."""
    B, H, D = 1, 2, 64
    _say(f"scale={scale} L={L} {str(dtype).split('.')[-1]}")
    q, k, v, do, gq, gk, gv = _inputs(B, H, L, D, dtype, seed=11)
    got = _hip_all(q, k, v, do, gq, gk, gv, scale, cuda)
    ref = _oracle_all(q, k, v, do, gq, gk, gv, scale, o=got[0], lse=got[1])
    _compare(got, ref, dtype, f"scale={scale} L={L}")


@pytest.mark.parametrize("B,H,L", [(52000, 8, 81), (4700, 8, 900)])
def test_more_than_2_31_elements(cuda, B, H, L):
    """Tensors of more than 2^31 elements (B H L D = 2.16e9 at D = 64, 4.3 GB each in bf16): every kernel family
    (the persistent L = 81 kernels, the long L = 900 kernels) forms its offsets in 64 bits. Inputs are drawn on the
    GPU; the last slices (offsets past 2^31 elements) and a few random ones are checked against the oracle."""
    D, dtype = 64, torch.bfloat16
    assert B * H * L * D > 2**31
    _say(f"more than 2^31 elements B={B} H={H} L={L}")
    g = torch.Generator(device=cuda).manual_seed(3)
    t = [torch.randn((B, H, L, D), generator=g, device=cuda, dtype=torch.float32).to(dtype) for _ in range(7)]
    for i in range(3):
        t[i].mul_(0.125)
    q, k, v, do, gq, gk, gv = t
    scale = D**-0.5
    o, lse = torch.ops.ebr_fused.attn_fwd(q, k, v, scale)
    dq, dk, dv = torch.ops.ebr_fused.attn_bwd(q, k, v, o, lse, do, scale)
    hq, hk, hv, hdo = torch.ops.ebr_fused.attn_bwd_bwd(q, k, v, o, lse, do, dq, gq, gk, gv, scale)
    torch.cuda.synchronize()
    gen = torch.Generator().manual_seed(5)
    idx = torch.cat([torch.arange(B * H - 4, B * H), torch.randint(0, B * H, (4,), generator=gen)]).to(cuda)

    def pick(x):
        return x.reshape(B * H, *x.shape[2:])[idx].unsqueeze(0).cpu()

    got = [pick(x) for x in (o, lse, dq, dk, dv, hq, hk, hv, hdo)]
    sub = [pick(x) for x in t]
    del t, q, k, v, do, gq, gk, gv, o, lse, dq, dk, dv, hq, hk, hv, hdo
    torch.cuda.empty_cache()
    ref = _oracle_all(*sub, scale, o=got[0], lse=got[1])
    _compare(got, ref, dtype, f"more than 2^31 elements L={L}")


# Forced kernel families (kernels.PLAN_OVERRIDE over the C ABI's *_plan entry points): every family on shapes it
# runs, each checked against the oracle; a family that does not run the shape raises ValueError.
PLAN_CASES = [
    # (B, H, L, D, dtype, {op key: (families that run, families that raise)})
    (2, 3, 81, 64, torch.bfloat16, {"fwd": ("generic resident", "persistent long"),
                                    "bwd_mode": ("generic resident persistent", "long"),
                                    "bob_mode": ("generic resident persistent", "long")}),
    (2, 2, 100, 64, torch.bfloat16, {"bwd_mode": ("generic resident persistent", "long"),
                                     "bob_mode": ("generic resident", "persistent long")}),
    (2, 2, 100, 128, torch.float16, {"fwd": ("generic resident", "long"),
                                     "bwd_mode": ("generic resident persistent", "long"),
                                     "bob_mode": ("generic resident", "persistent")}),
    (2, 2, 200, 64, torch.bfloat16, {"fwd": ("generic long", "resident persistent"),
                                     "bwd_mode": ("generic long", "resident persistent"),
                                     "bob_mode": ("generic long", "resident persistent")}),
    (2, 2, 200, 128, torch.bfloat16, {"fwd": ("generic long", "resident"),
                                      "bwd_mode": ("generic long", "resident persistent"),
                                      "bob_mode": ("generic long", "resident persistent")}),
    (2, 2, 81, 256, torch.bfloat16, {"fwd": ("generic", "resident long"),
                                     "bwd_mode": ("generic", "resident persistent long"),
                                     "bob_mode": ("generic", "resident persistent long")}),
    (2, 2, 81, 64, torch.float32, {"fwd": ("generic", "resident long"), "bwd_mode": ("generic", "persistent"),
                                   "bob_mode": ("generic", "resident persistent long")}),
]


@pytest.mark.parametrize("case", range(len(PLAN_CASES)))
def test_forced_plans(cuda, case, monkeypatch):
    from ebr_amd.fused_attn import kernels

    B, H, L, D, dtype, plans = PLAN_CASES[case]
    q, k, v, do, gq, gk, gv = _inputs(B, H, L, D, dtype, seed=case)
    scale = D**-0.5
    t = [x.to(cuda) for x in (q, k, v, do, gq, gk, gv)]
    ref = None
    for key, (run, refuse) in plans.items():
        for fam in run.split():
            label = f"plan {key}={fam} B={B} H={H} L={L} D={D} {str(dtype).split('.')[-1]}"
            _say(label)
            monkeypatch.setattr(kernels, "PLAN_OVERRIDE", {key: fam})
            o, lse = kernels.attn_fwd(*t[:3], scale)
            dq, dk, dv = kernels.attn_bwd(*t[:3], o, lse, t[3], scale)
            hs = kernels.attn_bwd_bwd(*t[:3], o, lse, t[3], dq, *t[4:], scale)
            torch.cuda.synchronize()
            got = [x.cpu() for x in (o, lse, dq, dk, dv, *hs)]
            ref = _oracle_all(q, k, v, do, gq, gk, gv, scale, o=got[0], lse=got[1])
            _compare(got, ref, dtype, label)
        for fam in refuse.split():
            monkeypatch.setattr(kernels, "PLAN_OVERRIDE", {key: fam})
            o, lse = kernels.attn_fwd(*t[:3], scale) if key != "fwd" else (None, None)
            with pytest.raises(ValueError, match="plan"):
                if key == "fwd":
                    kernels.attn_fwd(*t[:3], scale)
                elif key == "bwd_mode":
                    kernels.attn_bwd(*t[:3], o, lse, t[3], scale)
                else:
                    kernels.attn_bwd_bwd(*t[:3], o, lse, t[3], None, *t[4:], scale)


REF_PLAN_CASES = [
    # (B, H, L, D, dtype, PLAN_OVERRIDE written against the reference's launchers)
    (2, 3, 81, 64, torch.bfloat16, {"fwd": (64, 32, 4, 3), "bwd_mode": "single", "bwd_single": (32, 128, 4, 1),
                                    "bob_mode": "single", "bob_single": (16, 128, 4, 1)}),
    (2, 3, 81, 64, torch.bfloat16, {"bwd_mode": "two", "bob_mode": "two", "bwd_col": (64, 64, 4, 3),
                                    "bob_row": (64, 32, 4, 3), "bob_col": (64, 64, 4, 2)}),
    (2, 2, 200, 64, torch.bfloat16, {"fwd": (64, 64, 4, 3), "bwd_mode": "two", "bob_mode": "two"}),
    (2, 2, 81, 64, torch.float32, {"fwd": (128, 32, 8, 3), "bwd_mode": "two", "bob_mode": "single"}),
]


@pytest.mark.parametrize("case", range(len(REF_PLAN_CASES)))
def test_reference_plan_override_values(cuda, case, monkeypatch):
    """PLAN_OVERRIDE dictionaries in the reference's own form (block-shape tuples, 'single' / 'two' modes) run the
    launchers to the oracle's values."""
    from ebr_amd.fused_attn import kernels

    B, H, L, D, dtype, override = REF_PLAN_CASES[case]
    _say(f"reference-style plan override {override} B={B} H={H} L={L} D={D} {str(dtype).split('.')[-1]}")
    q, k, v, do, gq, gk, gv = _inputs(B, H, L, D, dtype, seed=40 + case)
    scale = D**-0.5
    t = [x.to(cuda) for x in (q, k, v, do, gq, gk, gv)]
    monkeypatch.setattr(kernels, "PLAN_OVERRIDE", override)
    o, lse = kernels.attn_fwd(*t[:3], scale)
    dq, dk, dv = kernels.attn_bwd(*t[:3], o, lse, t[3], scale)
    hs = kernels.attn_bwd_bwd(*t[:3], o, lse, t[3], dq, *t[4:], scale)
    torch.cuda.synchronize()
    got = [x.cpu() for x in (o, lse, dq, dk, dv, *hs)]
    ref = _oracle_all(q, k, v, do, gq, gk, gv, scale, o=got[0], lse=got[1])
    _compare(got, ref, dtype, f"reference-style plan override case {case}")


def _random_cases(n, seed=2024, dmin=1, dmax=128):
    g = torch.Generator().manual_seed(seed)
    out = []
    for i in range(n):
        dtype = [torch.float32, torch.bfloat16, torch.float16][int(torch.randint(0, 3, (1,), generator=g))]
        L = int(torch.randint(1, 320, (1,), generator=g))
        D = int(torch.randint(dmin, dmax + 1, (1,), generator=g))
        B = int(torch.randint(1, 4, (1,), generator=g))
        H = int(torch.randint(1, 4, (1,), generator=g))
        out.append((i, B, H, L, D, dtype))
    return out


@pytest.mark.parametrize("i,B,H,L,D,dtype", _random_cases(40))
def test_random_shapes(cuda, i, B, H, L, D, dtype):
    """Seeded random shapes (any L up to 319, any head dim up to 128, three dtypes, small B and H): whatever plan
    and padding the ops pick, every output matches the oracle."""
    _case(B, H, L, D, dtype, cuda, seed=100 + i)


@pytest.mark.parametrize("i,B,H,L,D,dtype", _random_cases(8, seed=77, dmin=129, dmax=256))
def test_random_wide_shapes(cuda, i, B, H, L, D, dtype):
    """Seeded random shapes with head dims 129..256 (the 256-wide streamed kernels, padded widths included)."""
    _case(B, H, L, D, dtype, cuda, seed=300 + i)
