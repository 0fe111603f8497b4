"""ebr_attn_bwd_bwd_noalloc (the entry point that allocates nothing) against ebr_attn_bwd_bwd, through the C ABI.

Both run the same kernels; the no-allocation entry takes the two-launch shapes' row-statistics scratch from the
library's own per-GPU device array instead of a caller buffer, so the outputs must be bit-identical. Two calls in a
row, the second smaller than the first (the array keeps the first call's contents), then a shape that needs no
scratch, each checked against the scratch-taking entry point.
"""

import ctypes

import pytest
import torch

import oracle
from ebr_amd import _capi
from ebr_amd.fused_attn import ops  # noqa: F401  (registers torch.ops.ebr_fused.*)

pytestmark = pytest.mark.gpu

CODE = {torch.bfloat16: _capi.DTYPE_BF16, torch.float16: _capi.DTYPE_F16, torch.float32: _capi.DTYPE_F32}


def _run(lib, entry, B, H, L, D, dtype, seed, dev):
    q, k, v, do, gq, gk, gv = (t.to(dev) for t in oracle.make_inputs(B, H, L, D, dtype=dtype, seed=seed,
                                                                      qkv_scale=0.125))
    scale = D**-0.5
    o, lse = torch.ops.ebr_fused.attn_fwd(q, k, v, scale)
    outs = [torch.full_like(q, float("nan")) for _ in range(4)]
    s3 = _capi.strides3
    args = [CODE[dtype], B, H, L, D, ctypes.c_float(scale), q.data_ptr(), s3(q), k.data_ptr(), s3(k), v.data_ptr(),
            s3(v), o.data_ptr(), lse.data_ptr(), do.data_ptr(), s3(do), gq.data_ptr(), s3(gq), gk.data_ptr(), s3(gk),
            gv.data_ptr(), s3(gv), *(t.data_ptr() for t in outs)]
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    scratch = None
    if entry == "ebr_attn_bwd_bwd":
        nbytes = int(lib.ebr_attn_scratch_bytes(_capi.OP_BWD_BWD, B, H, L, D))
        scratch = torch.full((max(1, nbytes // 4),), float("nan"), device=dev) if nbytes else None
        args.append(scratch.data_ptr() if scratch is not None else None)
    args.append(stream)
    with torch.cuda.device(dev):
        rc = getattr(lib, entry)(*args)
    _capi.check(rc, entry)
    torch.cuda.synchronize()
    return [t.cpu() for t in outs]


@pytest.mark.parametrize("shape", [(6, 8, 900, 64, torch.bfloat16), (2, 4, 300, 64, torch.bfloat16),
                                   (3, 4, 81, 64, torch.bfloat16), (2, 2, 200, 32, torch.float16)])
def test_noalloc_equals_scratch_entry(cuda, shape):
    B, H, L, D, dtype = shape
    print(f"[case] noalloc B={B} H={H} L={L} D={D} {dtype}", flush=True)
    lib = _capi.load()
    want = _run(lib, "ebr_attn_bwd_bwd", B, H, L, D, dtype, L, cuda)
    got = _run(lib, "ebr_attn_bwd_bwd_noalloc", B, H, L, D, dtype, L, cuda)
    for name, g, w in zip(("hq", "hk", "hv", "hdo"), got, want):
        assert torch.isfinite(g.float()).all(), name
        assert torch.equal(g, w), name


def test_noalloc_two_calls_second_smaller(cuda):
    print("[case] noalloc two calls, second smaller", flush=True)
    lib = _capi.load()
    for B, H, L in ((8, 8, 700, ), (1, 2, 257)):
        want = _run(lib, "ebr_attn_bwd_bwd", B, H, L, 64, torch.bfloat16, 3, cuda)
        got = _run(lib, "ebr_attn_bwd_bwd_noalloc", B, H, L, 64, torch.bfloat16, 3, cuda)
        for g, w in zip(got, want):
            assert torch.equal(g, w)


def test_noalloc_rejects_oversize_shape(cuda):
    lib = _capi.load()
    B, H, L, D = 600, 8, 900, 64  # 3 * B * H * L * 4 bytes > EBR_NOALLOC_SCRATCH_BYTES
    assert 3 * B * H * L * 4 > _capi.NOALLOC_SCRATCH_BYTES
    z = (ctypes.c_int64 * 3)(0, 0, 0)
    rc = lib.ebr_attn_bwd_bwd_noalloc(_capi.DTYPE_BF16, B, H, L, D, ctypes.c_float(0.125), *([16, z] * 3), 16, 16,
                                      *([16, z] * 4), 16, 16, 16, 16, None)
    assert rc == _capi.ERR_NOALLOC_SIZE
