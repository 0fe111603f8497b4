"""ebr_attn_bwd_bwd_noalloc (the entry point that allocates nothing) against ebr_attn_bwd_bwd, through the C ABI.

Both run the same kernels; the no-allocation entry takes the two-launch shapes' row-statistics scratch from the
library's own per-GPU device array instead of a caller buffer, so the outputs must be bit-identical. Two calls in a
row, the second smaller than the first (the array keeps the first call's contents), then a shape that needs no
scratch, each checked against the scratch-taking entry point. Then, in a fresh process, the entry's first call on
the device made inside a ``torch.cuda.graph`` capture (its per-device lookup then runs under capture), the graph
replayed and each replay compared bit for bit with the scratch-taking entry point. The rejection of shapes beyond the
array is checked on the CPU (``tests/test_capi.py``), since it needs no GPU.
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
                                   (3, 4, 81, 64, torch.bfloat16), (2, 2, 200, 32, torch.float16),
                                   (2, 2, 40, 256, torch.bfloat16), (2, 2, 150, 128, torch.bfloat16)])
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


CAPTURE_CHILD = r"""
import ctypes, sys, torch
sys.path.insert(0, sys.argv[1])
import oracle
from ebr_amd import _capi
from ebr_amd.fused_attn import ops  # noqa: F401
dev = torch.device("cuda", 0)
lib = _capi.load()
B, H, L, D = 4, 4, 300, 64
q, k, v, do, gq, gk, gv = (t.to(dev) for t in oracle.make_inputs(B, H, L, D, dtype=torch.bfloat16, seed=11,
                                                                  qkv_scale=0.125))
scale = D ** -0.5
o, lse = torch.ops.ebr_fused.attn_fwd(q, k, v, scale)
s3 = _capi.strides3
outs = [torch.full_like(q, float("nan")) for _ in range(4)]
ins = [q.data_ptr(), s3(q), k.data_ptr(), s3(k), v.data_ptr(), s3(v), o.data_ptr(), lse.data_ptr(), do.data_ptr(),
       s3(do), gq.data_ptr(), s3(gq), gk.data_ptr(), s3(gk), gv.data_ptr(), s3(gv)]
head = [_capi.DTYPE_BF16, B, H, L, D, ctypes.c_float(scale)]
want = [torch.empty_like(q) for _ in range(4)]
nbytes = int(lib.ebr_attn_scratch_bytes(_capi.OP_BWD_BWD, B, H, L, D))
scratch = torch.empty(nbytes // 4, device=dev)
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):  # the entry's first call in this process: its device lookup runs under capture
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)  # the capture stream
    rc = lib.ebr_attn_bwd_bwd_noalloc(*head, *ins, *(t.data_ptr() for t in outs), st)
_capi.check(rc, "ebr_attn_bwd_bwd_noalloc under capture")
st0 = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
_capi.check(lib.ebr_attn_bwd_bwd(*head, *ins, *(t.data_ptr() for t in want), scratch.data_ptr(), st0),
            "ebr_attn_bwd_bwd")
torch.cuda.synchronize()
for rep in range(3):
    for t in outs:
        t.fill_(float("nan"))
    # eager work on the same device between replays (the library's other entry, torch kernels)
    torch.ops.ebr_fused.attn_fwd(q * 0.5, k, v, scale)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    for name, a, b in zip(("hq", "hk", "hv", "hdo"), outs, want):
        assert torch.equal(a, b), (rep, name)
print("capture ok: 3 replays bit-identical", flush=True)
"""


def test_noalloc_first_call_inside_graph_capture(cuda, tmp_path):
    """The first call of the entry on a device made inside graph capture (a fresh process, so no earlier call has
    looked the array up), replayed three times with eager work between, each replay equal bit for bit to
    ebr_attn_bwd_bwd."""
    import subprocess
    import sys
    from pathlib import Path

    print("[case] noalloc first call inside torch.cuda.graph capture (child process)", flush=True)
    root = str(Path(__file__).resolve().parents[1])
    script = tmp_path / "capture_child.py"
    script.write_text(CAPTURE_CHILD)
    proc = subprocess.run([sys.executable, "-u", str(script), root], capture_output=True, text=True, timeout=110)
    print(proc.stdout[-2000:], proc.stderr[-2000:], flush=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    assert "capture ok" in proc.stdout
