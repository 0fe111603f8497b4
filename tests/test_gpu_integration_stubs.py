"""The maintainer-facing ctypes stubs of the integration guide, run exactly as written there (only the library path
filled in): the attention launchers against the CPU oracle, the RoPE split / merge launchers against the oracle's
closed forms (bit for bit, as the ops are), the descent launchers against this package's descent ops (bit for bit).

A stub that drifts from the C ABI (an argument added, reordered or retyped) fails here rather than in a
maintainer's hands.
"""

import os
import re

import pytest
import torch

import oracle
from ebr_amd import _capi, descent
from ebr_amd.fused_attn import ops  # noqa: F401  (registers torch.ops.ebr_fused.*)

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GUIDE = os.path.join(ROOT, "INTEGRATION.md")


def _stub(first_line: str) -> dict:
    """Execute the guide's python block that starts with ``first_line``; returns its namespace."""
    with open(GUIDE) as f:
        text = f.read()
    for block in re.findall(r"```python\n(.*?)```", text, re.S):
        if block.startswith(first_line):
            src = block.replace('"/path/to/ebr_amd/_lib/libebr_attn.so"', repr(str(_capi.LIB_PATH)))
            assert src != block, "the stub no longer loads the library from the placeholder path"
            ns: dict = {}
            exec(compile(src, f"<stub {first_line}>", "exec"), ns)
            return ns
    raise AssertionError(f"no stub starting with {first_line!r}")


def _say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.mark.parametrize("L,dtype", [(81, torch.bfloat16), (200, torch.bfloat16), (45, torch.float16), (64, torch.float32)])
def test_attention_stub_matches_oracle(cuda, L, dtype):
    stub = _stub("# models/fused_attn/hip_kernels.py")
    B, H, D = 2, 3, 64
    _say(f"attention stub L={L} {dtype}")
    scale = 0.125 if dtype != torch.float32 else None
    q, k, v, do, gq, gk, gv = oracle.make_inputs(B, H, L, D, dtype=dtype, seed=L, qkv_scale=scale)
    t = [x.to(cuda) for x in (q, k, v, do, gq, gk, gv)]
    s = D**-0.5
    o, lse = stub["attn_fwd"](t[0], t[1], t[2], s)
    dq, dk, dv = stub["attn_bwd"](t[0], t[1], t[2], o, lse, t[3], s)
    hs = stub["attn_bwd_bwd"](t[0], t[1], t[2], o, lse, t[3], dq, t[4], None, t[6], s)
    torch.cuda.synchronize()
    got = [x.cpu() for x in (o, lse, dq, dk, dv, *hs)]
    ro, rlse = oracle.attn_fwd(q, k, v, s)
    rdq, rdk, rdv = oracle.attn_bwd(q, k, v, got[0], got[1], do, s)
    rh = oracle.attn_bwd_bwd(q, k, v, got[0], got[1], do, rdq, gq, torch.zeros_like(gk), gv, s)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for name, a, r in zip(["o", "lse", "dq", "dk", "dv", "hq", "hk", "hv", "hdo"], got, [ro, rlse, rdq, rdk, rdv, *rh]):
        err = oracle.rel_err(a, r)
        assert err <= tol, f"{name}: {err:.2e} > {tol}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rope_stub_matches_oracle_exactly(cuda, dtype):
    stub = _stub("# models/fused_attn/rope_split_hip.py")
    B, N, H, D = 2, 81, 4, 64
    _say(f"rope stub {dtype}")
    qkv, (gq, gk, gv) = oracle.make_rope_inputs(B, N, H, D, dtype=dtype, seed=5)
    h, w = oracle.grid_shape(N)
    cos, sin = oracle.rotary_tables(D, h, w)
    qs = torch.linspace(0.5, 1.5, H)
    q, k, v = stub["rope_split"](qkv.to(cuda), cos.to(cuda), sin.to(cuda), H, qs.to(cuda))
    g = stub["rope_merge"](gq.to(cuda), gk.to(cuda), gv.to(cuda), cos.to(cuda), sin.to(cuda), qs.to(cuda))
    torch.cuda.synchronize()
    for a, r in zip((q, k, v), oracle.ref_split(qkv, cos, sin, H, qs)):
        assert torch.equal(a.cpu(), r)
    assert torch.equal(g.cpu(), oracle.ref_merge(gq, gk, gv, cos, sin, qs))


def test_descent_stub_matches_the_ops_exactly(cuda):
    stub = _stub("# models/descent_hip.py")
    B, L, C = 6, 81, 512
    _say("descent stub")
    gen = torch.Generator(device=cuda).manual_seed(9)
    z, noise, v, g = (torch.randn(B, L, C, generator=gen, device=cuda).to(torch.bfloat16) for _ in range(4))
    sigma = torch.rand(B, 1, 1, generator=gen, device=cuda).to(torch.bfloat16)
    alpha = torch.rand(B, 1, 1, generator=gen, device=cuda).to(torch.bfloat16)
    active = torch.tensor([True, False, True, True, False, True], device=cuda).reshape(B, 1, 1)
    eps = descent.RMS_NORM_EPS
    assert torch.equal(stub["noisy_point"](z, noise, sigma, eps), descent.noisy_point(z, noise, sigma, eps))
    assert torch.equal(stub["noisy_point"](z, noise, None, eps), descent.noisy_point_replayed(z, noise, eps))
    out, rms = stub["step_and_project"](v, g, alpha, z, active, eps)
    assert torch.equal(out, descent.step_and_project(v, g, alpha, z, active, eps))
    assert rms.shape == (B,) and torch.isfinite(rms).all()
