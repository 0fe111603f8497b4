"""Writes tests/golden/attn_small.npz: seeded fp64 inputs and the outputs of attn_fwd, attn_bwd and attn_bwd_bwd for a
few small shapes (edge cases L = 1 and L not a multiple of 16 included).

The outputs come from the CPU oracle and are accepted only if they also match torch autograd through the eager
softmax attention (first and second order) to 1e-11, so the fixture is pinned independently of the oracle's closed
forms. The reference ships no golden vectors for this path, so these are the build's own.

Run from the repo root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402

CASES = [(1, 2, 1, 16), (2, 2, 5, 16), (1, 3, 17, 32), (2, 1, 40, 64), (1, 1, 81, 32)]
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "attn_small.npz")


def main() -> None:
    arrays = {}
    for ci, (B, H, L, D) in enumerate(CASES):
        # inputs are fp32 values (stored as fp32) carried in fp64; outputs are fp64
        ins = oracle.make_inputs(B, H, L, D, dtype=torch.float32, seed=100 + ci, qkv_scale=0.5)
        q, k, v, do, gq, gk, gv = (t.double() for t in ins)
        s = D**-0.5
        o, lse = oracle.attn_fwd(q, k, v, s)
        dq, dk, dv = oracle.attn_bwd(q, k, v, o, lse, do, s)
        hq, hk, hv, hdo = oracle.attn_bwd_bwd(q, k, v, o, lse, do, dq, gq, gk, gv, s)
        first = oracle.autograd_bwd(q, k, v, do)
        second = oracle.autograd_bwd_bwd(q, k, v, do, gq, gk, gv)
        o_ref = oracle.math_attention(q, k, v)
        assert torch.allclose(o, o_ref, atol=1e-12)
        for a, b in zip((dq, dk, dv, hq, hk, hv, hdo), (*first, *second)):
            assert torch.allclose(a, b, atol=1e-11), float((a - b).abs().max())
        names = dict(q=q, k=k, v=v, do=do, gq=gq, gk=gk, gv=gv, o=o, lse=lse, dq=dq, dk=dk, dv=dv, hq=hq, hk=hk,
                     hv=hv, hdo=hdo)
        for n, t in names.items():
            arrays[f"c{ci}_{n}"] = t.float().numpy() if n in ("q", "k", "v", "do", "gq", "gk", "gv") else t.numpy()
        arrays[f"c{ci}_shape"] = np.array([B, H, L, D], dtype=np.int64)
        arrays[f"c{ci}_scale"] = np.array([s], dtype=np.float64)
    arrays["ncases"] = np.array([len(CASES)], dtype=np.int64)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(CASES)} cases)")


if __name__ == "__main__":
    main()
