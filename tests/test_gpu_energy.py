"""The EBR harness on the GPU: a graded latent-descent training step and an inference descent through the fused
attention agree with the same steps through the eager math attention (fp32, small sizes)."""

import pytest
import torch

from ebr_amd import energy as en

pytestmark = pytest.mark.gpu


def _pair(grid=(4, 4), hidden=64, heads=4):
    models = []
    for backend in ("fused", "math"):
        cfg = en.EnergyConfig(hidden_size=hidden, num_heads=heads, grid=grid, attn_backend=backend,
                              attn_nograd_backend=backend)
        models.append(en.build(cfg, torch.device("cuda", 0), seed=3))
    return models


def test_train_step_fused_matches_math(cuda):
    print("[case] energy train step fp32", flush=True)
    (mf, df), (mm, dm) = _pair()
    g = torch.Generator("cpu").manual_seed(1)
    B, L = 3, 16
    x = torch.randint(0, 11, (B, L), generator=g).to(cuda)
    z0 = torch.randn(B, L, 64, generator=g).to(cuda)
    tg = torch.randint(0, 11, (B, L), generator=g).to(cuda)
    lf = en.train_step(mf, df, x, z0, tg, steps=4)
    lm = en.train_step(mm, dm, x, z0, tg, steps=4)
    assert abs(float(lf) - float(lm)) <= 1e-5 * max(1.0, abs(float(lm)))
    for (n, pf), (_, pm) in zip(mf.named_parameters(), mm.named_parameters()):
        if pm.grad is None:
            continue
        err = float((pf.grad - pm.grad).abs().max() / pm.grad.abs().max().clamp_min(1e-12))
        assert err <= 1e-4, (n, err)


def test_train_step_bf16_runs_and_is_close(cuda):
    print("[case] energy train step bf16", flush=True)
    (mf, df), (mm, dm) = _pair(grid=(9, 9), hidden=128, heads=2)
    g = torch.Generator("cpu").manual_seed(2)
    B, L = 4, 81
    x = torch.randint(0, 11, (B, L), generator=g).to(cuda)
    z0 = torch.randn(B, L, 128, generator=g).to(cuda, torch.bfloat16)
    tg = torch.randint(0, 11, (B, L), generator=g).to(cuda)
    lf = en.train_step(mf, df, x, z0, tg, steps=3)
    lm = en.train_step(mm, dm, x, z0, tg, steps=3)
    assert torch.isfinite(lf) and abs(float(lf) - float(lm)) <= 2e-2 * abs(float(lm))


def test_infer_fused_matches_math(cuda):
    print("[case] energy inference", flush=True)
    (mf, _), (mm, _) = _pair(grid=(5, 5))
    for m in (mf, mm):
        for p in m.parameters():
            p.requires_grad_(False)
    g = torch.Generator("cpu").manual_seed(3)
    x = torch.randint(0, 3, (3, 25), generator=g).to(cuda)
    z0 = torch.randn(3 * 4, 25, 64, generator=g).to(cuda)
    vf, ef = en.infer(mf, x, z0, samples=4, steps=5)
    vm, em = en.infer(mm, x, z0, samples=4, steps=5)
    assert torch.allclose(ef, em, rtol=1e-4, atol=1e-5)
    assert float((vf - vm).abs().max()) <= 1e-3
