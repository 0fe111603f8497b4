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


def test_compiled_energy_grad_matches_eager(cuda):
    """dE/dz through torch.compile (aot_eager) and torch.func.grad around the fused ops: the reference's second-order
    gate passes, and a graded training step and a non-graded descent match the eager ones."""
    print("[case] compiled energy gradient", flush=True)
    cfg = en.EnergyConfig(hidden_size=64, num_heads=4, grid=(4, 4), attn_backend="fused", attn_nograd_backend="fused")
    model, dec = en.build(cfg, cuda, seed=5)
    g = torch.Generator("cpu").manual_seed(6)
    B, L = 3, 16
    x = torch.randint(0, 11, (B, L), generator=g).to(cuda)
    z0 = torch.randn(B, L, 64, generator=g).to(cuda)
    tg = torch.randint(0, 11, (B, L), generator=g).to(cuda)
    compiled = en.compiled_energy_grad(model)
    for module in model.modules():
        if hasattr(module, "_ensure_verified"):
            module._ensure_verified(cuda, torch.float32)
    errs = en.verify_compiled_energy_grad(model, compiled, z0, model.puzzle_embedding(x, z0.dtype))
    print("compiled vs eager:", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)

    lc = en.train_step(model, dec, x, z0, tg, steps=3, compiled=compiled)
    gc = {n: p.grad.clone() for n, p in model.named_parameters() if p.grad is not None}
    model.zero_grad(set_to_none=True)
    dec.zero_grad(set_to_none=True)
    le = en.train_step(model, dec, x, z0, tg, steps=3)
    assert abs(float(lc) - float(le)) <= 1e-5 * max(1.0, abs(float(le)))
    for n, p in model.named_parameters():
        if p.grad is None:
            continue
        err = float((gc[n] - p.grad).abs().max() / p.grad.abs().max().clamp_min(1e-12))
        assert err <= 1e-4, (n, err)

    x_emb = model.puzzle_embedding(x, z0.dtype).detach()
    vc = en.descend(model, z0, x_emb, 4, 0.1, create_graph=False, compiled=compiled)
    ve = en.descend(model, z0, x_emb, 4, 0.1, create_graph=False)
    vc, ve = vc.detach(), ve.detach()
    assert float((vc - ve).abs().max()) <= 1e-4 * float(ve.abs().max())


def test_graph_train_step_replays_match_eager(cuda):
    """The config-3 step (fused RoPE, block and split-K gradients, bf16) captured in a HIP graph: three replays, each
    on new latents copied into the static input and with eager steps of a twin model run between the replays, give
    the eager step's loss and gradients on the same inputs."""
    print("[case] graph-captured train step bf16", flush=True)
    kw = dict(hidden_size=128, num_heads=2, grid=(9, 9), attn_backend="fused", attn_nograd_backend="fused",
              rope_impl="fused", block_impl="fused", linear_impl="splitk")
    mg, dg = en.build(en.EnergyConfig(**kw), cuda, seed=5)
    me, de = en.build(en.EnergyConfig(**kw), cuda, seed=5)
    g = torch.Generator("cpu").manual_seed(6)
    B, L = 4, 81
    x = torch.randint(0, 11, (B, L), generator=g).to(cuda)
    tg = torch.randint(0, 11, (B, L), generator=g).to(cuda)
    z0 = torch.randn(B, L, 128, generator=g).to(cuda, torch.bfloat16)
    graph, loss = en.graph_train_step(mg, dg, x, z0, tg, steps=3)
    for rep in range(3):
        z0.copy_(torch.randn(B, L, 128, generator=g).to(cuda, torch.bfloat16))
        graph.replay()
        me.zero_grad(set_to_none=True)
        de.zero_grad(set_to_none=True)
        le = en.train_step(me, de, x, z0, tg, steps=3)  # eager work between the replays
        torch.cuda.synchronize()
        assert torch.isfinite(loss) and abs(float(loss) - float(le)) <= 1e-4 * abs(float(le)), (rep, loss, le)
        for (n, pg), (_, pe) in zip((*mg.named_parameters(), *dg.named_parameters()),
                                    (*me.named_parameters(), *de.named_parameters())):
            if pe.grad is None:
                assert pg.grad is None, n
                continue
            err = float((pg.grad.float() - pe.grad.float()).abs().max() / pe.grad.float().abs().max().clamp_min(1e-12))
            assert err <= 1e-3, (rep, n, err)
