"""Energy network and latent descent: the harness BASELINE configurations 3 and 4 run the attention path through.

Follows the reference's structure, restated at the size BASELINE names:
- ``ScalarEnergy`` (models/energy.py:204-216): E(z; x) from ``num_layers`` post-norm blocks
  (models/attention.py:248-266) over z + embed(x). BASELINE config 3 names a mean-pooled linear energy head, used
  here instead of the reference's per-cell MLP head (models/energy.py:190-201).
- ``energy_grad`` (models/energy.py:345-350): opens the second-order window when the graph is kept, runs the energy
  forward and takes dE/dz with ``torch.autograd.grad`` (``create_graph`` for graded steps).
- ``compiled_energy_grad`` / ``verify_compiled_energy_grad`` (models/energy.py:352-434): the same dE/dz as
  ``torch.func.grad`` of a ``functional_call``, under ``torch.compile`` with the ``aot_eager`` backend (no Triton), and
  the second-order probe that must agree with eager before the compiled gradient is used.
- ``descend``: z <- z - alpha dE/dz for ``steps`` steps, or, with ``wrapper``, the reference's full
  microstep (``microstep``, models/energy.py:293-319): v = rms_norm(z) + noise, z <- where(active, sphere(v - alpha
  dE/dv), z), its pointwise work either as the eager torch formulas (models/energy.py:219-241, the reference's
  ``descent_wrapper_compile: false``) or as the fused HIP kernels of ``ebr_amd.descent``.
- ``train_step`` (config 3): ``steps`` graded descent steps, a linear decode head, cross-entropy to targets, backward.
- ``infer`` (config 4): descent without a graph over ``samples`` latents per input, then the lowest-energy sample per
  input (evaluators/protocol.py:10-12).

The attention backend is a parameter: ``fused`` (the gfx950 kernels) on the GPU; the CPU baseline passes ``math``.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn.functional as F
from torch import nn

from ebr_amd.attention import EnergyReasoningBlock, second_order_window
from ebr_amd.layers import (
    RMS_NORM_EPS,
    CastedLinear,
    RotaryEmbedding2D,
    RotaryTable2D,
    check_linear_impl,
    rms_norm,
    trunc_normal_init_,
)


@dataclass
class EnergyConfig:
    hidden_size: int = 512
    num_heads: int = 8
    num_layers: int = 2
    expansion: float = 4.0
    vocab_size: int = 11
    grid: tuple = (9, 9)  # board height x width; L = height * width
    attn_backend: str = "fused"
    attn_nograd_backend: str = "fused"
    rope: bool = True
    rope_impl: str = "broadcast"  # "fused": the HIP RoPE split/merge (RotaryTable2D), reference rope_impl
    block_impl: str = "eager"  # "fused": rms_norm and the SwiGLU activation as HIP kernels (ebr_amd.block)
    linear_impl: str = "eager"  # "splitk": projection weight gradients as split-K GEMMs (ebr_amd.linear)


class ScalarEnergy(nn.Module):
    def __init__(self, cfg: EnergyConfig) -> None:
        super().__init__()
        self.cfg = cfg
        self.embed = nn.Parameter(trunc_normal_init_(torch.empty(cfg.vocab_size, cfg.hidden_size), std=1.0))
        self.layers = nn.ModuleList(EnergyReasoningBlock(cfg) for _ in range(cfg.num_layers))
        self.energy_head = CastedLinear(cfg.hidden_size, 1, bias=False)
        head_dim = cfg.hidden_size // cfg.num_heads
        if not cfg.rope:
            self.rope = None
        elif cfg.rope_impl == "fused":
            self.rope = RotaryTable2D(head_dim, *cfg.grid)
        elif cfg.rope_impl == "broadcast":
            self.rope = RotaryEmbedding2D(head_dim, *cfg.grid)
        else:
            raise ValueError(f"rope_impl must be 'broadcast' or 'fused', got {cfg.rope_impl!r}")

    def puzzle_embedding(self, x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
        return F.embedding(x, self.embed.to(dtype))

    def forward(self, z: torch.Tensor, x_emb: torch.Tensor) -> torch.Tensor:
        """Energy per row, fp32 [B]."""
        cos_sin = self.rope() if self.rope is not None else None
        h = z + x_emb
        for layer in self.layers:
            h = layer(cos_sin, h)
        return self.energy_head(h.mean(dim=1)).float().squeeze(-1)


def energy_grad(model: ScalarEnergy, v: torch.Tensor, x_emb: torch.Tensor, create_graph: bool) -> torch.Tensor:
    with second_order_window(create_graph):
        e = model(v, x_emb)
    (g,) = torch.autograd.grad(e.sum(), v, create_graph=create_graph)
    return g


COMPILE_BACKEND = "aot_eager"  # a non-Triton torch.compile backend


def compiled_energy_grad(model: ScalarEnergy):
    """dE/dz as ``torch.func.grad`` of the energy (a ``functional_call`` over the given parameters), compiled. Call as
    ``fn(z, x_emb, params)`` with ``params`` in ``model.named_parameters()`` order (models/energy.py:368-384)."""
    names = [n for n, _ in model.named_parameters()]

    def grad_fn(z: torch.Tensor, x_emb: torch.Tensor, params: list) -> torch.Tensor:
        weights = dict(zip(names, params, strict=True))

        def total_energy(zz: torch.Tensor) -> torch.Tensor:
            return torch.func.functional_call(model, weights, (zz, x_emb)).sum()

        return torch.func.grad(total_energy)(z)

    torch._dynamo.config.cache_size_limit = max(torch._dynamo.config.cache_size_limit, 64)
    return torch.compile(grad_fn, backend=COMPILE_BACKEND, dynamic=False)


def verify_compiled_energy_grad(model: ScalarEnergy, compiled, v: torch.Tensor, x_emb: torch.Tensor,
                                tol: float = 1e-3) -> dict:
    """The reference's gate (models/energy.py:386-434): on up to two rows in float32 with a private generator, the
    compiled dE/dz, d2E/dz2 . u and d2E/dtheta dz . u must match eager within ``tol`` (relative 2-norm), else raise.
    Returns the three errors."""
    rows = min(2, v.shape[0])
    z0 = v.detach()[:rows].float()
    x0 = x_emb.detach()[:rows].float()
    gen = torch.Generator(device=z0.device).manual_seed(1234)
    u = torch.randn(z0.shape, generator=gen, device=z0.device, dtype=z0.dtype)
    params = [p for _, p in model.named_parameters()]

    def probe(grad_fn):
        z = z0.clone().requires_grad_(True)
        with torch.enable_grad(), second_order_window(True):
            g = grad_fn(z)
            hz, *ht = torch.autograd.grad((g * u).sum(), [z] + params, allow_unused=True)
        return g.detach(), hz, ht

    def eager(z):
        return torch.autograd.grad(model(z, x0).sum(), z, create_graph=True)[0]

    prev = torch.get_float32_matmul_precision()
    torch.set_float32_matmul_precision("highest")
    try:
        ref_g, ref_hz, ref_ht = probe(eager)
        got_g, got_hz, got_ht = probe(lambda z: compiled(z, x0, params))
    finally:
        torch.set_float32_matmul_precision(prev)

    def rel(a, r):
        if r is None:
            return 0.0 if a is None else float("inf")
        if a is None:
            return float("inf")
        return float((a.float() - r.float()).norm() / r.float().norm().clamp_min(1e-12))

    errs = {
        "dE/dz": rel(got_g, ref_g),
        "d2E/dz2": rel(got_hz, ref_hz),
        "d2E/dtheta dz": max(rel(a, r) for a, r in zip(got_ht, ref_ht, strict=True)),
    }
    if not all(e < tol for e in errs.values()):
        raise RuntimeError("compiled dE/dz does not match eager: " + ", ".join(f"{k}={e:.3e}" for k, e in errs.items()))
    return errs


def _gradient(model, v, x_emb, create_graph: bool, compiled, params):
    if compiled is None:
        return energy_grad(model, v, x_emb, create_graph)
    with second_order_window(create_graph):
        if create_graph:
            return compiled(v, x_emb, params)
        with torch.no_grad():
            return compiled(v, x_emb, params)


def _verify_before_compiled(model, v, compiled, create_graph: bool) -> None:
    if compiled is not None and create_graph:
        # the attention's second-order self-test runs eagerly, before dynamo traces the module (energy.py:356-360)
        for module in model.modules():
            if hasattr(module, "_ensure_verified"):
                module._ensure_verified(v.device, v.dtype)


# -- the descent wrapper's pointwise work as eager torch formulas (reference models/energy.py:219-241) ------------------


def sphere(z: torch.Tensor, eps: float = RMS_NORM_EPS) -> torch.Tensor:
    """Each row (the whole board) rescaled to unit RMS in fp32, the RMS clamped below at ``eps``. z is cast twice, as
    the reference does, so that autograd rounds the two terms of the gradient to z's dtype separately."""
    rms = z.float().square().mean(dim=(1, 2), keepdim=True).sqrt().clamp_min(eps)
    return (z.float() / rms).to(z.dtype)


def _eager_noisy_point(z, noise, sigma, eps):
    v = rms_norm(z, eps)
    if noise is None:
        return v
    return v + noise * sigma if sigma is not None else v + noise.to(dtype=v.dtype)


def _eager_step_and_project(v, g, alpha, z, active, eps):
    z_next = sphere(v - alpha * g, eps)
    return z_next if active is None else torch.where(active, z_next, z.to(dtype=z_next.dtype))


WRAPPERS = ("eager", "fused")


def _wrapper_fns(wrapper: str):
    if wrapper == "eager":
        return _eager_noisy_point, _eager_step_and_project
    if wrapper == "fused":
        from ebr_amd import descent

        def noisy(z, noise, sigma, eps):
            if noise is None:
                return descent.normalize(z, eps)
            if sigma is None:
                return descent.noisy_point_replayed(z, noise, eps)
            return descent.noisy_point(z, noise, sigma, eps)

        return noisy, descent.step_and_project
    raise ValueError(f"wrapper must be one of {WRAPPERS}, got {wrapper!r}")


def microstep(model, z, x_emb, *, alpha, create_graph: bool, sigma=None, noise=None, active=None,
              wrapper: str = "fused", compiled=None, params=None, eps: float = RMS_NORM_EPS) -> torch.Tensor:
    """One reference descent microstep (EnergyDescent.forward, models/energy.py:293-319): v = rms_norm(z) + noise
    (``noise`` replayed as given, else drawn as randn * ``sigma`` when ``sigma`` is set, else none), g = dE/dv,
    z' = where(active, sphere(v - alpha g), z). ``alpha``/``sigma``: a float or a per-row [B, 1, 1] tensor in z's
    dtype; ``active``: a [B, 1, 1] bool mask or None."""
    noisy, step = _wrapper_fns(wrapper)
    if noise is None and sigma is not None:
        noise = torch.randn_like(z)  # drawn eagerly, as the reference does (energy.py:331-332)
    elif noise is not None:
        sigma = None
    with torch.set_grad_enabled(create_graph):
        v = noisy(z, noise, sigma, eps)
    if not v.requires_grad:
        v = v.detach().requires_grad_(True)
    g = _gradient(model, v, x_emb, create_graph, compiled, params)
    with torch.set_grad_enabled(create_graph):
        z_next = step(v, g, alpha, z, active, eps)
    return z_next if create_graph else z_next.detach()


def descend(model, z, x_emb, steps: int, alpha, create_graph: bool, compiled=None, wrapper: Optional[str] = None,
            sigma=None, noises=None, active=None) -> torch.Tensor:
    """``steps`` descent steps; with ``compiled`` (from ``compiled_energy_grad``) dE/dz comes from the compiled
    function, under the same second-order window the eager path opens. ``wrapper`` None: z <- z - alpha dE/dz;
    "eager" / "fused": the reference microstep (``microstep``) with ``sigma``, ``noises[t]`` and ``active[t]``."""
    v = z if z.requires_grad else z.detach().requires_grad_(True)
    params = [p for _, p in model.named_parameters()] if compiled is not None else None
    _verify_before_compiled(model, v, compiled, create_graph)
    for t in range(steps):
        if wrapper is not None:
            v = microstep(model, v, x_emb, alpha=alpha, create_graph=create_graph, sigma=sigma,
                          noise=None if noises is None else noises[t], active=None if active is None else active[t],
                          wrapper=wrapper, compiled=compiled, params=params)
            continue
        g = _gradient(model, v, x_emb, create_graph, compiled, params)
        v = v - alpha * g
        if not create_graph:
            v = v.detach().requires_grad_(True)
    return v


class Decoder(nn.Module):
    def __init__(self, cfg: EnergyConfig) -> None:
        super().__init__()
        self.lm_head = CastedLinear(cfg.hidden_size, cfg.vocab_size, bias=False)

    def forward(self, v: torch.Tensor) -> torch.Tensor:
        return self.lm_head(v).float()


def train_step(model, decoder, x, z0, targets, steps: int = 16, alpha=0.1, compiled=None,
               wrapper: Optional[str] = None, sigma=None, noises=None, active=None) -> torch.Tensor:
    """One config-3 training step: graded descent (create_graph), CE to ``targets``, backward. Returns the loss.
    ``wrapper`` and the rest select the reference microstep (``descend``)."""
    x_emb = model.puzzle_embedding(x, z0.dtype)
    z = z0.detach().requires_grad_(True)
    v = descend(model, z, x_emb, steps, alpha, create_graph=True, compiled=compiled, wrapper=wrapper, sigma=sigma,
                noises=noises, active=active)
    logits = decoder(v)
    loss = F.cross_entropy(logits.reshape(-1, logits.shape[-1]), targets.reshape(-1))
    loss.backward()
    return loss.detach()


def graph_train_step(model, decoder, x, z0, targets, steps: int = 16, alpha=0.1, warmup: int = 2):
    """``train_step`` captured in a HIP graph over static inputs ``x``, ``z0``, ``targets`` (config 3 with the fused
    kernels: every launch goes to torch's current stream, nothing synchronises with the host, no allocation outside
    torch's allocator). Returns ``(graph, loss)``: ``graph.replay()`` re-runs the whole step (graded descent, CE,
    backward) on the inputs' current contents and writes ``loss`` and every parameter's ``.grad`` in place (the
    gradients are assigned, not accumulated: they are allocated by the captured backward). Warm-up steps run on a side
    stream first, as capture needs (the attention self-test and the allocator's pools settle there)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(warmup):
            train_step(model, decoder, x, z0, targets, steps, alpha)
            model.zero_grad(set_to_none=True)
            decoder.zero_grad(set_to_none=True)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        loss = train_step(model, decoder, x, z0, targets, steps, alpha)
    return graph, loss


@torch.no_grad()
def _energies(model, v, x_emb):
    return model(v, x_emb)


def infer(model, x, z0, samples: int, steps: int = 64, alpha: float = 0.1):
    """Config 4: ``x`` [N, L] inputs, ``z0`` [N * samples, L, hidden] latents; returns (best latent per input [N, L,
    hidden], its energy [N])."""
    n = x.shape[0]
    xs = x.repeat_interleave(samples, dim=0)
    with torch.no_grad():
        x_emb = model.puzzle_embedding(xs, z0.dtype)
    v = descend(model, z0, x_emb, steps, alpha, create_graph=False)
    e = _energies(model, v, x_emb).view(n, samples)
    best = e.argmin(dim=1)
    idx = torch.arange(n, device=x.device) * samples + best
    return v.detach()[idx], e.gather(1, best[:, None]).squeeze(1)


def build(cfg: EnergyConfig, device: torch.device, seed: int = 0):
    torch.manual_seed(seed)
    model = ScalarEnergy(cfg).to(device)
    decoder = Decoder(cfg).to(device)
    impl = check_linear_impl(cfg.linear_impl)
    for m in (*model.modules(), *decoder.modules()):
        if isinstance(m, CastedLinear):
            m.impl = impl
    return model, decoder


__all__ = [
    "Decoder",
    "EnergyConfig",
    "ScalarEnergy",
    "build",
    "compiled_energy_grad",
    "descend",
    "energy_grad",
    "graph_train_step",
    "infer",
    "microstep",
    "sphere",
    "train_step",
    "verify_compiled_energy_grad",
]
