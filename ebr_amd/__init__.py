"""ebr_amd: MI355X (gfx950) fused second-order attention for Energy-Based Reasoners.

- ``ebr_amd.fused_attn``: ``fused_attention`` and the ``ebr_fused::attn_fwd/attn_bwd/attn_bwd_bwd`` ops, backed by the
  hand-written HIP kernels of ``libebr_attn.so``.
- ``ebr_amd.attention``: the caller side (backend registry, second-order tier flag and self-test, EnergyAttention).
- ``ebr_amd.layers`` / ``ebr_amd.energy``: the energy network and descent step used as the end-to-end harness.
"""

__version__ = "0.1.0"
