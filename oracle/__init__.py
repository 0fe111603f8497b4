"""CPU oracle for the fused second-order attention path.

TEST INFRASTRUCTURE ONLY. Nothing in the shipped package (``ebr_amd``) imports this package. It may be imported by
``tests/``, by ``__graft_entry__.smoke()`` (as the checker of one small GPU call) and by ``bench.py``'s
``cpu_baseline`` leg (timed as the host-CPU eager path). It is never the implementation under measurement.

Contents:
- ``attention_ref``: dense restatement of the reference's eager attention and of its three fused ops
  (``models/fused_attn/reference.py``, ``models/attention.py:49-54``), plus the autograd recipes that pin them.
- ``rope_ref``: dense restatement of the fused 2D-RoPE split and merge and of their tables.
- ``descent_ref``: restatement of the descent wrapper's pointwise functions and their autograd VJPs.

Pinning (each function has at least one check that does not retype its formula):
- ``attn_fwd``: ``torch.softmax``/``torch.logsumexp`` closed forms and known answers (L = 1, Q = 0, row shift,
  key/value permutation) in ``tests/test_oracle.py``.
- ``attn_bwd``: the VJP of ``math_attention`` through torch autograd, fp64 ``gradcheck`` on tiny shapes, linearity in
  dO and the identity rowsum(dO*O) = rowsum(P*dP).
- ``attn_bwd_bwd``: the double backward of ``math_attention`` through torch autograd (create_graph), fp64
  ``gradgradcheck``, a central finite-difference Hessian-vector check, linearity in (gQ, gK, gV) and the
  zero-cotangent special cases.
- ``math_attention``: ``torch.nn.functional.scaled_dot_product_attention`` (fp64) and the known answers above.
- ``rope_ref`` (the fused 2D-RoPE split/merge, ``models/fused_attn/rope_split.py:32-66``): ``ref_split`` equals the
  textbook broadcast 2D RoPE (rotate_half per half) on the full tables and preserves each rotated pair's norm;
  ``ref_merge`` is its exact adjoint (<split x, y> = <x, merge y> in fp64) and equals torch autograd's VJP of it.
- ``descent_ref`` (the descent wrapper, ``models/energy.py:219-241``, ``models/layers.py:37-42``): ``rms_norm`` equals
  ``torch.nn.functional.rms_norm`` and has the closed-form RMS mean/(mean + eps); ``sphere`` equals the L2-normalised
  row times sqrt(N) (``torch.linalg.vector_norm``), is scale invariant and divides by eps under the clamp;
  ``noisy_point`` is affine in the noise with slope sigma; ``step_and_project`` keeps masked rows bit-exactly; the
  autograd VJPs equal the closed forms ``rms_norm_vjp`` / ``sphere_vjp`` and fp64 ``gradcheck``.
No function is left "parity unpinned".
"""

from oracle.attention_ref import (  # noqa: F401
    attn_bwd,
    attn_bwd_bwd,
    attn_fwd,
    autograd_bwd,
    autograd_bwd_bwd,
    default_scale,
    make_inputs,
    math_attention,
    rel_err,
)
from oracle.rope_ref import (  # noqa: F401,E402
    grid_shape,
    make_rope_inputs,
    quarter_swap,
    ref_merge,
    ref_split,
    rotary_tables,
)
from oracle.descent_ref import (  # noqa: F401,E402
    RMS_NORM_EPS,
    make_descent_inputs,
    noisy_point,
    noisy_point_replayed,
    rms_norm,
    rms_norm_vjp,
    sphere,
    sphere_vjp,
    step_and_project,
    vjp_noisy_point,
    vjp_step_and_project,
)
