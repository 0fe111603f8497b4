"""The three attention ops, their autograd wiring and ``fused_attention`` (drop-in for reference
``models/fused_attn/ops.py``).

Ops (``torch.ops.ebr_fused.*``; functional, fresh contiguous outputs, the reference's schemas):
- ``attn_fwd(q, k, v, scale) -> (o, lse)``                                          reference ops.py:65-77
- ``attn_bwd(q, k, v, o, lse, do, scale) -> (dq, dk, dv)``                          reference ops.py:80-95
- ``attn_bwd_bwd(q, k, v, o, lse, do, dq, gq, gk, gv, scale) -> (hq, hk, hv, hdo)``  reference ops.py:98-121

Where each call runs (``route``):
- a GPU tensor runs the gfx950 kernels of ``libebr_attn.so`` on torch's current stream. If the library cannot be
  loaded the call raises ``RuntimeError``: this build never swaps in another implementation behind a GPU caller's
  back (the reference's ``auto`` mode would fall back to its dense functions, ``ops.py:34-36``);
- ``EBR_FUSED_ATTN_IMPL=reference`` runs the dense torch functions of ``dense.py`` on any device (reference
  ``loader.py:21-23``);
- a tensor off the GPU runs the dense functions (reference ``ops.py:68-70``).

Head dims the kernels do not take natively (16-bit D not a multiple of 8, fp32 D not a multiple of 4) are zero-padded
to the next such width and the outputs cut back: zero columns add nothing to any score and produce zero columns in
every output, so the result is exact (the reference pads the same way inside its kernels, ``triton_kernels.py:587-589``).
Head dims up to 256 run on the GPU; wider ones raise ``ValueError``. Above 128 the 16-bit and fp32 calls take the
streamed two-launch kernels at every N (a 16-row tile of 256-wide rows needs a whole SIMD's registers), and fp64 its
kernels with 8-row tiles.

Autograd: ``_FusedAttn`` (its backward is ``_FusedAttnBwd``) and ``_FusedAttnBwd`` (its backward is attn_bwd_bwd),
both with ``setup_context`` as ``torch.func`` requires; ``fused_attention`` stays a single dynamo node through
``allow_in_graph`` (reference ops.py:124-190).
"""

# No ``from __future__ import annotations``: custom_op schema inference needs real type objects.
from typing import Optional, Tuple, Union

import ctypes

import torch
import torch.nn.functional as F

from ebr_amd import _capi
from ebr_amd.fused_attn import dense
from ebr_amd.fused_attn.loader import hip_library, mode

Tensor = torch.Tensor

MAX_HEAD_DIM = 256

_DTYPE_CODE = {
    torch.float32: _capi.DTYPE_F32,
    torch.bfloat16: _capi.DTYPE_BF16,
    torch.float16: _capi.DTYPE_F16,
    torch.float64: _capi.DTYPE_F64,
}


def default_scale(q: Tensor, scale: Optional[float]) -> float:
    """D ** -0.5 unless given (reference models/fused_attn/reference.py:19-20)."""
    return float(q.shape[-1] ** -0.5) if scale is None else float(scale)


def lse_dtype_for(x: Tensor) -> torch.dtype:
    """lse is fp32; fp64 inputs keep fp64 (reference reference.py:14-16)."""
    return torch.float64 if x.dtype == torch.float64 else torch.float32


def route(device: Union[torch.device, str]) -> str:
    """'hip' or 'reference': which implementation the ops use for tensors on ``device`` under the current
    ``EBR_FUSED_ATTN_IMPL``. 'hip' means the kernels or an error, never a fallback."""
    if mode() == "reference" or torch.device(device).type != "cuda":
        return "reference"
    return "hip"


def implementation(device: Union[torch.device, str] = "cuda") -> str:
    """What the ops dispatch to on ``device``: 'hip' (the gfx950 kernels; the reference names its kernels 'triton'),
    'reference' (the dense functions), or 'unavailable' when a GPU call would raise because the library cannot be
    loaded (reference ops.py:23-27)."""
    if route(device) == "reference":
        return "reference"
    try:
        hip_library()
        return "hip"
    except RuntimeError:
        return "unavailable"


def _check(q: Tensor, k: Tensor, v: Tensor) -> None:
    """The q, k, v contract of reference ops.py:51-57 (one shape [B, H, N, D], one dtype, ``ValueError`` otherwise),
    plus one device."""
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError(
            f"fused attention: q, k and v must share one [B, H, N, D] shape, got {tuple(q.shape)}, "
            f"{tuple(k.shape)}, {tuple(v.shape)}"
        )
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError(f"fused attention: q, k and v must share one dtype, got {q.dtype}, {k.dtype}, {v.dtype}")
    if not (q.device == k.device == v.device):
        raise ValueError(f"fused attention: q, k and v must be on one device, got {q.device}, {k.device}, {v.device}")


def _check_like(q: Tensor, **named: Tensor) -> None:
    """o, dO and the cotangents are read as [B, H, N, D] and lse as [B, H, N] by q's sizes (the C ABI takes only
    those), so a tensor of another shape or device is refused before any launch."""
    for name, t in named.items():
        want = q.shape[:-1] if name == "lse" else q.shape
        if t.shape != want or t.device != q.device:
            raise ValueError(f"fused attention: {name} is {tuple(t.shape)} on {t.device}, expected {tuple(want)} on "
                             f"{q.device}")


def _dtype_code(t: Tensor) -> int:
    code = _DTYPE_CODE.get(t.dtype)
    if code is None:
        raise TypeError(
            f"fused attention: unsupported dtype {t.dtype} (gfx950 kernels take float32, bfloat16, float16, float64)"
        )
    return code


def kernel_head_dim(dtype: torch.dtype, d: int) -> int:
    """Width the kernels run a head dim of ``d`` at: ``d`` itself when they take it, else the next multiple of the
    16-byte row vector (8 for 16-bit types, 4 for fp32); fp64 takes any width."""
    if d < 1 or d > MAX_HEAD_DIM:
        raise ValueError(f"fused attention on the GPU takes head dims 1..{MAX_HEAD_DIM}, got {d}")
    if dtype == torch.float64:
        return d
    vec = 4 if dtype == torch.float32 else 8
    return -(-d // vec) * vec


def _pad_d(t: Tensor, width: int) -> Tensor:
    return t if t.shape[-1] == width else F.pad(t, (0, width - t.shape[-1]))


def _cut_d(t: Tensor, d: int) -> Tensor:
    return t if t.shape[-1] == d else t[..., :d].contiguous()


def _align(t: Tensor) -> int:
    """Row-start alignment the kernels need: 16 bytes, or the element (8 bytes) for the fp64 kernels."""
    return 8 if t.dtype == torch.float64 else 16


def _rows(t: Tensor) -> Tensor:
    """Keep any B/H/L strides (views of a fused qkv projection, expanded zero rows) when every row start is aligned
    and D is unit-stride; otherwise copy (reference triton_kernels.py:598-601 keeps unit-D views)."""
    es, al = t.element_size(), _align(t)
    ok = t.stride(-1) == 1 and t.data_ptr() % al == 0
    ok = ok and all(s >= 0 and (s * es) % al == 0 for s in t.stride()[:3])
    return t if ok else t.contiguous()


def _contig(t: Tensor) -> Tensor:
    return t if t.is_contiguous() and t.data_ptr() % 16 == 0 else t.contiguous()


def _stream(t: Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _scratch(op: int, q: Tensor) -> Tuple[Optional[Tensor], int]:
    if q.dtype == torch.float64:  # the fp64 kernels need none
        return None, 0
    B, H, L, D = q.shape
    nbytes = int(hip_library().ebr_attn_scratch_bytes(op, B, H, L, D))
    if nbytes <= 0:
        return None, 0
    buf = torch.empty((nbytes + 3) // 4, device=q.device, dtype=torch.float32)
    return buf, buf.data_ptr()


def _empty_out(like: Tensor, n: int):
    return tuple(torch.empty(like.shape, device=like.device, dtype=like.dtype) for _ in range(n))


# ----------------------------------------------------------------------------------------------------------------------
# The GPU path: operands prepared for the C ABI, outputs allocated here (the library allocates nothing)
# ----------------------------------------------------------------------------------------------------------------------


def _no_rows(q: Tensor) -> bool:
    """No (b, h, row) at all: every output is empty (a zero head dim with rows is refused by kernel_head_dim)."""
    return q.shape[0] * q.shape[1] * q.shape[2] == 0


def _hip_fwd(q: Tensor, k: Tensor, v: Tensor, scale: float, plan: int = 0) -> Tuple[Tensor, Tensor]:
    B, H, L, D = q.shape
    lse = torch.empty((B, H, L), device=q.device, dtype=lse_dtype_for(q))
    if _no_rows(q):
        return torch.empty_like(q, memory_format=torch.contiguous_format), lse
    lib = hip_library()
    code = _dtype_code(q)
    W = kernel_head_dim(q.dtype, D)
    q, k, v = (_rows(_pad_d(t, W)) for t in (q, k, v))
    o = torch.empty((B, H, L, W), device=q.device, dtype=q.dtype)
    args = (
        code, B, H, L, W, ctypes.c_float(scale),
        q.data_ptr(), _capi.strides3(q), k.data_ptr(), _capi.strides3(k), v.data_ptr(), _capi.strides3(v),
        o.data_ptr(), lse.data_ptr(), _stream(q),
    )  # fmt: skip
    with torch.cuda.device(q.device):
        rc = lib.ebr_attn_fwd_plan(*args, plan) if plan else lib.ebr_attn_fwd(*args)
    _capi.check(rc, "ebr_attn_fwd")
    return _cut_d(o, D), lse


def _hip_bwd(q, k, v, o, lse, do, scale, plan: int = 0) -> Tuple[Tensor, Tensor, Tensor]:
    B, H, L, D = q.shape
    if _no_rows(q):
        return _empty_out(q, 3)
    lib = hip_library()
    code = _dtype_code(q)
    W = kernel_head_dim(q.dtype, D)
    q, k, v, do = (_rows(_pad_d(t, W)) for t in (q, k, v, do))
    o, lse = _contig(_pad_d(o.to(q.dtype), W)), _contig(lse.to(lse_dtype_for(q)))
    dq, dk, dv = (torch.empty((B, H, L, W), device=q.device, dtype=q.dtype) for _ in range(3))
    scratch, sp = _scratch(_capi.OP_BWD, q)
    args = (
        code, B, H, L, W, ctypes.c_float(scale),
        q.data_ptr(), _capi.strides3(q), k.data_ptr(), _capi.strides3(k), v.data_ptr(), _capi.strides3(v),
        o.data_ptr(), lse.data_ptr(), do.data_ptr(), _capi.strides3(do),
        dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), sp, _stream(q),
    )  # fmt: skip
    with torch.cuda.device(q.device):
        rc = lib.ebr_attn_bwd_plan(*args, plan) if plan else lib.ebr_attn_bwd(*args)
    _capi.check(rc, "ebr_attn_bwd")
    del scratch  # the caching allocator keeps it valid for the work already queued on this stream
    return _cut_d(dq, D), _cut_d(dk, D), _cut_d(dv, D)


def _hip_bwd_bwd(q, k, v, o, lse, do, gq, gk, gv, scale, plan: int = 0) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    B, H, L, D = q.shape
    do_dtype = do.dtype
    if _no_rows(q):
        return (*_empty_out(q, 3), torch.empty(q.shape, device=q.device, dtype=do_dtype))
    lib = hip_library()
    code = _dtype_code(q)
    W = kernel_head_dim(q.dtype, D)
    q, k, v = (_rows(_pad_d(t, W)) for t in (q, k, v))
    do, gq, gk, gv = (_rows(_pad_d(t.to(q.dtype), W)) for t in (do, gq, gk, gv))
    o, lse = _contig(_pad_d(o.to(q.dtype), W)), _contig(lse.to(lse_dtype_for(q)))
    hq, hk, hv, hdo = (torch.empty((B, H, L, W), device=q.device, dtype=q.dtype) for _ in range(4))
    scratch, sp = _scratch(_capi.OP_BWD_BWD, q)
    args = (
        code, B, H, L, W, ctypes.c_float(scale),
        q.data_ptr(), _capi.strides3(q), k.data_ptr(), _capi.strides3(k), v.data_ptr(), _capi.strides3(v),
        o.data_ptr(), lse.data_ptr(), do.data_ptr(), _capi.strides3(do),
        gq.data_ptr(), _capi.strides3(gq), gk.data_ptr(), _capi.strides3(gk), gv.data_ptr(), _capi.strides3(gv),
        hq.data_ptr(), hk.data_ptr(), hv.data_ptr(), hdo.data_ptr(), sp, _stream(q),
    )  # fmt: skip
    with torch.cuda.device(q.device):
        rc = lib.ebr_attn_bwd_bwd_plan(*args, plan) if plan else lib.ebr_attn_bwd_bwd(*args)
    _capi.check(rc, "ebr_attn_bwd_bwd")
    del scratch
    return _cut_d(hq, D), _cut_d(hk, D), _cut_d(hv, D), _cut_d(hdo, D).to(do_dtype)


# ----------------------------------------------------------------------------------------------------------------------
# Ops
# ----------------------------------------------------------------------------------------------------------------------


@torch.library.custom_op("ebr_fused::attn_fwd", mutates_args=())
def attn_fwd(q: Tensor, k: Tensor, v: Tensor, scale: float) -> Tuple[Tensor, Tensor]:
    _check(q, k, v)
    if route(q.device) == "reference":
        return dense.attn_fwd(q, k, v, scale)
    return _hip_fwd(q, k, v, scale)


@attn_fwd.register_fake
def _(q: Tensor, k: Tensor, v: Tensor, scale: float) -> Tuple[Tensor, Tensor]:
    o = torch.empty_like(q, memory_format=torch.contiguous_format)
    lse = q.new_empty(q.shape[:-1], dtype=lse_dtype_for(q))
    return o, lse


@torch.library.custom_op("ebr_fused::attn_bwd", mutates_args=())
def attn_bwd(
    q: Tensor, k: Tensor, v: Tensor, o: Tensor, lse: Tensor, do: Tensor, scale: float
) -> Tuple[Tensor, Tensor, Tensor]:
    _check(q, k, v)
    _check_like(q, o=o, lse=lse, do=do)
    do = do.to(q.dtype)  # reference ops.py:84
    if route(q.device) == "reference":
        return dense.attn_bwd(q, k, v, o, lse, do, scale)
    return _hip_bwd(q, k, v, o, lse, do, scale)


@attn_bwd.register_fake
def _(
    q: Tensor, k: Tensor, v: Tensor, o: Tensor, lse: Tensor, do: Tensor, scale: float
) -> Tuple[Tensor, Tensor, Tensor]:
    return tuple(torch.empty_like(t, memory_format=torch.contiguous_format) for t in (q, k, v))


@torch.library.custom_op("ebr_fused::attn_bwd_bwd", mutates_args=())
def attn_bwd_bwd(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    o: Tensor,
    lse: Tensor,
    do: Tensor,
    dq: Tensor,
    gq: Tensor,
    gk: Tensor,
    gv: Tensor,
    scale: float,
) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    del dq  # in the op's signature; neither implementation reads it (reference reference.py:74)
    _check(q, k, v)
    _check_like(q, o=o, lse=lse, do=do, gq=gq, gk=gk, gv=gv)
    if route(q.device) == "reference":
        return dense.attn_bwd_bwd(q, k, v, o, lse, do, gq, gk, gv, scale)
    return _hip_bwd_bwd(q, k, v, o, lse, do, gq, gk, gv, scale)


@attn_bwd_bwd.register_fake
def _(q, k, v, o, lse, do, dq, gq, gk, gv, scale):
    return tuple(torch.empty_like(t, memory_format=torch.contiguous_format) for t in (q, k, v, do))


# ----------------------------------------------------------------------------------------------------------------------
# Autograd: fwd -> bwd -> bwd_bwd (reference ops.py:124-185)
# ----------------------------------------------------------------------------------------------------------------------


def _zero_rows(like: Tensor) -> Tensor:
    """An all-zero cotangent as one zero row expanded to [B, H, L, D] (strides 0, 0, 0, 1): no L x D memory is written.
    The reference materialises ``zeros_like`` here (ops.py:147-149); the values are identical."""
    return torch.zeros((like.shape[-1],), device=like.device, dtype=like.dtype).expand(like.shape)


class _FusedAttnBwd(torch.autograd.Function):
    """First derivative as a differentiable node: forward is attn_bwd, backward is attn_bwd_bwd."""

    @staticmethod
    def forward(q, k, v, o, lse, do, scale):
        return torch.ops.ebr_fused.attn_bwd(q, k, v, o, lse, do, scale)

    @staticmethod
    def setup_context(ctx, inputs, output):
        q, k, v, o, lse, do, scale = inputs
        ctx.save_for_backward(q, k, v, o, lse, do, output[0])
        ctx.scale = scale
        # An output nobody differentiates arrives as None and becomes an expanded zero row in backward.
        ctx.set_materialize_grads(False)

    @staticmethod
    def backward(ctx, gq, gk, gv):
        q, k, v, o, lse, do, dq = ctx.saved_tensors
        cot = [_zero_rows(ref) if g is None else g.to(ref.dtype) for g, ref in ((gq, q), (gk, k), (gv, v))]
        hq, hk, hv, hdo = torch.ops.ebr_fused.attn_bwd_bwd(q, k, v, o, lse, do, dq, *cot, ctx.scale)
        # o and lse are treated as constants: their dependence is folded into hq / hk / hv / hdo.
        return hq, hk, hv, None, None, hdo, None


class _FusedAttn(torch.autograd.Function):
    """Attention as a node returning (o, lse); lse carries no gradient, the backward is the _FusedAttnBwd node."""

    @staticmethod
    def forward(q, k, v, scale):
        return torch.ops.ebr_fused.attn_fwd(q, k, v, scale)

    @staticmethod
    def setup_context(ctx, inputs, output):
        q, k, v, scale = inputs
        o, lse = output
        ctx.mark_non_differentiable(lse)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.scale = scale

    @staticmethod
    def backward(ctx, do, _dlse):
        q, k, v, o, lse = ctx.saved_tensors
        return (*_FusedAttnBwd.apply(q, k, v, o, lse, do, ctx.scale), None)


def _fused_attention_apply(q: Tensor, k: Tensor, v: Tensor, scale: float) -> Tensor:
    return _FusedAttn.apply(q, k, v, scale)[0]


# dynamo sees one opaque call; AOTAutograd then traces the two Functions, so compiled graphs hold the three ops.
_fused_attention_apply = torch._dynamo.allow_in_graph(_fused_attention_apply)


def fused_attention(q: Tensor, k: Tensor, v: Tensor, scale: Optional[float] = None) -> Tensor:
    """Non-causal softmax attention on [B, H, N, D], differentiable to second order."""
    return _fused_attention_apply(q, k, v, default_scale(q, scale))


__all__ = [
    "attn_bwd",
    "attn_bwd_bwd",
    "attn_fwd",
    "default_scale",
    "fused_attention",
    "implementation",
    "kernel_head_dim",
    "route",
]
