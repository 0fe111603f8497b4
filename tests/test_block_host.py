"""Host-side checks of the fused energy block (``ebr_amd.block``), no GPU: the ops' fake implementations give the
shapes and dtypes the kernels write, argument errors are raised before any kernel runs, and the harness accepts only
the two block implementations. Numerical parity of the kernels is in ``tests/test_gpu_block.py``."""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from ebr_amd import block, layers
from ebr_amd import energy as en


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float64])
def test_block_fakes_match_contract(dtype):
    with FakeTensorMode():
        x = torch.empty(3, 81, 512, dtype=dtype)
        y = torch.ops.ebr_fused.block_rmsnorm(x, 1e-5)
        assert y.shape == x.shape and y.dtype == dtype and y.is_contiguous()
        dx = torch.ops.ebr_fused.block_rmsnorm_bwd(x, x, 1e-5)
        assert dx.shape == x.shape and dx.dtype == dtype
        gx, gdy = torch.ops.ebr_fused.block_rmsnorm_bwd2(x, x, x, 1e-5)
        assert gx.shape == gdy.shape == x.shape
        gu = torch.empty(3, 81, 2 * 1536, dtype=dtype)
        a = torch.ops.ebr_fused.block_swiglu(gu)
        assert a.shape == (3, 81, 1536) and a.dtype == dtype
        dgu = torch.ops.ebr_fused.block_swiglu_bwd(gu, a)
        assert dgu.shape == gu.shape
        ggu, gdy = torch.ops.ebr_fused.block_swiglu_bwd2(gu, a, gu)
        assert ggu.shape == gu.shape and gdy.shape == a.shape


def test_block_argument_errors():
    with pytest.raises(ValueError, match="even last dim"):
        block.swiglu(torch.zeros(2, 3))
    with pytest.raises(TypeError):
        block._code(torch.zeros(2, dtype=torch.int32))
    with pytest.raises(ValueError):
        layers.SwiGLU(hidden_size=64, expansion=4.0, impl="triton")
    cfg = en.EnergyConfig()
    assert cfg.block_impl == "eager"  # the reference's formulas unless asked


def test_block_ops_have_no_host_kernel():
    """No silent host fallback: the ops are registered for the HIP device only, so CPU tensors raise."""
    x = torch.zeros(2, 4)
    with pytest.raises(NotImplementedError):
        torch.ops.ebr_fused.block_rmsnorm(x, 1e-5)
    with pytest.raises(NotImplementedError):
        torch.ops.ebr_fused.block_swiglu(x)
