"""SiLU-and-mul gfx950 kernel vs the oracle: within 1 bf16/fp16 ulp."""

import pytest
import torch

from my_vllm_amd import ops
from my_vllm_amd.layers import SiluAndMul
from my_vllm_amd.custom_op import CustomOpConfig
from workloads import silu_input
from oracle.reference import silu_and_mul_eager, silu_and_mul_fused
from tests._util import max_ulp_diff

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", [(18,), (31, 64), (2, 3, 14), (0, 16), (5, 24), (7, 6150), (3, 2, 4096)])
def test_silu_and_mul_matches_oracle(gpu, dtype, shape):
    gen = torch.Generator().manual_seed(23)
    x = torch.randn(shape, generator=gen).to(dtype)
    xd = x.to(gpu)
    original = xd.clone()
    out = ops.silu_and_mul(xd)
    assert out.shape == (*shape[:-1], shape[-1] // 2)
    assert out.dtype == dtype and out.is_contiguous() and out.device == xd.device
    assert torch.equal(xd, original)
    if out.numel():
        assert out.data_ptr() != xd.data_ptr()
    assert max_ulp_diff(out, silu_and_mul_fused(x)) <= 1
    assert max_ulp_diff(out, silu_and_mul_eager(x)) <= 1


def test_silu_and_mul_qwen3_mlp_shape(gpu):
    x = silu_input(4096, 6144, seed=0)
    out = ops.silu_and_mul(x.to(gpu)).cpu()
    assert max_ulp_diff(out, silu_and_mul_fused(x)) <= 1
    assert max_ulp_diff(out, silu_and_mul_eager(x)) <= 1


def test_silu_unaligned_input_takes_scalar_path(gpu):
    x = torch.randn(9, 34, generator=torch.Generator().manual_seed(3)).bfloat16()
    base = torch.empty(x.numel() + 1, dtype=torch.bfloat16, device=gpu)
    xd = base[1:].view(9, 34)
    xd.copy_(x.to(gpu))
    out = ops.silu_and_mul(xd)
    assert max_ulp_diff(out, silu_and_mul_fused(x)) <= 1


@pytest.mark.parametrize(
    ("make", "pattern"),
    [
        (lambda d: torch.randn(4, 7, device=d, dtype=torch.float16), "even"),
        (lambda d: torch.randn(4, 8, device=d, dtype=torch.float32), "supports"),
        (lambda d: torch.randn(4, 8, device=d, dtype=torch.float16).t(), "contiguous"),
    ],
)
def test_silu_rejects_unsupported_inputs(gpu, make, pattern):
    with pytest.raises(RuntimeError, match=pattern):
        ops.silu_and_mul(make(gpu))


@pytest.mark.parametrize("override", ["auto", "hip", "custom_cuda", "adaptive_cuda", "flashinfer"])
def test_custom_op_selects_gfx950_kernel(gpu, override):
    # The reference's provider names all select the gfx950 kernel.
    layer = SiluAndMul(CustomOpConfig(platform="cuda", dtype=torch.bfloat16, overrides={"silu_and_mul": override}))
    assert layer.provider_name == "hip"
    x = torch.randn(5, 192, generator=torch.Generator().manual_seed(29)).bfloat16()
    out = layer(x.to(gpu))
    assert max_ulp_diff(out, silu_and_mul_fused(x)) <= 1
