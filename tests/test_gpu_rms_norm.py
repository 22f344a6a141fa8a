"""RMSNorm / fused residual-add RMSNorm on gfx950 vs the CPU oracle.

Bar, against the oracle's restatement of nanovllm/layers/layernorm.py:31-52
(fp32 statistics; the scaled row a = T(x * rsqrt(mean(x^2) + eps)) is rounded
before the weight multiply, y = T(a * w)): every output equals T(a' * w) for
an a' within 1 ulp of the oracle's a (a different fp32 summation order may
move a across a rounding boundary; the weight multiply then scales that one
ulp), and with unit weights the output is within 1 ulp.  The returned
residual is bit-exact.  Covers the
vector path (hidden a multiple of 8, up to 8192), the scalar path (other
widths, wider rows, unaligned rows), fp32 and storage-type weights, strided
rows, in-place calls, empty inputs and the CustomOp provider contract.
"""

import pytest
import torch

from my_vllm_amd import ops
from my_vllm_amd.custom_op import CustomOpConfig
from my_vllm_amd.layers import RMSNorm
from oracle.reference import fused_add_rms_norm, rms_norm, rms_scaled
from tests._util import max_ulp_diff


def assert_rms_matches(got, x32, w, eps):
    """got == T(a' * w) elementwise for some a' within 1 ulp of the oracle's a."""
    dtype = got.dtype
    a = rms_scaled(x32, eps, dtype)
    bits = a.view(torch.int16)
    ok = torch.zeros(a.shape, dtype=torch.bool)
    got = got.cpu()
    for delta in (0, 1, -1):
        cand = (bits + delta).view(dtype) if delta else a
        y = (cand.float() * w.float()).to(dtype)
        ok |= (y.view(torch.int16) == got.view(torch.int16)) | (y.isnan() & got.isnan())
    assert bool(ok.all()), f"{int((~ok).sum())} elements outside T(a' w), |a' - a| <= 1 ulp"

pytestmark = pytest.mark.gpu

SHAPES = [(4096, 1024), (7, 2560), (3, 5120), (2, 8192), (5, 8200), (9, 100), (1, 8), (33, 4096)]


def _inputs(shape, dtype, wdtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = (3 * torch.randn(*shape, generator=g)).to(dtype)
    r = torch.randn(*shape, generator=g).to(dtype)
    w = (1 + 0.5 * torch.randn(shape[-1], generator=g)).to(wdtype)
    return x, r, w


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dtype,wdtype", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
                                          (torch.bfloat16, torch.float32)])
def test_rms_norm_within_one_ulp(gpu, shape, dtype, wdtype):
    x, r, w = _inputs(shape, dtype, wdtype, 11)
    got = ops.rms_norm(x.to(gpu), w.to(gpu), 1e-6)
    assert_rms_matches(got, x.float(), w, 1e-6)
    out, res = ops.fused_add_rms_norm(x.to(gpu), r.to(gpu), w.to(gpu), 1e-6)
    _, exp_res = fused_add_rms_norm(x, r, w, 1e-6)
    assert torch.equal(res.cpu(), exp_res)
    assert_rms_matches(out, x.float() + r.float(), w, 1e-6)
    ones = torch.ones(shape[-1], dtype=wdtype)
    assert max_ulp_diff(ops.rms_norm(x.to(gpu), ones.to(gpu), 1e-6), rms_norm(x, ones, 1e-6)) <= 1
    out1, _ = ops.fused_add_rms_norm(x.to(gpu), r.to(gpu), ones.to(gpu), 1e-6)
    assert max_ulp_diff(out1, fused_add_rms_norm(x, r, ones, 1e-6)[0]) <= 1


def test_in_place_and_strided_rows(gpu):
    x, r, w = _inputs((64, 2048), torch.bfloat16, torch.bfloat16, 12)
    _, exp_res = fused_add_rms_norm(x, r, w, 1e-5)
    xd, rd = x.to(gpu), r.to(gpu)
    out, res = ops.fused_add_rms_norm(xd, rd, w.to(gpu), 1e-5, inplace=True)
    assert out.data_ptr() == xd.data_ptr() and res.data_ptr() == rd.data_ptr()
    assert torch.equal(res.cpu(), exp_res)
    assert_rms_matches(out, x.float() + r.float(), w, 1e-5)
    # Rows with a stride of 2 * hidden (the first half of a wider projection).
    wide = torch.randn(32, 2, 1024, generator=torch.Generator().manual_seed(13)).bfloat16()
    view = wide[:, 0, :]
    w1 = torch.ones(1024).bfloat16()
    got = ops.rms_norm(wide.to(gpu)[:, 0, :], w1.to(gpu), 1e-6)
    assert max_ulp_diff(got, rms_norm(view, w1, 1e-6)) <= 1
    # 3-D input and an empty batch.
    x3 = torch.randn(2, 3, 128, generator=torch.Generator().manual_seed(14)).bfloat16()
    w3 = torch.randn(128, generator=torch.Generator().manual_seed(15)).bfloat16()
    assert_rms_matches(ops.rms_norm(x3.to(gpu), w3.to(gpu), 1e-6), x3.float(), w3, 1e-6)
    assert ops.rms_norm(torch.empty(0, 64, dtype=torch.bfloat16, device=gpu), w3[:64].to(gpu), 1e-6).shape == (0, 64)


def test_constant_rows_return_the_weight_bit_exactly(gpu):
    w = torch.randn(512, generator=torch.Generator().manual_seed(16)).bfloat16()
    x = torch.cat([torch.full((4, 512), 2.0), torch.full((4, 512), -0.5)]).bfloat16()
    got = ops.rms_norm(x.to(gpu), w.to(gpu), 1e-6).cpu()
    assert torch.equal(got[:4], w.expand(4, -1)) and torch.equal(got[4:], (-w).expand(4, -1))


def test_custom_op_providers(gpu):
    norm = RMSNorm(1024, 1e-6, CustomOpConfig(platform="cuda", dtype=torch.bfloat16)).to(gpu, torch.bfloat16)
    assert norm.rms_provider_name == "hip" and norm.add_rms_provider_name == "hip"
    x, r, w = _inputs((16, 1024), torch.bfloat16, torch.bfloat16, 17)
    with torch.no_grad():
        norm.weight.copy_(w)
    assert_rms_matches(norm(x.to(gpu)), x.float(), w, 1e-6)
    out, res = norm(x.to(gpu), r.to(gpu))
    _, exp_res = fused_add_rms_norm(x, r, w, 1e-6)
    assert torch.equal(res.cpu(), exp_res)
    assert_rms_matches(out, x.float() + r.float(), w, 1e-6)
    alias = RMSNorm(1024, 1e-6, CustomOpConfig(platform="cuda", overrides={"rms_norm": "flashinfer"}))
    assert alias.rms_provider_name == "hip"
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        ops.rms_norm(x, w.to(gpu), 1e-6)


def test_rms_norm_of_head_views_of_a_packed_projection(gpu):
    # The reference applies q_norm / k_norm to [tokens, heads, head_dim] views
    # of the packed qkv projection (token stride != heads * head_dim).
    tokens, hq, hkv = 19, 32, 8
    qkv = torch.randn(tokens, (hq + 2 * hkv) * 128, generator=torch.Generator().manual_seed(18)).bfloat16()
    w = (1 + 0.2 * torch.randn(128, generator=torch.Generator().manual_seed(19))).bfloat16()
    q = qkv[:, : hq * 128].view(tokens, hq, 128)
    k = qkv[:, hq * 128:(hq + hkv) * 128].view(tokens, hkv, 128)
    qd = qkv.to(gpu)[:, : hq * 128].view(tokens, hq, 128)
    kd = qkv.to(gpu)[:, hq * 128:(hq + hkv) * 128].view(tokens, hkv, 128)
    assert_rms_matches(ops.rms_norm(qd, w.to(gpu), 1e-6), q.float(), w, 1e-6)
    assert_rms_matches(ops.rms_norm(kd, w.to(gpu), 1e-6), k.float(), w, 1e-6)
    norm = RMSNorm(128, 1e-6, CustomOpConfig(platform="cuda", dtype=torch.bfloat16)).to(gpu, torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_(w)
    assert_rms_matches(norm(qd), q.float(), w, 1e-6)
