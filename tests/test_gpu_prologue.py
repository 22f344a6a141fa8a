"""Attention prologue (q/k RMSNorm + neox RoPE + KV store) and the
RotaryEmbedding provider on gfx950 vs the CPU oracle.

Bars: RoPE alone is bit-exact (same fp32 cos/sin table, separate fp32
multiplies and adds, one rounding); with q/k norms the result is within the
bound set by one ulp of the normalised intermediate (scaled by the weight and
the rotation), and almost every element is bit-exact; the cache rows are
bit-exact copies of the rotated k and of v at their slots, -1 slots untouched.
"""

import pytest
import torch

from my_vllm_amd import ops
from my_vllm_amd.custom_op import CustomOpConfig
from my_vllm_amd.layers import RMSNorm
from my_vllm_amd.layers import RotaryEmbedding
from oracle.reference import qk_norm_rope, rope, rope_cos_sin_cache

pytestmark = pytest.mark.gpu


def _packed(tokens, hq, hkv, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    qkv = (2 * torch.randn(tokens, (hq + 2 * hkv) * 128, generator=g)).to(dtype)
    pos = torch.randint(0, 4096, (tokens,), generator=g)
    return qkv, pos


def _views(qkv, hq, hkv):
    q = qkv[:, : hq * 128].view(-1, hq, 128)
    k = qkv[:, hq * 128:(hq + hkv) * 128].view(-1, hkv, 128)
    v = qkv[:, (hq + hkv) * 128:].view(-1, hkv, 128)
    return q, k, v


@pytest.mark.parametrize("tokens,hq,hkv", [(1, 16, 8), (37, 32, 8), (300, 64, 8), (5, 12, 3)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rope_alone_is_bit_exact(gpu, tokens, hq, hkv, dtype):
    qkv, pos = _packed(tokens, hq, hkv, 21, dtype)
    table = rope_cos_sin_cache(128, 4096, 1e6)
    q, k, _ = _views(qkv, hq, hkv)
    qd, kd, _ = _views(qkv.to(gpu), hq, hkv)
    got_q, got_k = ops.qk_norm_rope_store(pos.to(gpu), qd, kd, table.to(gpu))
    assert got_q.data_ptr() == qd.data_ptr()
    assert torch.equal(got_q.cpu(), rope(q, pos, table)) and torch.equal(got_k.cpu(), rope(k, pos, table))


@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32])
def test_fused_prologue_norm_rope_and_store(gpu, wdtype):
    tokens, hq, hkv = 70, 32, 8
    qkv, pos = _packed(tokens, hq, hkv, 22)
    g = torch.Generator().manual_seed(23)
    wq = (1 + 0.3 * torch.randn(128, generator=g)).to(wdtype)
    wk = (1 + 0.3 * torch.randn(128, generator=g)).to(wdtype)
    table = rope_cos_sin_cache(128, 4096, 1e6)
    q, k, v = _views(qkv, hq, hkv)
    exp_q, exp_k = qk_norm_rope(q, k, pos, table, wq, wk, 1e-6)
    pages = 20
    k_cache = torch.full((pages, 16, hkv, 128), 7.0, dtype=torch.bfloat16, device=gpu)
    v_cache = torch.full_like(k_cache, 7.0)
    slots = torch.randperm(pages * 16, generator=g)[:tokens].to(torch.int32)
    slots[::9] = -1
    qd, kd, vd = _views(qkv.to(gpu), hq, hkv)
    got_q, got_k = ops.qk_norm_rope_store(pos.to(gpu), qd, kd, table.to(gpu), wq.to(gpu), wk.to(gpu), 1e-6,
                                          vd, k_cache, v_cache, slots.to(gpu))
    bound = 2 ** -7 * 2 * float(max(wq.abs().max(), wk.abs().max())) * 2 + 2 ** -6
    for got, exp in ((got_q.cpu(), exp_q), (got_k.cpu(), exp_k)):
        diff = (got.float() - exp.float()).abs()
        assert diff.max().item() <= bound * max(1.0, exp.float().abs().max().item() / 4)
        assert (diff == 0).float().mean().item() > 0.99
    kc, vc = k_cache.cpu().view(-1, hkv, 128), v_cache.cpu().view(-1, hkv, 128)
    for t in range(tokens):
        s = int(slots[t])
        if s >= 0:
            assert torch.equal(kc[s], got_k[t].cpu()) and torch.equal(vc[s], v[t])
    untouched = torch.ones(pages * 16, dtype=torch.bool)
    untouched[slots[slots >= 0].long()] = False
    assert bool((kc[untouched] == 7.0).all()) and bool((vc[untouched] == 7.0).all())


def test_rotary_embedding_custom_op(gpu):
    rope_op = RotaryEmbedding(128, 128, 4096, 1e6, CustomOpConfig(platform="cuda", dtype=torch.bfloat16)).to(gpu)
    assert rope_op.provider_name == "hip"
    qkv, pos = _packed(9, 16, 8, 24)
    q = qkv[:, : 16 * 128].contiguous()
    k = qkv[:, 16 * 128:24 * 128].contiguous()
    got_q, got_k = rope_op(pos.to(gpu), q.to(gpu), k.to(gpu))
    assert got_q.shape == q.shape and got_k.shape == k.shape
    table = rope_cos_sin_cache(128, 4096, 1e6)
    assert torch.equal(got_q.cpu().view(9, 16, 128), rope(q.view(9, 16, 128), pos, table))
    # forward_fused with RMSNorm modules (no cache): rotated in place.
    qn = RMSNorm(128, 1e-6, CustomOpConfig(platform="cuda")).to(gpu, torch.bfloat16)
    kn = RMSNorm(128, 1e-6, CustomOpConfig(platform="cuda")).to(gpu, torch.bfloat16)
    qd, kd, _ = _views(qkv.to(gpu), 16, 8)
    out_q, _ = rope_op.forward_fused(pos.to(gpu), qd, kd, None, qn, kn, None, None, None)
    exp_q, _ = qk_norm_rope(*_views(qkv, 16, 8)[:2], pos, table, qn.weight.cpu(), kn.weight.cpu(), 1e-6)
    assert (out_q.cpu().float() - exp_q.float()).abs().max().item() <= 2 ** -5


@pytest.mark.parametrize("tokens,hq,hkv,slot_dtype", [
    (9, 12, 3, torch.int64),      # 18 rows per token: the last quad holds two
    (33, 64, 8, torch.int32),     # 80 rows: four chunks per token
    (41, 16, 8, torch.int64),
    (9000, 32, 8, torch.int32),   # 18,000 chunks: the wavefronts loop past the grid cap
])
def test_prologue_store_shapes_and_slot_types(gpu, tokens, hq, hkv, slot_dtype):
    """RoPE + store without norms: q, k and both cache rows bit-exact for
    int32 and int64 slot mappings; slots of -1 or past the cache are
    skipped and their rows left untouched."""
    qkv, pos = _packed(tokens, hq, hkv, 25)
    table = rope_cos_sin_cache(128, 4096, 1e6)
    q, k, v = _views(qkv, hq, hkv)
    g = torch.Generator().manual_seed(26)
    num_slots = ((tokens + 4 + 15) // 16) * 16
    slots = torch.randperm(num_slots, generator=g)[:tokens].to(slot_dtype)
    slots[::7] = -1
    slots[3::11] = num_slots + 5  # past the cache: skipped, as the reference's callers never send
    k_cache = torch.full((num_slots // 16, 16, hkv, 128), 7.0, dtype=torch.bfloat16, device=gpu)
    v_cache = torch.full_like(k_cache, 7.0)
    qd, kd, vd = _views(qkv.to(gpu), hq, hkv)
    got_q, got_k = ops.qk_norm_rope_store(pos.to(gpu), qd, kd, table.to(gpu), None, None, 1e-6,
                                          vd, k_cache, v_cache, slots.to(gpu))
    exp_k = rope(k, pos, table)
    assert torch.equal(got_q.cpu(), rope(q, pos, table)) and torch.equal(got_k.cpu(), exp_k)
    kc, vc = k_cache.cpu().view(-1, hkv, 128), v_cache.cpu().view(-1, hkv, 128)
    live = (slots >= 0) & (slots < num_slots)
    idx = slots[live].long()
    assert torch.equal(kc[idx], exp_k[live]) and torch.equal(vc[idx], v[live])
    untouched = torch.ones(num_slots, dtype=torch.bool)
    untouched[idx] = False
    assert bool((kc[untouched] == 7.0).all()) and bool((vc[untouched] == 7.0).all())


def test_prologue_strided_slot_mapping_and_host_slots(gpu):
    """A strided slot_mapping view stores at the slots it shows; a host
    slot_mapping is refused before any launch."""
    tokens, hq, hkv = 12, 16, 8
    qkv, pos = _packed(tokens, hq, hkv, 27)
    table = rope_cos_sin_cache(128, 4096, 1e6)
    _, k, v = _views(qkv, hq, hkv)
    wide = torch.arange(2 * tokens, dtype=torch.int32).flip(0)  # slots 2T-1, ..., 0
    slots = wide[::2]  # stride 2: 2T-1, 2T-3, ...
    k_cache = torch.zeros((2, 16, hkv, 128), dtype=torch.bfloat16, device=gpu)
    v_cache = torch.zeros_like(k_cache)
    qd, kd, vd = _views(qkv.to(gpu), hq, hkv)
    with pytest.raises(ValueError):
        ops.qk_norm_rope_store(pos.to(gpu), qd, kd, table.to(gpu), None, None, 1e-6, vd, k_cache, v_cache, slots)
    _, got_k = ops.qk_norm_rope_store(pos.to(gpu), qd, kd, table.to(gpu), None, None, 1e-6, vd, k_cache, v_cache,
                                      wide.to(gpu)[::2])
    kc, vc = k_cache.cpu().view(-1, hkv, 128), v_cache.cpu().view(-1, hkv, 128)
    idx = slots.long()
    assert torch.equal(kc[idx], rope(k, pos, table)) and torch.equal(vc[idx], v)
    assert bool((kc[idx - 1] == 0).all())  # the even slots the view skips stay untouched
