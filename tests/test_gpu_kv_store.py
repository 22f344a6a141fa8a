"""slot_mapping KV store on gfx950: bit-exact against the oracle scatter."""

import numpy as np
import pytest
import torch

from my_vllm_amd import ops
from my_vllm_amd.layers import KVCacheStore
from my_vllm_amd.custom_op import CustomOpConfig
from oracle.reference import kv_store

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.cpu().contiguous().view(torch.int16).numpy()


def test_reference_known_answer(gpu):
    # tests/test_custom_op_dispatch.py:75-95 of the reference, on the GPU path.
    key = torch.arange(1, 25, dtype=torch.float32).reshape(3, 2, 4).bfloat16()
    value = key + 100
    k_cache = torch.full((2, 2, 2, 4), -1.0).bfloat16()
    v_cache = torch.full((2, 2, 2, 4), -1.0).bfloat16()
    slots = torch.tensor([3, -1, 0], dtype=torch.int64)
    kd, vd = k_cache.to(gpu), v_cache.to(gpu)
    ops.store_kvcache(key.to(gpu), value.to(gpu), kd, vd, slots.to(gpu))
    expected_k = k_cache.clone()
    expected_v = v_cache.clone()
    expected_k.view(-1, 2, 4)[3] = key[0]
    expected_v.view(-1, 2, 4)[3] = value[0]
    expected_k.view(-1, 2, 4)[0] = key[2]
    expected_v.view(-1, 2, 4)[0] = value[2]
    assert torch.equal(kd.cpu(), expected_k) and torch.equal(vd.cpu(), expected_v)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("slot_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("num_kv_heads,num_q_heads", [(8, 16), (8, 32), (1, 8), (3, 6)])
def test_store_from_packed_qkv_is_bit_exact(gpu, dtype, slot_dtype, num_kv_heads, num_q_heads):
    rng = np.random.default_rng(5)
    head_dim, page, pages, tokens = 128, 16, 37, 203
    gen = torch.Generator().manual_seed(11)
    qkv = torch.randn(tokens, (num_q_heads + 2 * num_kv_heads) * head_dim, generator=gen).to(dtype)
    split = [num_q_heads * head_dim, num_kv_heads * head_dim, num_kv_heads * head_dim]
    _, k, v = qkv.split(split, dim=-1)
    k = k.view(tokens, num_kv_heads, head_dim)
    v = v.view(tokens, num_kv_heads, head_dim)
    slots = rng.permutation(pages * page)[:tokens].astype(np.int64)
    slots[rng.random(tokens) < 0.2] = -1
    k_cache = torch.randn(pages, page, num_kv_heads, head_dim, generator=gen).to(dtype)
    v_cache = torch.randn(pages, page, num_kv_heads, head_dim, generator=gen).to(dtype)
    exp_k, exp_v = _bits(k_cache).copy(), _bits(v_cache).copy()
    kv_store(_bits(k), _bits(v), exp_k, exp_v, slots)

    qkv_d = qkv.to(gpu)
    _, kd, vd = qkv_d.split(split, dim=-1)
    kd = kd.view(tokens, num_kv_heads, head_dim)
    vd = vd.view(tokens, num_kv_heads, head_dim)
    assert kd.stride(0) == (num_q_heads + 2 * num_kv_heads) * head_dim
    kcd, vcd = k_cache.to(gpu), v_cache.to(gpu)
    ops.store_kvcache(kd, vd, kcd, vcd, torch.from_numpy(slots).to(slot_dtype).to(gpu))
    assert np.array_equal(_bits(kcd), exp_k)
    assert np.array_equal(_bits(vcd), exp_v)


def test_out_of_range_slots_are_skipped_and_empty_batch_is_noop(gpu):
    k = torch.ones(3, 2, 128, dtype=torch.bfloat16, device=gpu)
    cache = torch.zeros(1, 16, 2, 128, dtype=torch.bfloat16, device=gpu)
    vcache = torch.zeros_like(cache)
    ops.store_kvcache(k, k, cache, vcache, torch.tensor([16, -5, 2], dtype=torch.int32, device=gpu))
    flat = cache.view(-1, 2, 128).cpu()
    assert flat[2].eq(1).all() and flat.sum().item() == 256
    ops.store_kvcache(k[:0], k[:0], cache, vcache, torch.empty(0, dtype=torch.int32, device=gpu))


def test_custom_op_binds_gfx950_store(gpu):
    store = KVCacheStore(CustomOpConfig(platform="cuda"))
    assert store.kv_store_provider_name == "hip"
    k = torch.randn(4, 2, 128, device=gpu).bfloat16()
    kc = torch.zeros(2, 16, 2, 128, dtype=torch.bfloat16, device=gpu)
    vc = torch.zeros_like(kc)
    assert store(k, k, kc, vc, torch.tensor([0, 1, 17, -1], dtype=torch.int32, device=gpu)) is None
    assert torch.equal(kc.view(-1, 2, 128)[17], k[2])
