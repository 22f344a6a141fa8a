"""CPU: construction-time provider dispatch of the ordinary ops (no kernel launches).

Mirrors the reference's dispatch tests (tests/test_custom_op_dispatch.py,
tests/test_custom_cuda_silu.py:53-66): providers are bound once at
construction, a GPU platform binds the gfx950 kernels, and the explicit torch
providers stay selectable by name.
"""

import json
from pathlib import Path

import pytest
import torch

from my_vllm_amd import ops
from my_vllm_amd.activation import SiluAndMul
from my_vllm_amd.attention import KVCacheStore
from my_vllm_amd.custom_op import CustomOpConfig
from oracle.reference import silu_and_mul_eager

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def test_kv_store_cpu_platform_reference_known_answer():
    # The reference's own CPU test (tests/test_custom_op_dispatch.py:75-95).
    kat = KATS["kv_store"]
    store = KVCacheStore(CustomOpConfig(platform="cpu"))
    assert store.kv_store_provider_name == "native_torch"
    key = torch.arange(kat["key"]["arange_from"], kat["key"]["arange_to"], dtype=torch.float32).reshape(
        kat["key"]["shape"])
    value = key + kat["value_offset"]
    k_cache = torch.full(kat["cache_shape"], kat["cache_fill"])
    v_cache = torch.full(kat["cache_shape"], kat["cache_fill"])
    expected_k, expected_v = k_cache.clone(), v_cache.clone()
    for row, token in kat["writes"]:
        expected_k.view(-1, 2, 4)[row] = key[token]
        expected_v.view(-1, 2, 4)[row] = value[token]
    assert store(key, value, k_cache, v_cache, torch.tensor(kat["slot_mapping"])) is None
    assert torch.equal(k_cache, expected_k) and torch.equal(v_cache, expected_v)


def test_gpu_platform_binds_the_gfx950_providers():
    config = CustomOpConfig(platform="cuda")
    assert KVCacheStore(config).kv_store_provider_name == "hip"
    silu = SiluAndMul(config)
    assert silu.provider_name == "hip" and silu.forward_impl is ops.silu_and_mul
    named = SiluAndMul(CustomOpConfig(platform="cuda", overrides={"silu_and_mul": "custom_cuda"}))
    assert named.provider_name == "custom_cuda"
    torch_named = SiluAndMul(CustomOpConfig(platform="cuda", overrides={"silu_and_mul": "native_torch"}))
    assert torch_named.provider_name == "native_torch"


def test_unknown_providers_are_rejected():
    with pytest.raises(ValueError, match="kv_cache_store"):
        KVCacheStore(CustomOpConfig(platform="cuda", overrides={"kv_cache_store": "native_triton_x"}))
    with pytest.raises(RuntimeError, match="requires CUDA"):
        KVCacheStore(CustomOpConfig(platform="cpu", overrides={"kv_cache_store": "hip"}))
    with pytest.raises(ValueError):
        CustomOpConfig(platform="tpu")


def test_config_overrides_are_frozen_and_normalised():
    config = CustomOpConfig(platform="CUDA", overrides={"silu_and_mul": "HIP"})
    assert config.platform == "cuda" and config.implementation_for("silu_and_mul") == "hip"
    assert config.implementation_for("other") == "auto"
    with pytest.raises(TypeError):
        config.overrides["silu_and_mul"] = "native"


def test_silu_cpu_platform_is_the_reference_native_path():
    x = torch.randn(5, 24, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16)
    op = SiluAndMul(CustomOpConfig(platform="cpu"))
    assert op.provider_name == "native_torch"
    out = op(x)
    assert torch.equal(out, silu_and_mul_eager(x)) and out.data_ptr() != x.data_ptr()


def test_silu_kernel_entry_rejects_host_tensors_like_the_reference():
    # tests/test_custom_cuda_silu.py:53-66: a non-GPU tensor is a RuntimeError naming CUDA.
    with pytest.raises(RuntimeError, match=KATS["silu"]["errors"]["cpu"]):
        ops.silu_and_mul(torch.zeros(4, 8, dtype=torch.bfloat16))


def test_store_entry_checks_layout_before_launch():
    key = torch.zeros(3, 2, 128, dtype=torch.bfloat16)
    cache = torch.zeros(2, 16, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="one slot per token"):
        ops.store_kvcache(key, key, cache, cache, torch.zeros(2, dtype=torch.int32))
    with pytest.raises(TypeError):
        ops.store_kvcache(key, key, cache, cache, torch.zeros(3, dtype=torch.float32))
    with pytest.raises(ValueError, match="unit stride"):
        ops.store_kvcache(key.transpose(1, 2).contiguous().transpose(1, 2), key, cache, cache,
                          torch.zeros(3, dtype=torch.int32))
    spread = torch.zeros(3, 4, 128, dtype=torch.bfloat16)[:, ::2]  # head stride 2*D
    with pytest.raises(ValueError, match="packed"):
        ops.store_kvcache(spread, spread, cache, cache, torch.zeros(3, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="CUDA"):
        ops.store_kvcache(key, key, cache, cache, torch.zeros(3, dtype=torch.int32))
