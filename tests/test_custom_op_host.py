"""CPU: construction-time provider selection of the drop-in operators (no launches).

The dispatch base follows the reference's contract (tests/test_custom_op_dispatch.py):
``forward`` is bound once at construction, CPU falls back to ``forward_native``,
unknown provider names are ValueErrors, GPU-only names off CUDA are
RuntimeErrors, and the override map is normalised and frozen.  The operators
answer to the reference's own provider names (``example_optimized.py:10-16``)
with the gfx950 kernels and refuse, loudly, what they cannot serve.
"""

import json
from pathlib import Path

import pytest
import torch

from my_vllm_amd import ops, providers
from my_vllm_amd.custom_op import CustomOp, CustomOpConfig
from my_vllm_amd.layers import KVCacheStore, RMSNorm, RotaryEmbedding, SiluAndMul

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())

# The reference's "fully optimized" override map (example_optimized.py:10-16).
REFERENCE_OPTIMIZED_OVERRIDES = {
    "silu_and_mul": "adaptive_cuda",
    "rms_norm": "flashinfer",
    "fused_add_rms_norm": "flashinfer",
    "rotary_embedding": "flashinfer",
    "kv_cache_store": "native_triton",
}


def _build_all(config):
    return (SiluAndMul(config), KVCacheStore(config), RMSNorm(64, custom_op_config=config),
            RotaryEmbedding(128, 128, 64, 1e6, custom_op_config=config))


class _Counting(CustomOp):
    op_name = "counting"

    def __init__(self, config):
        self.dispatches = 0
        self.native_calls = 0
        super().__init__(config)

    def dispatch_forward(self):
        self.dispatches += 1
        return super().dispatch_forward()

    def forward_native(self, value):
        self.native_calls += 1
        return value + 1


def test_dispatch_is_bound_once_and_cpu_falls_back_to_native():
    op = _Counting(CustomOpConfig(platform="cpu"))
    assert [op(v) for v in range(3)] == [1, 2, 3]
    assert op.dispatches == 1 and op.native_calls == 3 and op.platform == "cpu"


def test_config_overrides_are_frozen_and_normalised():
    overrides = {"silu_and_mul": "HIP"}
    config = CustomOpConfig(platform="CUDA", overrides=overrides)
    overrides["silu_and_mul"] = "native"  # the config keeps its own copy
    assert config.platform == "cuda" and config.implementation_for("silu_and_mul") == "hip"
    assert config.implementation_for("other") == "auto"
    with pytest.raises(TypeError):
        config.overrides["silu_and_mul"] = "native"
    assert hash(config) == hash(CustomOpConfig(platform="cuda", overrides={"silu_and_mul": "hip"}))
    with pytest.raises(ValueError):
        CustomOpConfig(platform="tpu")


def test_reference_optimized_override_map_binds_every_operator_to_the_kernels():
    ops_built = _build_all(CustomOpConfig(platform="cuda", overrides=REFERENCE_OPTIMIZED_OVERRIDES))
    silu, store, norm, rope = ops_built
    assert silu.provider_name == store.kv_store_provider_name == "hip"
    assert norm.rms_provider_name == norm.add_rms_provider_name == rope.provider_name == "hip"
    assert all(op._forward_method == op.forward_cuda for op in ops_built)


@pytest.mark.parametrize("op_name", providers.operator_names())
def test_every_reference_gpu_name_and_auto_select_the_kernel(op_name):
    spec = providers.provider(op_name)
    builders = {"silu_and_mul": SiluAndMul, "kv_cache_store": KVCacheStore,
                "rms_norm": lambda c: RMSNorm(64, custom_op_config=c),
                "fused_add_rms_norm": lambda c: RMSNorm(64, custom_op_config=c),
                "rotary_embedding": lambda c: RotaryEmbedding(128, 128, 64, 1e6, custom_op_config=c)}
    for name in sorted(spec.aliases | {"auto", "hip"}):
        op = builders[op_name](CustomOpConfig(platform="cuda", overrides={op_name: name}))
        bound = {"kv_cache_store": "kv_store_provider_name", "rms_norm": "rms_provider_name",
                 "fused_add_rms_norm": "add_rms_provider_name"}.get(op_name, "provider_name")
        assert getattr(op, bound) == "hip", (op_name, name)


def test_unknown_provider_names_are_value_errors():
    with pytest.raises(ValueError, match="does_not_exist"):
        SiluAndMul(CustomOpConfig(platform="cpu", overrides={"silu_and_mul": "does_not_exist"}))
    with pytest.raises(ValueError, match="kv_cache_store"):
        KVCacheStore(CustomOpConfig(platform="cuda", overrides={"kv_cache_store": "native_triton_x"}))


def test_gpu_names_off_cuda_and_torch_names_are_refused_loudly():
    with pytest.raises(RuntimeError, match="requires CUDA"):
        SiluAndMul(CustomOpConfig(platform="cpu", overrides={"silu_and_mul": "flashinfer"}))
    with pytest.raises(RuntimeError, match="requires CUDA"):
        KVCacheStore(CustomOpConfig(platform="cpu"))  # "auto" off a GPU: no CPU fallback
    for name in ("native", "native_torch"):
        with pytest.raises(RuntimeError, match="torch implementation"):
            SiluAndMul(CustomOpConfig(platform="cuda", overrides={"silu_and_mul": name}))
    with pytest.raises(RuntimeError, match="does not support dtype"):
        SiluAndMul(CustomOpConfig(platform="cuda", dtype=torch.float32))


def test_missing_library_fails_at_construction(monkeypatch, tmp_path):
    from my_vllm_amd import _native

    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setattr(_native, "LIB_PATH", tmp_path / "absent.so")
    with pytest.raises(RuntimeError, match="missing"):
        SiluAndMul(CustomOpConfig(platform="cuda"))


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


def test_rope_table_follows_the_reference_fp32_steps():
    # The table the rotary kernel reads: cos | sin of position * base^(-2i/d),
    # with the inverse frequencies and the products rounded to fp32 first.
    from oracle.reference import rope_cos_sin_cache

    from my_vllm_amd.layers import rope_table

    table = rope_table(128, 300, 1e6)
    assert table.shape == (300, 1, 128) and table.dtype == torch.float32
    assert torch.equal(table, rope_cos_sin_cache(128, 300, 1e6))
