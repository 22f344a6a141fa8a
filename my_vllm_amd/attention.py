"""Attention layer and slot_mapping KV-cache store (mirror of the reference).

``KVCacheStore`` restates nanovllm/layers/attention.py:44-101 with the gfx950
scatter kernel as the GPU provider; ``Attention`` restates :104-143 (store
first, then the backend, on the current stream).  The store stays a separate
launch ahead of attention: sequences of one batch may read pages another
sequence writes in the same step, so every write must land before any read.
"""

from __future__ import annotations

import torch
from torch import nn

from . import _native, ops
from .attention_backend import AttentionBackend
from .context import get_context
from .custom_op import CustomOp, CustomOpConfig


class KVCacheStore(CustomOp):
    """Write K/V tensors into the NHD paged cache."""

    op_name = "kv_cache_store"
    _IMPLEMENTATIONS = frozenset({"auto", "native", "native_torch", "hip"})

    def __init__(self, custom_op_config: CustomOpConfig | None = None) -> None:
        super().__init__(custom_op_config)
        implementation = self.requested_implementation
        if implementation not in self._IMPLEMENTATIONS:
            available = ", ".join(sorted(self._IMPLEMENTATIONS))
            raise ValueError(
                "unsupported 'kv_cache_store' implementation "
                f"{implementation!r}; available: {available}"
            )
        if self.platform == "cuda" and implementation in ("auto", "hip"):
            _native.load_library()  # raises if the gfx950 library is missing
            self.kv_store_provider_name = "hip"
            self.forward_impl = ops.store_kvcache
        elif implementation == "hip":
            raise RuntimeError("'hip' for 'kv_cache_store' requires CUDA")
        else:
            self.kv_store_provider_name = "native_torch"
            self.forward_impl = self.forward_native

    def forward_native(self, key, value, k_cache, v_cache, slot_mapping) -> None:
        if slot_mapping.numel() != key.shape[0]:
            raise ValueError("slot_mapping must contain one slot per token")
        valid = slot_mapping >= 0
        num_heads, head_dim = key.shape[-2:]
        flat_k = k_cache.view(-1, num_heads, head_dim)
        flat_v = v_cache.view(-1, num_heads, head_dim)
        slots = slot_mapping[valid].to(dtype=torch.long)
        flat_k.index_copy_(0, slots, key[valid])
        flat_v.index_copy_(0, slots, value[valid])

    def forward_cuda(self, key, value, k_cache, v_cache, slot_mapping) -> None:
        self.forward_impl(key, value, k_cache, v_cache, slot_mapping)


class Attention(nn.Module):
    def __init__(
        self,
        num_heads,
        head_dim,
        scale,
        num_kv_heads,
        attention_backend: AttentionBackend | None = None,
        custom_op_config: CustomOpConfig | None = None,
    ):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.k_cache = self.v_cache = torch.tensor([])
        if attention_backend is None:
            raise ValueError("Attention requires a selected AttentionBackend instance")
        self.backend = attention_backend
        self.kv_store = KVCacheStore(custom_op_config=custom_op_config)
        self.kv_store_provider_name = self.kv_store.kv_store_provider_name

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
        context = get_context()
        metadata = context.attention_metadata
        plan = context.attention_plan
        if metadata is None or plan is None:
            raise RuntimeError("attention metadata and plan must be prepared before forward")
        k_cache, v_cache = self.k_cache, self.v_cache
        if k_cache.numel() and v_cache.numel():
            fused = getattr(self.backend, "forward_with_kv_store", None)
            if fused is not None:
                # The MI355X backend folds the store into a piece-list decode
                # launch and otherwise runs self.kv_store first.
                return fused(q, k, v, k_cache, v_cache, metadata.slot_mapping, plan, self.kv_store)
            self.kv_store(k, v, k_cache, v_cache, metadata.slot_mapping)
        return self.backend.forward(q, k, v, k_cache, v_cache, plan)
