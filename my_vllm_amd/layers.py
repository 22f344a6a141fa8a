"""Drop-in operator classes with the reference's constructors and attributes,
bound to this package's gfx950 kernels through ``providers.resolve``.

* ``SiluAndMul`` (nanovllm/layers/activation.py:7-84): ``x[..., :I]``, gated,
  times ``x[..., I:]``; attribute ``provider_name``.
* ``KVCacheStore`` (nanovllm/layers/attention.py:44-101): slot_mapping scatter
  of K/V rows into the paged cache; attribute ``kv_store_provider_name``.
* ``RMSNorm`` (nanovllm/layers/layernorm.py:7-154): ``forward(x)``,
  ``forward(x, residual)`` and ``forward_inplace(x, residual)``; attributes
  ``rms_provider_name`` and ``add_rms_provider_name``.
* ``RotaryEmbedding`` (nanovllm/layers/rotary_embedding.py:18-110): neox RoPE
  over the whole head from the ``cos_sin_cache`` buffer; attribute
  ``provider_name``.  ``forward_fused`` adds the per-head q/k RMSNorm and the
  KV store to the same launch.

Each class implements ``forward_cuda`` only: the provider check at
construction has already refused every other platform.
"""

from __future__ import annotations

import torch
from torch import nn

from . import ops, providers
from .custom_op import CustomOp, CustomOpConfig


class SiluAndMul(CustomOp):
    """SwiGLU activation with construction-time platform dispatch."""

    op_name = "silu_and_mul"

    def __init__(self, custom_op_config: CustomOpConfig | None = None) -> None:
        super().__init__(custom_op_config)
        self.provider_name = providers.resolve(self)

    def forward_cuda(self, x: torch.Tensor) -> torch.Tensor:
        return ops.silu_and_mul(x)


class KVCacheStore(CustomOp):
    """Write K/V tensors into the NHD paged cache."""

    op_name = "kv_cache_store"

    def __init__(self, custom_op_config: CustomOpConfig | None = None) -> None:
        super().__init__(custom_op_config)
        self.kv_store_provider_name = providers.resolve(self)

    def forward_cuda(self, key, value, k_cache, v_cache, slot_mapping) -> None:
        ops.store_kvcache(key, value, k_cache, v_cache, slot_mapping)


class RMSNorm(CustomOp):
    """RMSNorm and fused residual-add RMSNorm ordinary operator."""

    op_name = "rms_norm"

    def __init__(self, hidden_size: int, eps: float = 1e-6, custom_op_config: CustomOpConfig | None = None) -> None:
        super().__init__(custom_op_config)
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.rms_provider_name = providers.resolve(self, "rms_norm")
        self.add_rms_provider_name = providers.resolve(self, "fused_add_rms_norm")

    def forward_cuda(self, x: torch.Tensor, residual: torch.Tensor | None = None):
        if residual is None:
            return ops.rms_norm(x, self.weight, self.eps)
        return ops.fused_add_rms_norm(x, residual, self.weight, self.eps)

    def forward_inplace(self, x: torch.Tensor, residual: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """``forward(x, residual)`` written into ``x`` and ``residual`` (both dead after the call)."""
        return ops.fused_add_rms_norm(x, residual, self.weight, self.eps, inplace=True)


def rope_table(rotary_dim: int, max_position: int, base: float) -> torch.Tensor:
    """The fp32 ``[max_position, 1, rotary_dim]`` table ``cos | sin`` of the
    neox rotation angles ``position * base^(-2i / rotary_dim)``.  The kernel
    reads this exact table, so its values follow the reference's fp32 steps
    (rotary_embedding.py:28-35): inverse frequencies, then one product per
    (position, frequency), then cos and sin."""
    inv_freq = 1.0 / torch.pow(base, torch.arange(0, rotary_dim, 2, dtype=torch.float32) / rotary_dim)
    angles = torch.outer(torch.arange(max_position, dtype=torch.float32), inv_freq)
    return torch.cat((angles.cos(), angles.sin()), dim=-1).unsqueeze(1)


class RotaryEmbedding(CustomOp):
    """Neox rotary embedding over the full head dimension."""

    op_name = "rotary_embedding"

    def __init__(self, head_size: int, rotary_dim: int, max_position_embeddings: int, base: float,
                 custom_op_config: CustomOpConfig | None = None) -> None:
        super().__init__(custom_op_config)
        if rotary_dim != head_size:
            raise ValueError("rotary_dim must equal head_size (the rotation covers the whole head)")
        if head_size != ops.HEAD_DIM:
            raise ValueError(f"the gfx950 rotary kernel supports head_size {ops.HEAD_DIM}")
        self.head_size = head_size
        self.register_buffer("cos_sin_cache", rope_table(rotary_dim, max_position_embeddings, base),
                             persistent=False)
        self.provider_name = providers.resolve(self)

    def forward_cuda(self, positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor):
        return ops.rotary_embedding(positions, query, key, self.cos_sin_cache, self.head_size)

    def forward_fused(self, positions, q, k, v, q_norm, k_norm, k_cache, v_cache, slot_mapping):
        """q_norm / k_norm (``RMSNorm`` modules over the head, or None), RoPE and
        the KV store in one launch; ``q``/``k`` are rotated in place and
        returned.  With ``k_cache`` None nothing is stored."""
        if (q_norm is None) != (k_norm is None):
            raise ValueError("give both q_norm and k_norm or neither")
        if q_norm is not None and q_norm.eps != k_norm.eps:
            raise ValueError("q_norm and k_norm must share eps")
        return ops.qk_norm_rope_store(
            positions, q, k, self.cos_sin_cache,
            None if q_norm is None else q_norm.weight, None if k_norm is None else k_norm.weight,
            1e-6 if q_norm is None else q_norm.eps, v, k_cache, v_cache, slot_mapping,
        )


__all__ = ["KVCacheStore", "RMSNorm", "RotaryEmbedding", "SiluAndMul", "rope_table"]
