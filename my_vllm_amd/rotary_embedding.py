"""Rotary embedding CustomOp with a gfx950 provider.

Mirrors nanovllm/layers/rotary_embedding.py:18-151: neox-style RoPE over the
whole head, a precomputed fp32 ``cos_sin_cache`` ``[max_position, 1, dim]``
(cos | sin), the provider bound once at construction.  Providers:

* ``hip`` (alias ``flashinfer``, the reference's accelerated provider name):
  the gfx950 prologue kernel (``mva_qk_norm_rope_store`` without norm or
  store);
* ``native`` / ``native_torch``: the reference's torch formulation;
* ``auto``: ``hip`` on a GPU platform, ``native_torch`` otherwise.

``forward_fused`` additionally applies the per-head q/k RMSNorm and stores the
rotated K and V into the paged cache in the same launch (the reference runs
q_norm, k_norm, rotary_emb and the KV store as four ops,
nanovllm/models/qwen3.py:96-100 and nanovllm/layers/attention.py:140-141).
"""

from __future__ import annotations

from functools import lru_cache

import torch

from . import _native, ops
from .custom_op import CustomOp, CustomOpConfig


def apply_rotary_emb(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    x1, x2 = torch.chunk(x.float(), 2, dim=-1)
    y1 = x1 * cos - x2 * sin
    y2 = x2 * cos + x1 * sin
    return torch.cat((y1, y2), dim=-1).to(x.dtype)


class RotaryEmbedding(CustomOp):
    """Neox rotary embedding over the full head dimension."""

    op_name = "rotary_embedding"
    _SUPPORTED = frozenset({"auto", "native", "native_torch", "hip", "flashinfer"})

    def __init__(self, head_size: int, rotary_dim: int, max_position_embeddings: int, base: float,
                 custom_op_config: CustomOpConfig | None = None) -> None:
        super().__init__(custom_op_config)
        self.head_size = head_size
        assert rotary_dim == head_size
        inv_freq = 1.0 / (base ** (torch.arange(0, rotary_dim, 2, dtype=torch.float) / rotary_dim))
        t = torch.arange(max_position_embeddings, dtype=torch.float)
        freqs = torch.einsum("i,j -> ij", t, inv_freq)
        cache = torch.cat((freqs.cos(), freqs.sin()), dim=-1).unsqueeze_(1)
        self.register_buffer("cos_sin_cache", cache, persistent=False)
        self.provider_name, self.forward_impl = self._select_cuda_impl()

    def forward_native(self, positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor):
        cos_sin = self.cos_sin_cache[positions]
        cos, sin = cos_sin.chunk(2, dim=-1)
        return apply_rotary_emb(query, cos, sin), apply_rotary_emb(key, cos, sin)

    def forward_cuda(self, positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor):
        return self.forward_impl(positions, query, key)

    def forward_fused(self, positions, q, k, v, q_norm, k_norm, k_cache, v_cache, slot_mapping):
        """q_norm / k_norm (``RMSNorm`` modules over the head), RoPE and the KV
        store in one launch; ``q``/``k`` are rotated in place and returned."""
        if self.provider_name != "hip":
            raise RuntimeError("the fused prologue needs the hip rotary provider")
        eps = q_norm.eps if q_norm is not None else 1e-6
        if q_norm is not None and k_norm is not None and q_norm.eps != k_norm.eps:
            raise ValueError("q_norm and k_norm must share eps")
        return ops.qk_norm_rope_store(
            positions, q, k, self.cos_sin_cache,
            q_norm.weight if q_norm is not None else None, k_norm.weight if k_norm is not None else None, eps,
            v, k_cache, v_cache, slot_mapping,
        )

    def _select_cuda_impl(self):
        implementation = self.custom_op_config.implementation_for(self.op_name)
        if implementation not in self._SUPPORTED:
            available = ", ".join(sorted(self._SUPPORTED))
            raise ValueError(f"unsupported 'rotary_embedding' implementation {implementation!r}; available: {available}")
        if self.platform != "cuda" and implementation not in ("auto", "native", "native_torch"):
            raise RuntimeError(f"{implementation!r} for 'rotary_embedding' requires CUDA")
        if implementation in ("native", "native_torch") or self.platform != "cuda":
            return "native_torch", self.forward_native
        dtype = self.custom_op_config.dtype
        if dtype not in (torch.float16, torch.bfloat16, None) or self.head_size != ops.HEAD_DIM:
            if implementation == "auto":
                return "native_torch", self.forward_native
            raise RuntimeError(f"{implementation!r} for 'rotary_embedding' needs fp16/bf16 and head_size 128")
        _native.load_library()  # raises if the gfx950 library is missing

        def forward(positions, query, key):
            return ops.rotary_embedding(positions, query, key, self.cos_sin_cache, self.head_size)

        return "hip", forward


@lru_cache(1)
def _get_rope(head_size: int, rotary_dim: int, max_position: int, base: float, custom_op_config: CustomOpConfig):
    return RotaryEmbedding(head_size, rotary_dim, max_position, base, custom_op_config=custom_op_config)


def get_rope(head_size: int, rotary_dim: int, max_position: int, base: float | None, rope_scaling: dict | None = None,
             custom_op_config: CustomOpConfig | None = None):
    """Shared RotaryEmbedding per configuration (reference rotary_embedding.py:134-151)."""
    if rope_scaling is not None:
        rope_type = rope_scaling.get("rope_type", rope_scaling.get("type", "default"))
        if rope_type != "default":
            raise NotImplementedError(f"RoPE type {rope_type!r} is not supported")
        base = rope_scaling.get("rope_theta", base)
    if base is None:
        raise ValueError("RoPE theta is missing from the model configuration")
    return _get_rope(head_size, rotary_dim, max_position, float(base), custom_op_config or CustomOpConfig())
