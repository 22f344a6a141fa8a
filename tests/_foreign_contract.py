"""A second, independent class family with the reference's contract shape.

The reference-side integration builds the backend on the reference's own
``AttentionBackend``, ``AttentionPlan``, ``AttentionRoute``, ``BatchType`` and
``CommonAttentionMetadata`` and registers it in its ``AttentionBackendRegistry``
(nanovllm/layers/attention_backend.py:112-275, 1228-1273;
nanovllm/utils/context.py:7-43).  The reference cannot be imported here, so
these stand-ins are distinct classes with the same field names and enum
values: a backend that only works with this package's classes fails against
them.  Test infrastructure only.
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import Enum
from typing import Any

import torch


class ForeignBatchType(str, Enum):
    PURE_PREFILL = "pure_prefill"
    PURE_DECODE = "pure_decode"
    MIXED = "mixed"


class ForeignRoute(str, Enum):
    WARMUP = "warmup"
    PREFILL = "prefill"
    DECODE = "decode"
    MIXED_UNIFIED = "mixed_unified"
    MIXED_SPLIT = "mixed_split"


@dataclass(frozen=True)
class ForeignCommon:
    num_prefill_seqs: int
    num_decode_seqs: int
    num_prefill_tokens: int
    num_decode_tokens: int
    query_start_loc: torch.Tensor
    seq_lens: torch.Tensor
    slot_mapping: torch.Tensor
    block_tables: torch.Tensor | None = None
    max_q_len: int = 0
    max_kv_len: int = 0
    block_counts: tuple[int, ...] = ()
    num_kv_blocks: int = 0
    num_prefill_kv_blocks: int = 0
    trusted: bool = False

    @property
    def num_seqs(self) -> int:
        return self.num_prefill_seqs + self.num_decode_seqs

    @property
    def num_query_tokens(self) -> int:
        return self.num_prefill_tokens + self.num_decode_tokens


@dataclass(frozen=True)
class ForeignPlan:
    batch_type: ForeignBatchType
    route: ForeignRoute
    common: ForeignCommon
    metadata: Any


class ForeignBackendBase:
    """Only what a registered backend relies on: the constructor's fields and
    the capability classmethods."""

    def __init__(self, num_q_heads, num_kv_heads, head_dim, block_size, dtype):
        self.num_q_heads, self.num_kv_heads = num_q_heads, num_kv_heads
        self.head_dim, self.block_size, self.dtype = head_dim, block_size, dtype
        self.softmax_scale = head_dim ** -0.5

    @classmethod
    def support_reason(cls, **_: Any):
        return None

    @classmethod
    def supports(cls, **capabilities: Any) -> bool:
        return cls.support_reason(**capabilities) is None


class ForeignRegistry:
    """Name -> class map that accepts only subclasses of the foreign base."""

    backends: dict[str, type] = {}

    @classmethod
    def register(cls, name: str, backend_type: type) -> None:
        key = name.strip().lower()
        if not key or key == "auto" or key in cls.backends:
            raise ValueError(f"cannot register {name!r}")
        if not (isinstance(backend_type, type) and issubclass(backend_type, ForeignBackendBase)):
            raise TypeError("backend_type must be an AttentionBackend subclass")
        cls.backends[key] = backend_type

    @classmethod
    def support(cls, name: str, **capabilities: Any):
        backend_type = cls.backends[name]
        supported = backend_type.supports(**capabilities)
        return supported, (None if supported else backend_type.support_reason(**capabilities))


def to_foreign(common) -> ForeignCommon:
    """The same batch as a ForeignCommon."""
    return ForeignCommon(**common.__dict__)
