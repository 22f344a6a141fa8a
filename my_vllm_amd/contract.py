"""The backend-neutral attention contract this package plugs into.

Names, fields, enum values, exception classes and messages are those of the
reference, because callers and their tests see them:

* ``BatchType`` and ``CommonAttentionMetadata``: nanovllm/utils/context.py:7-43,
  the per-step contract the model runner fills
  (nanovllm/engine/model_runner.py:361-484);
* ``AttentionRoute`` / ``AttentionPlan``: nanovllm/layers/attention_backend.py:112-135;
* ``AttentionBackend``: the lifecycle base, :174-275;
* ``check_common_metadata``: the metadata rules of :1384-1481;
* ``classify_batch``: :1484-1491.

The per-step metadata, in brief: ``query_start_loc[S+1]`` packed query
offsets, ``seq_lens[S]`` context lengths including the step's new tokens,
``slot_mapping[T]`` cache slots ``page * 16 + offset`` (``-1`` skips),
``block_tables[S, W]`` page ids padded with ``-1``, all int32 on the GPU; host
ints describe the same batch so that trusted planning reads nothing back from
the device.  Prefill sequences come first, then decode sequences of one query
token each.

A backend that must live in the reference's own class family (to register in
its registry) names that family's classes in the attributes ``plan_type``,
``route_type``, ``batch_type_enum`` and ``common_type``; every check here takes
them as arguments.
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import Enum
from math import sqrt
from typing import Any

import torch


class BatchType(str, Enum):
    PURE_PREFILL = "pure_prefill"
    PURE_DECODE = "pure_decode"
    MIXED = "mixed"


@dataclass(frozen=True)
class CommonAttentionMetadata:
    """Backend-neutral metadata produced once for one scheduled batch."""

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


class AttentionRoute(str, Enum):
    WARMUP = "warmup"
    PREFILL = "prefill"
    DECODE = "decode"
    MIXED_UNIFIED = "mixed_unified"
    MIXED_SPLIT = "mixed_split"


@dataclass(frozen=True)
class AttentionPlan:
    """One explicit, backend-owned execution decision for a scheduled batch."""

    batch_type: BatchType
    route: AttentionRoute
    common: CommonAttentionMetadata
    metadata: Any

    @property
    def common_metadata(self) -> CommonAttentionMetadata:
        return self.common

    @property
    def backend_metadata(self) -> Any:
        return self.metadata


def _graph_unsupported(backend: Any) -> RuntimeError:
    return RuntimeError(f"{type(backend).__name__} does not support full decode CUDA Graph")


class AttentionBackend:
    """Unified lifecycle implemented by every complete attention backend.

    Subclasses implement ``build_metadata``, ``build_plan`` and ``forward``;
    the full-decode graph hooks default to "unsupported", which makes the
    model runner run decode eagerly.
    """

    backend_name = "base"
    supports_full_decode_graph = False

    def __init__(self, num_q_heads: int, num_kv_heads: int, head_dim: int, block_size: int,
                 dtype: torch.dtype) -> None:
        if min(num_q_heads, num_kv_heads) <= 0:
            raise ValueError("attention head counts must be positive")
        if num_q_heads % num_kv_heads != 0:
            raise ValueError("num_q_heads must be divisible by num_kv_heads")
        if min(head_dim, block_size) <= 0:
            raise ValueError("head_dim and block_size must be positive")
        self.num_q_heads, self.num_kv_heads = num_q_heads, num_kv_heads
        self.head_dim, self.block_size, self.dtype = head_dim, block_size, dtype
        self.softmax_scale = 1.0 / sqrt(head_dim)

    @classmethod
    def support_reason(cls, **capabilities: Any) -> str | None:
        return None

    @classmethod
    def supports(cls, **capabilities: Any) -> bool:
        return cls.support_reason(**capabilities) is None

    def build_metadata(self, common: CommonAttentionMetadata) -> Any:
        raise NotImplementedError

    def build_plan(self, common: CommonAttentionMetadata, metadata: Any | None = None) -> AttentionPlan:
        raise NotImplementedError

    def forward(self, q, k, v, k_cache, v_cache, plan: AttentionPlan) -> torch.Tensor:
        raise NotImplementedError

    def create_full_decode_graph_state(self, batch_size: int, page_indices_capacity: int, device) -> Any:
        raise _graph_unsupported(self)

    def full_decode_graph_metadata_fits(self, state: Any, plan: AttentionPlan) -> bool:
        return False

    def plan_full_decode_graph(self, state: Any, plan: AttentionPlan) -> None:
        raise _graph_unsupported(self)

    def activate_full_decode_graph(self, state: Any) -> None:
        raise _graph_unsupported(self)

    def deactivate_full_decode_graph(self) -> None:
        return None


# ---------------------------------------------------------------------------
# Metadata rules.  Each rule raises the reference's exception and message;
# they run in the reference's order, so a batch that breaks several rules
# reports the same first one.
# ---------------------------------------------------------------------------

_COUNT_FIELDS = ("num_prefill_seqs", "num_decode_seqs", "num_prefill_tokens", "num_decode_tokens", "max_q_len",
                 "max_kv_len", "num_kv_blocks", "num_prefill_kv_blocks")
_INDEX_TENSORS = ("query_start_loc", "seq_lens", "slot_mapping")


def _fail_unless(ok: bool, error: type[Exception], message: str) -> None:
    if not ok:
        raise error(message)


def _is_plain_int(value: Any) -> bool:
    return isinstance(value, int) and not isinstance(value, bool)


def _check_counts(common: Any) -> None:
    for name in _COUNT_FIELDS:
        value = getattr(common, name)
        _fail_unless(_is_plain_int(value), TypeError, f"common.{name} must be an int")
        _fail_unless(value >= 0, ValueError, f"common.{name} must be non-negative")
    _fail_unless(common.num_seqs > 0, ValueError, "attention metadata must contain at least one sequence")
    _fail_unless(common.num_decode_tokens == common.num_decode_seqs, ValueError,
                 "decode suffix must contain one query token per sequence")
    _fail_unless(isinstance(common.trusted, bool), TypeError, "common.trusted must be a bool")


def _check_index_tensor(common: Any, name: str, require_cuda: bool) -> None:
    tensor = getattr(common, name)
    _fail_unless(isinstance(tensor, torch.Tensor), TypeError, f"common.{name} must be a torch.Tensor")
    _fail_unless(tensor.dtype == torch.int32, TypeError, f"common.{name} must have dtype torch.int32")
    _fail_unless(tensor.ndim == 1, ValueError, f"common.{name} must be one-dimensional")
    _fail_unless(not require_cuda or tensor.device.type == "cuda", ValueError, f"common.{name} must be on CUDA")


def _check_lengths(common: Any) -> None:
    expected = {
        "query_start_loc": (common.num_seqs + 1, "query_start_loc length must equal number of sequences + 1"),
        "seq_lens": (common.num_seqs, "seq_lens length must equal number of sequences"),
        "slot_mapping": (common.num_query_tokens, "slot_mapping length must equal number of query tokens"),
    }
    for name, (length, message) in expected.items():
        _fail_unless(getattr(common, name).numel() == length, ValueError, message)


def _check_device_values(common: Any) -> None:
    """Rules that read device values; only untrusted metadata pays for them."""
    qsl = common.query_start_loc
    _fail_unless(int(qsl[0].item()) == 0, ValueError, "query_start_loc must start at zero")
    _fail_unless(int(qsl[-1].item()) == common.num_query_tokens, ValueError,
                 "query_start_loc must end at num_query_tokens")
    if common.num_decode_seqs:
        decode_lengths = qsl[common.num_prefill_seqs + 1:] - qsl[common.num_prefill_seqs:-1]
        _fail_unless(bool((decode_lengths == 1).all().item()), ValueError,
                     "every decode sequence must have one query token")
    _fail_unless(bool((common.seq_lens > 0).all().item()), ValueError, "all KV sequence lengths must be positive")


def _check_block_tables(common: Any, require_cuda: bool) -> None:
    table = common.block_tables
    if table is None:
        return
    _fail_unless(isinstance(table, torch.Tensor), TypeError, "common.block_tables must be a torch.Tensor")
    _fail_unless(table.dtype == torch.int32, TypeError, "common.block_tables must have dtype torch.int32")
    _fail_unless(table.ndim == 2, ValueError, "common.block_tables must be two-dimensional")
    _fail_unless(table.size(0) == common.num_seqs, ValueError,
                 "block_tables row count must equal number of sequences")
    _fail_unless(not require_cuda or table.device.type == "cuda", ValueError, "common.block_tables must be on CUDA")


def check_common_metadata(common: Any, *, require_cuda: bool, common_type: type = CommonAttentionMetadata) -> None:
    """Raise the reference's error for the first contract rule ``common`` breaks."""
    _fail_unless(isinstance(common, common_type), TypeError, "common must be CommonAttentionMetadata")
    _check_counts(common)
    for name in _INDEX_TENSORS:
        _check_index_tensor(common, name, require_cuda)
    _check_lengths(common)
    if not common.trusted:
        _check_device_values(common)
    _check_block_tables(common, require_cuda)


def classify_batch(common: Any, batch_types: type = BatchType):
    """PURE_DECODE without prefill sequences, PURE_PREFILL without decode
    sequences, MIXED otherwise (even when every query has one token)."""
    if common.num_prefill_seqs and common.num_decode_seqs:
        return batch_types.MIXED
    if common.num_prefill_seqs:
        return batch_types.PURE_PREFILL
    _fail_unless(common.num_decode_seqs > 0, ValueError, "pure decode batch must contain decode requests")
    return batch_types.PURE_DECODE


def plan_metadata(plan: Any, metadata_type: type, backend_name: str, plan_type: type = AttentionPlan) -> Any:
    """The backend metadata a plan carries, after checking both types."""
    _fail_unless(isinstance(plan, plan_type), TypeError, "attention forward requires AttentionPlan")
    _fail_unless(isinstance(plan.metadata, metadata_type), TypeError,
                 f"{backend_name} plan carries incompatible backend metadata")
    return plan.metadata


__all__ = [
    "AttentionBackend",
    "AttentionPlan",
    "AttentionRoute",
    "BatchType",
    "CommonAttentionMetadata",
    "check_common_metadata",
    "classify_batch",
    "plan_metadata",
]
