"""The MI355X (gfx950) attention backend.

``MI355XAttentionBackendMixin`` holds the whole implementation and takes the
plan/route/batch-type/metadata classes from class attributes, so the same code
runs on this package's contract classes (``MI355XAttentionBackend``) or on the
reference's own (``integrate`` builds those subclasses and registers them in
the reference's ``AttentionBackendRegistry``).

Per step: ``build_metadata`` turns the trusted host ints of
``CommonAttentionMetadata`` into device work lists (no device reads),
``build_plan`` classifies the batch once and picks one route, and ``forward``
launches the gfx950 kernels on the current stream into a reusable,
backend-owned output buffer:

* DECODE        -> paged GQA decode (piece lists or claims, split-K merge kernel)
* PREFILL       -> ragged causal chunked prefill over prefix-cached pages
* MIXED_UNIFIED -> one launch writing ``out[:P]`` (prefill) and ``out[P:]`` (decode)
* MIXED_SPLIT   -> prefill launch into ``out[:P]`` + decode launch into ``out[P:]``
* WARMUP        -> cacheless causal attention (no pages; one-time memory probe)
"""

from __future__ import annotations

from dataclasses import dataclass
from types import MappingProxyType
from typing import Any

import numpy as np
import torch

from . import _native, ops
from .contract import (
    AttentionBackend,
    AttentionPlan,
    AttentionRoute,
    BatchType,
    CommonAttentionMetadata,
    check_common_metadata,
    classify_batch,
    plan_metadata,
)


def _has_cache(cache: torch.Tensor | None) -> bool:
    return isinstance(cache, torch.Tensor) and cache.numel() > 0


# --------------------------------------------------------------------------
# MI355X backend.
# --------------------------------------------------------------------------

HEAD_DIM = ops.HEAD_DIM
PAGE_SIZE = ops.PAGE_SIZE
MAX_GROUP = 16


@dataclass(frozen=True)
class MI355XAttentionMetadata:
    """Backend-private per-step metadata: device work lists built on the host.

    ``decode_items`` is int32 ``[num_decode_items, 8]`` pieces run by
    ``num_decode_waves`` wavefronts, ``decode_waves_per_group`` to a
    workgroup; ``None`` without decode sequences.  With
    ``decode_wave_extra`` (int32 ``[num_decode_waves + 1]``) each wavefront
    runs its own piece list (``make_decode_plan_listed``); without it the
    wavefronts claim pieces (``make_decode_plan``).  ``decode_merges`` lists the split segments
    (``ops.decode_merge_list``) whose partials the merge kernel combines.
    Prefill query tiles are derived on the device from ``query_start_loc``
    and ``seq_lens``: ``prefill_max_tiles`` bounds those of the PREFILL and
    split routes (256-row tiles), ``mixed_prefill_max_tiles`` those of the
    single MIXED launch (128-row tiles).  ``kv_indptr`` is the page CSR
    offset list (host ints): sequence ``s`` owns pages
    ``block_tables[s, :kv_indptr[s+1]-kv_indptr[s]]``.
    """

    query_start_loc: torch.Tensor
    seq_lens: torch.Tensor
    block_tables: torch.Tensor | None
    kv_indptr: tuple[int, ...]
    num_pages: int
    num_prefill_pages: int
    decode_items: torch.Tensor | None = None
    num_decode_items: int = 0
    num_decode_waves: int = 0
    num_decode_part_slots: int = 0
    decode_merges: torch.Tensor | None = None
    num_decode_merges: int = 0
    decode_wave_extra: torch.Tensor | None = None
    decode_waves_per_group: int = 1
    # Host copy of a piece-list plan: (items, wave_extra, merges, workgroups).
    decode_host_plan: tuple | None = None
    # Bounds on the prefill query tiles (size the device-built tile list and
    # the MIXED launch's prefill pool).  On a MIXED batch,
    # mixed_prefill_max_tiles > 0 means one launch; 0 means prefill +
    # decode launches, for the reason in mixed_split_reason (split mode, or
    # more prefill sequences, KV heads or split-K pairs than one MIXED
    # launch takes).
    prefill_max_tiles: int = 0
    mixed_prefill_max_tiles: int = 0
    mixed_split_reason: str | None = None

    @property
    def is_cacheless(self) -> bool:
        return self.block_tables is None


# Decode wavefronts per CU.  The decode kernel fits 8 per CU (2 per SIMD), but
# fewer concurrent page streams read randomly permuted pages faster: measured
# on MI355X, 5 per CU beat 8 by 3-10% on 10 GB batches and matched it on a
# 1 GB batch (the UTCL1 miss rate grows with the streams in flight).  A
# single MIXED launch gives decode 6 per CU and leaves the remaining slots to
# the prefill tiles.
_DECODE_WAVES_PER_CU = 5
_MIXED_DECODE_WAVES_PER_CU = 6


def resident_decode_waves(device: torch.device | None = None, mixed: bool = False,
                          override: int | None = None) -> int:
    """Decode wavefronts per launch: CUs x 5 (x 6 in a MIXED launch); 1280 / 1536 on MI355X.

    ``override`` (a backend's ``decode_waves_override``) replaces the count."""
    if override:
        return max(1, int(override))
    per_cu = _MIXED_DECODE_WAVES_PER_CU if mixed else _DECODE_WAVES_PER_CU
    if device is not None and device.type == "cuda":
        return torch.cuda.get_device_properties(device).multi_processor_count * per_cu
    return 256 * per_cu


def _plan_counts(block_counts) -> np.ndarray:
    counts = np.ascontiguousarray(block_counts, dtype=np.int64).reshape(-1)
    if np.any(counts <= 0):
        raise ValueError("every decode sequence needs at least one page")
    return counts


def plan_decode_claims(
    block_counts: np.ndarray | tuple[int, ...],
    first_seq: int,
    first_q_row: int,
    num_kv_heads: int,
    num_waves: int,
    pieces_per_wave: float = 1.5,
    min_piece_pages: int = 4,
    max_piece_pages: int = ops.MAX_CHUNK_PAGES,
) -> tuple[np.ndarray, int, int, np.ndarray]:
    """:func:`make_decode_plan` plus its merge list (as
    :func:`ops.decode_merge_list` would give it), from the library's native
    planner ``mva_decode_plan_claims``."""
    counts = _plan_counts(block_counts)
    if not 1 <= min_piece_pages <= max_piece_pages <= ops.MAX_CHUNK_PAGES:
        raise ValueError("piece length bounds must satisfy 1 <= min <= max <= 128")
    n = counts.size
    if n == 0:
        empty = np.zeros((0, ops.DECODE_ITEM_INTS), np.int32)
        return empty, 0, 0, empty
    rows = int(_native.query("mva_decode_plan_claims_rows", n, int(counts.sum()), int(num_kv_heads),
                             int(min_piece_pages)))
    if rows < 0:
        raise ValueError("invalid decode plan arguments")
    items = np.empty((rows, ops.DECODE_ITEM_INTS), np.int32)
    merges = np.empty((n * int(num_kv_heads), ops.DECODE_ITEM_INTS), np.int32)
    out = np.zeros(4, np.int64)
    _native.call("mva_decode_plan_claims", counts.ctypes.data, n, int(first_seq), int(first_q_row),
                 int(num_kv_heads), int(num_waves), float(pieces_per_wave), int(min_piece_pages),
                 int(max_piece_pages), items.ctypes.data, rows, merges.ctypes.data, merges.shape[0],
                 out.ctypes.data)
    num_items, waves, slots, num_merges = (int(x) for x in out)
    return items[:num_items], waves, slots, merges[:num_merges]


def make_decode_plan(
    block_counts: np.ndarray | tuple[int, ...],
    first_seq: int,
    first_q_row: int,
    num_kv_heads: int,
    num_waves: int,
    pieces_per_wave: float = 1.5,
    min_piece_pages: int = 4,
    max_piece_pages: int = ops.MAX_CHUNK_PAGES,
) -> tuple[np.ndarray, int, int]:
    """Cut a decode batch into pieces that wavefronts claim dynamically.

    Sequence ``first_seq + i`` has ``block_counts[i]`` pages and reads query
    row ``first_q_row + i``.  Every (sequence, KV head) segment of ``L`` pages
    is cut into ``ceil(L / P)`` near-equal pieces, with the piece length ``P``
    chosen so that ``num_waves`` wavefronts see about ``pieces_per_wave``
    pieces each (clamped to ``[min_piece_pages, max_piece_pages]``); short
    pieces let the wavefronts on faster CUs take more of the work.  A piece
    is ``(seq, page_begin, page_end, chunk, n_chunks, part_base, q_row,
    kv_head)``; a sequence cut into ``n_chunks > 1`` pieces per KV head owns
    that many split-K partial slots from ``part_base``, shared by its KV
    heads (the kernel's slot is ``(part_base + chunk) * Hkv + kv_head``, as
    with piece lists).  Pieces are ordered longest
    first, then sequence-major with the KV head fastest (the head slices of
    one page are neighbours in the cache).  Returns ``(items, waves,
    num_part_slots)`` with ``waves = min(num_waves, len(items))``, the grid to
    launch.  The plan is computed by the library's host-side planner
    (``mva_decode_plan_claims``), once per step.
    """
    return plan_decode_claims(block_counts, first_seq, first_q_row, num_kv_heads, num_waves, pieces_per_wave,
                              min_piece_pages, max_piece_pages)[:3]


# Workgroups of a piece-list decode launch fill 8 wave slots per CU (the
# kernel's occupancy is 2 wavefronts per SIMD).
_LISTED_WAVES_PER_CU = 8
# Piece lists (an equal share of pages per wavefront, no claims) at every
# size when a workgroup holds all 8 KV heads of its range (one CU streams
# every head of the same pages): measured as fast as claims or faster from
# 1.3 to 11.2 GB of K/V (3.21 GB, 16 sequences of 32K-64K tokens: 5.6 against
# 4.95 TB/s; 4.6 GB, 256 sequences of 512-8192: 5.75 against 5.4 TB/s).  Other
# head counts use them up to this many K/V bytes per launch (at 4 KV heads
# and 4.8 GB, claims measured 2% faster); larger batches use claims.
_LISTED_MAX_BYTES = 2 << 30


def decode_schedule(total_pages: int, num_kv_heads: int, elem_bytes: int = 2, forced: str | None = None) -> str:
    """"listed" or "claims" for a decode batch of ``total_pages`` pages (``forced``,
    a backend's ``decode_schedule_override``, picks one)."""
    if forced is not None:
        if forced not in ("listed", "claims"):
            raise ValueError("decode schedule must be 'listed' or 'claims'")
        return forced
    if num_kv_heads == _LISTED_WAVES_PER_CU:
        return "listed"
    kv_bytes = total_pages * PAGE_SIZE * num_kv_heads * HEAD_DIM * elem_bytes * 2
    return "listed" if kv_bytes <= _LISTED_MAX_BYTES else "claims"


def listed_decode_groups(num_kv_heads: int, device: torch.device | None = None,
                         override: int | None = None) -> tuple[int, int]:
    """(workgroups, wavefronts per workgroup) of a piece-list decode launch.

    A workgroup holds one wavefront per KV head when the head count divides 8
    (so one CU streams every head of the same pages), else one wavefront.
    ``override`` (a backend's ``decode_waves_override``) sets the wavefront
    count the workgroups share.
    """
    per_group = num_kv_heads if num_kv_heads in (1, 2, 4, 8) else 1
    cus = 256
    if device is not None and device.type == "cuda":
        cus = torch.cuda.get_device_properties(device).multi_processor_count
    waves = max(1, int(override)) if override else cus * _LISTED_WAVES_PER_CU
    return max(1, waves // num_kv_heads), per_group


def plan_decode_listed(
    block_counts: np.ndarray | tuple[int, ...],
    first_seq: int,
    first_q_row: int,
    num_kv_heads: int,
    num_groups: int,
    max_piece_pages: int = ops.MAX_CHUNK_PAGES,
) -> tuple[np.ndarray, np.ndarray, int, int, np.ndarray]:
    """:func:`make_decode_plan_listed` plus its merge list (as
    :func:`ops.decode_merge_list` would give it), from the library's native
    planner ``mva_decode_plan_listed``."""
    counts = _plan_counts(block_counts)
    if not 1 <= max_piece_pages <= ops.MAX_CHUNK_PAGES:
        raise ValueError("piece length must be in [1, 128] pages")
    n = counts.size
    if n == 0:
        empty = np.zeros((0, ops.DECODE_ITEM_INTS), np.int32)
        return empty, np.zeros(1, np.int32), 0, 0, empty
    hkv = int(num_kv_heads)
    total = int(counts.sum())
    num_groups = max(1, int(num_groups))
    rows = int(_native.query("mva_decode_plan_listed_rows", n, total, hkv, num_groups, int(max_piece_pages)))
    if rows < 0:
        raise ValueError("invalid decode plan arguments")
    items = np.empty((rows, ops.DECODE_ITEM_INTS), np.int32)
    merges = np.empty((n * hkv, ops.DECODE_ITEM_INTS), np.int32)
    wave_extra = np.empty(min(num_groups, total) * hkv + 1, np.int32)
    out = np.zeros(4, np.int64)
    _native.call("mva_decode_plan_listed", counts.ctypes.data, n, int(first_seq), int(first_q_row), hkv,
                 num_groups, int(max_piece_pages), items.ctypes.data, rows, wave_extra.ctypes.data,
                 wave_extra.size, merges.ctypes.data, merges.shape[0], out.ctypes.data)
    num_items, waves, slots, num_merges = (int(x) for x in out)
    return items[:num_items], wave_extra, waves, slots, merges[:num_merges]


def make_decode_plan_listed(
    block_counts: np.ndarray | tuple[int, ...],
    first_seq: int,
    first_q_row: int,
    num_kv_heads: int,
    num_groups: int,
    max_piece_pages: int = ops.MAX_CHUNK_PAGES,
) -> tuple[np.ndarray, np.ndarray, int, int]:
    """An equal share of the batch's pages for every wavefront, as piece lists.

    The pages of all sequences, in batch order, are cut into ``G =
    min(num_groups, total pages)`` contiguous ranges of near-equal length
    (range ``g`` = pages ``[g*T//G, (g+1)*T//G)``).  Wavefront ``g*Hkv + h``
    streams KV head ``h`` of range ``g``: one piece per sequence the range
    touches (cut further to at most ``max_piece_pages``).  A (sequence, KV
    head) spread over several pieces is split-K: its pieces are chunks
    ``0..n-1`` in page order, with partial slots ``part_base .. part_base +
    n - 1`` shared by the sequence's KV heads (slot ``(part_base + chunk) *
    Hkv + h``).  Every wavefront gets at least one piece.

    Returns ``(items, wave_extra, waves, num_part_slots)``: items hold the
    first piece of wavefront ``w`` at row ``w`` and its later pieces, in page
    order, at rows ``wave_extra[w] .. wave_extra[w + 1] - 1``.  The plan is
    computed by the library's host-side planner (``mva_decode_plan_listed``),
    once per step.
    """
    return plan_decode_listed(block_counts, first_seq, first_q_row, num_kv_heads, num_groups, max_piece_pages)[:4]


def _to_device(array: np.ndarray, device: torch.device) -> torch.Tensor:
    """Host int32 array -> device tensor through pinned memory (async H2D)."""
    host = torch.from_numpy(np.ascontiguousarray(array))
    if device.type != "cuda":
        return host.to(device)
    return host.pin_memory().to(device, non_blocking=True)


class PinnedStaging:
    """A ring of pinned host buffers for the per-step int32 work lists.

    Each host-to-device copy takes the next buffer of the ring, allocated
    once and grown only when a list outgrows it; before refilling a buffer
    the host waits on the event of that buffer's previous copy, issued
    ``slots`` copies earlier and normally long complete.  So planning pins
    no memory per step and the host can run ahead of the device by up to
    ``slots`` steps.
    """

    def __init__(self, slots: int = 4):
        self._buffers: list[torch.Tensor | None] = [None] * slots
        self._events: list[Any] = [None] * slots
        self._next = 0

    def to_device(self, array: np.ndarray, device: torch.device) -> torch.Tensor:
        host = np.ascontiguousarray(array, dtype=np.int32).reshape(-1)
        if device.type != "cuda":
            return torch.from_numpy(host.copy()).to(device)
        k = self._next
        self._next = (k + 1) % len(self._buffers)
        if self._events[k] is not None:
            self._events[k].synchronize()
        buf = self._buffers[k]
        if buf is None or buf.numel() < host.size:
            buf = torch.empty(max(host.size, 4096, 2 * (buf.numel() if buf is not None else 0)),
                              dtype=torch.int32, pin_memory=True)
            self._buffers[k] = buf
        buf[: host.size].copy_(torch.from_numpy(host))
        out = torch.empty(host.size, dtype=torch.int32, device=device)
        out.copy_(buf[: host.size], non_blocking=True)
        # The copy runs on `device`'s current stream, which need not be the
        # current device's: record there.
        event = torch.cuda.Event()
        event.record(torch.cuda.current_stream(device))
        self._events[k] = event
        return out


def _device_arch(device: torch.device) -> str:
    props = torch.cuda.get_device_properties(device)
    return getattr(props, "gcnArchName", "") or ""


@dataclass
class MI355XFullDecodeGraphState:
    """Fixed-address buffers of one captured full-decode graph (one batch size).

    ``plan_buffer`` holds ``{num_items, num_waves, num_merges}``, then the
    pieces (``item_capacity`` x 8), the piece-list offsets (``wave_capacity``
    + 1) and the merge list (``merge_capacity`` x 8), as laid out by
    :func:`pack_graph_decode_plan`.  Mirrors the reference's
    ``_FlashInferFullDecodeGraphState`` (attention_backend.py:162-171).
    """

    batch_size: int
    page_indices_capacity: int
    groups: int
    waves_per_group: int
    item_capacity: int
    wave_capacity: int
    merge_capacity: int
    part_slot_capacity: int
    block_tables_buffer: torch.Tensor
    seq_lens_buffer: torch.Tensor
    plan_buffer: torch.Tensor
    # Two pinned staging copies of the plan, used in turn, each with the
    # event of its last host-to-device copy.
    plan_staging: list
    staging_ready: list
    workspace: torch.Tensor
    output: torch.Tensor
    plan: Any = None
    staging_turn: int = 0

    def views(self):
        """(counts, items, wave_extra, merges) views of the device plan buffer."""
        return split_graph_plan_buffer(self.plan_buffer, self.item_capacity, self.wave_capacity,
                                       self.merge_capacity)


def graph_decode_capacities(batch_size: int, page_capacity: int, num_kv_heads: int, groups: int) -> dict:
    """Largest piece-list plan of ``batch_size`` sequences over at most
    ``page_capacity`` pages (``make_decode_plan_listed`` with ``groups``
    workgroups): the page ranges and sequences cut the pages into at most
    ``groups + batch_size - 1`` intervals, each split into ``ceil(L/128)``
    pieces per KV head."""
    intervals = groups + batch_size + page_capacity // ops.MAX_CHUNK_PAGES + 1
    return {
        "item_capacity": intervals * num_kv_heads,
        "wave_capacity": groups * num_kv_heads,
        "merge_capacity": batch_size * num_kv_heads,
        "part_slot_capacity": intervals,
    }


def graph_plan_buffer_ints(item_capacity: int, wave_capacity: int, merge_capacity: int) -> int:
    return 3 + item_capacity * ops.DECODE_ITEM_INTS + wave_capacity + 1 + merge_capacity * ops.DECODE_ITEM_INTS


def split_graph_plan_buffer(buffer, item_capacity: int, wave_capacity: int, merge_capacity: int):
    """(counts, items, wave_extra, merges) views of a packed graph plan."""
    a = 3
    b = a + item_capacity * ops.DECODE_ITEM_INTS
    c = b + wave_capacity + 1
    d = c + merge_capacity * ops.DECODE_ITEM_INTS
    return (buffer[:a], buffer[a:b].reshape(item_capacity, ops.DECODE_ITEM_INTS), buffer[b:c],
            buffer[c:d].reshape(merge_capacity, ops.DECODE_ITEM_INTS))


def pack_graph_decode_plan(items: np.ndarray, wave_extra: np.ndarray, merges: np.ndarray, item_capacity: int,
                           wave_capacity: int, merge_capacity: int, out: np.ndarray | None = None) -> np.ndarray:
    """Lay a piece-list plan out at the fixed offsets of a graph plan buffer."""
    waves = wave_extra.size - 1
    if items.shape[0] > item_capacity or waves > wave_capacity or merges.shape[0] > merge_capacity:
        raise ValueError("decode plan exceeds the graph state's capacity")
    size = graph_plan_buffer_ints(item_capacity, wave_capacity, merge_capacity)
    if out is None:
        out = np.zeros(size, dtype=np.int32)
    counts, it, we, mg = split_graph_plan_buffer(out, item_capacity, wave_capacity, merge_capacity)
    counts[:] = (items.shape[0], waves, merges.shape[0])
    it[: items.shape[0]] = items
    we[: waves + 1] = wave_extra
    mg[: merges.shape[0]] = merges
    return out


class MI355XAttentionBackendMixin:
    """The MI355X backend implementation, independent of the concrete base class.

    Subclasses combine it with an ``AttentionBackend`` base and name the
    plan/route/batch-type/metadata classes of that base's family.
    """

    backend_name = "mi355x"
    supports_full_decode_graph = True
    default_attention_mode = "unified"
    plan_type: type = AttentionPlan
    route_type: type = AttentionRoute
    batch_type_enum: type = BatchType
    common_type: type = CommonAttentionMetadata
    # Metadata tensors must live on the GPU (the reference's contract,
    # attention_backend.py:1436-1440); host-only planning tests relax it.
    require_device_metadata = True
    # Planning overrides, set as attributes by tests and tuning scripts (never
    # read from the environment): the decode wavefront count, and "listed" or
    # "claims" for the decode schedule.  None keeps the measured defaults.
    decode_waves_override: int | None = None
    decode_schedule_override: str | None = None
    # Debug check of forward_with_kv_store: read the fused store's error word
    # after each fused launch (a device read) and raise if a row's slot was
    # not its sequence's last position.
    check_fused_store: bool = False

    def __init__(
        self,
        num_q_heads: int,
        num_kv_heads: int,
        head_dim: int,
        block_size: int,
        dtype: torch.dtype,
        attention_mode: str | None = None,
    ) -> None:
        super().__init__(num_q_heads, num_kv_heads, head_dim, block_size, dtype)
        attention_mode = attention_mode or self.default_attention_mode
        if attention_mode not in ("unified", "split"):
            raise ValueError("attention_mode must be 'unified' or 'split'")
        if dtype not in (torch.float16, torch.bfloat16):
            raise TypeError("MI355X attention supports only float16 and bfloat16")
        if head_dim != HEAD_DIM:
            raise ValueError(f"MI355X attention requires head_dim {HEAD_DIM}")
        if block_size != PAGE_SIZE:
            raise ValueError(f"MI355X attention requires block_size {PAGE_SIZE}")
        if num_q_heads // num_kv_heads > MAX_GROUP:
            raise ValueError(f"MI355X attention supports at most {MAX_GROUP} query heads per KV head")
        _native.load_library()
        self.attention_mode = attention_mode
        self._reset_state()
        self._mixed_attention_unavailable_reason = self._backend_mixed_reason()

    def _reset_state(self) -> None:
        self._planned_route: str | None = None
        self._route_counts = {route.value: 0 for route in self.route_type}
        self._output_buffer: torch.Tensor | None = None
        self._workspace: torch.Tensor | None = None
        self._prefill_workspace: torch.Tensor | None = None
        # The metadata whose device tile plan the prefill workspace holds:
        # the first prefill launch of a step plans, the other layers reuse it.
        self._prefill_planned_for: MI355XAttentionMetadata | None = None
        self._staging = PinnedStaging()
        self._active_graph_state: MI355XFullDecodeGraphState | None = None
        # (key, value, slot_mapping) of the step while forward_with_kv_store
        # folds the KV store into the decode launch.
        self._pending_store: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None

    # ---- capability contract -------------------------------------------------
    @classmethod
    def support_reason(
        cls,
        *,
        block_size: int,
        dtype: torch.dtype,
        device: torch.device | str | None = None,
        num_q_heads: int | None = None,
        num_kv_heads: int | None = None,
        head_dim: int | None = None,
        attention_mode: str = "unified",
        **_: Any,
    ) -> str | None:
        if block_size != PAGE_SIZE:
            return f"block_size must be {PAGE_SIZE}"
        if head_dim is not None and head_dim != HEAD_DIM:
            return f"head_dim must be {HEAD_DIM}"
        if dtype not in (torch.float16, torch.bfloat16):
            return "dtype must be float16 or bfloat16"
        if attention_mode not in ("unified", "split"):
            return "attention_mode must be 'unified' or 'split'"
        if num_q_heads is not None and num_kv_heads is not None:
            if num_kv_heads <= 0 or num_q_heads % num_kv_heads:
                return "num_q_heads must be a multiple of num_kv_heads"
            if num_q_heads // num_kv_heads > MAX_GROUP:
                return f"at most {MAX_GROUP} query heads per KV head"
        selected = (
            torch.device(device)
            if device is not None
            else torch.device("cuda", torch.cuda.current_device() if torch.cuda.is_available() else 0)
        )
        if selected.type != "cuda" or not torch.cuda.is_available():
            return "a ROCm GPU device is required"
        arch = _device_arch(selected)
        if not arch.startswith("gfx950"):
            return f"a gfx950 (MI355X) device is required, found {arch or 'unknown'}"
        if not _native.native_available():
            return f"native library unavailable ({_native.LIB_PATH}); run `python -m my_vllm_amd.build`"
        return None

    @property
    def planned_route(self) -> str | None:
        return self._planned_route

    @property
    def route_counts(self):
        return MappingProxyType(dict(self._route_counts))

    # ---- MIXED capability (reference attention_backend.py:626-663) -----------
    @property
    def mixed_attention_available(self) -> bool:
        """Whether MIXED batches run as one launch (route MIXED_UNIFIED).

        False in split mode and beyond one MIXED launch's limits; after a
        MIXED batch is planned it describes that batch, so the route
        ``build_plan`` returned always equals the capability route
        (``"mixed_unified"`` if available, else ``"mixed_split"``).
        """
        return self._mixed_attention_unavailable_reason is None

    @property
    def mixed_attention_unavailable_reason(self) -> str | None:
        """Why MIXED batches run as prefill + decode launches (None when they
        run as one launch)."""
        return self._mixed_attention_unavailable_reason

    def _backend_mixed_reason(self) -> str | None:
        if self.attention_mode != "unified":
            return "unified mixed attention is disabled in split mode"
        if self.num_kv_heads > ops.MIXED_MAX_KV_HEADS:
            return (f"one MIXED launch takes at most {ops.MIXED_MAX_KV_HEADS} KV heads, "
                    f"the backend has {self.num_kv_heads}")
        return None

    def _batch_mixed_reason(self, common) -> str | None:
        """Why this MIXED batch cannot run as one launch (None if it can),
        before its decode plan is known."""
        reason = self._backend_mixed_reason()
        if reason is None and common.num_prefill_seqs > ops.MIXED_PREFILL_SEQS_MAX:
            reason = (f"one MIXED launch orders at most {ops.MIXED_PREFILL_SEQS_MAX} prefill sequences, "
                      f"the batch has {common.num_prefill_seqs}")
        return reason

    # ---- per-step metadata and plan ------------------------------------------
    def build_metadata(self, common) -> MI355XAttentionMetadata:
        check_common_metadata(common, require_cuda=self.require_device_metadata, common_type=self.common_type)
        if common.block_tables is None:
            return MI355XAttentionMetadata(
                query_start_loc=common.query_start_loc,
                seq_lens=common.seq_lens,
                block_tables=None,
                kv_indptr=(),
                num_pages=0,
                num_prefill_pages=0,
            )
        block_tables = common.block_tables
        max_pages = block_tables.size(1)
        if common.trusted:
            block_counts = common.block_counts
            if not isinstance(block_counts, tuple):
                raise TypeError("trusted block_counts must be a tuple")
            if len(block_counts) != common.num_seqs:
                raise ValueError("trusted block_counts length must equal num_seqs")
            # Plain ints within range (the common case) pass on two builtin
            # scans; anything else is judged element by element.
            if not all(type(count) is int for count in block_counts) or (
                block_counts and not (min(block_counts) > 0 and max(block_counts) <= max_pages)
            ):
                if any(
                    isinstance(count, bool) or not isinstance(count, int) or not 0 < count <= max_pages
                    for count in block_counts
                ):
                    raise ValueError("trusted block_counts contains an invalid row count")
            counts = np.asarray(block_counts, dtype=np.int64)
        else:
            page_counts = (common.seq_lens.to(torch.int64) + self.block_size - 1) // self.block_size
            counts = page_counts.cpu().numpy()
            if np.any(counts <= 0) or np.any(counts > max_pages):
                raise ValueError("seq_lens need more pages than block_tables holds")
            columns = torch.arange(max_pages, device=block_tables.device)
            needed = columns.unsqueeze(0) < page_counts.to(block_tables.device).unsqueeze(1)
            if bool(torch.any(block_tables[needed] < 0).item()):
                raise ValueError("block_tables contains an invalid page index")
        offsets = np.concatenate(([0], np.cumsum(counts)))
        num_pages = int(offsets[-1])
        num_prefill_pages = int(offsets[common.num_prefill_seqs])
        if common.trusted:
            if common.num_kv_blocks != num_pages:
                raise ValueError("trusted num_kv_blocks must match block_counts")
            if common.num_prefill_kv_blocks != num_prefill_pages:
                raise ValueError("trusted num_prefill_kv_blocks must match block_counts")

        decode_items = None
        decode_merges = None
        decode_wave_extra = None
        decode_host_plan = None
        num_decode_items = 0
        num_decode_merges = 0
        num_decode_waves = 0
        num_part_slots = 0
        waves_per_group = 1
        # A MIXED batch runs as one launch when it fits that launch's limits;
        # split_reason says why not.
        mixed = bool(common.num_prefill_seqs and common.num_decode_seqs)
        split_reason = self._batch_mixed_reason(common) if mixed else None
        one_launch = mixed and split_reason is None
        if common.num_decode_seqs:
            decode_counts = counts[common.num_prefill_seqs:]
            wave_extra = None
            if one_launch:
                items, num_decode_waves, num_part_slots, _ = plan_decode_claims(
                    decode_counts, common.num_prefill_seqs, common.num_prefill_tokens, self.num_kv_heads,
                    resident_decode_waves(block_tables.device, mixed=True, override=self.decode_waves_override),
                )
                # Its split-K arrival counters cover a bounded number of
                # (partial slot, KV head) pairs.
                if num_part_slots * self.num_kv_heads > ops.MIXED_ARRIVAL_COUNTERS:
                    one_launch = False
                    split_reason = (f"one MIXED launch merges at most {ops.MIXED_ARRIVAL_COUNTERS} split-K "
                                    f"(partial slot, KV head) pairs, the decode plan has "
                                    f"{num_part_slots * self.num_kv_heads}")
            if not one_launch:
                schedule = decode_schedule(int(decode_counts.sum()), self.num_kv_heads,
                                           forced=self.decode_schedule_override)
                if schedule == "listed":
                    groups, waves_per_group = listed_decode_groups(self.num_kv_heads, block_tables.device,
                                                                   override=self.decode_waves_override)
                    items, wave_extra, num_decode_waves, num_part_slots, merges = plan_decode_listed(
                        decode_counts, common.num_prefill_seqs, common.num_prefill_tokens, self.num_kv_heads, groups
                    )
                else:
                    items, num_decode_waves, num_part_slots, merges = plan_decode_claims(
                        decode_counts,
                        common.num_prefill_seqs,
                        common.num_prefill_tokens,
                        self.num_kv_heads,
                        resident_decode_waves(block_tables.device, override=self.decode_waves_override),
                    )
            else:
                # The single MIXED launch merges split segments itself.
                merges = np.zeros((0, ops.DECODE_ITEM_INTS), np.int32)
            num_decode_items = items.shape[0]
            num_decode_merges = merges.shape[0]
            # Pieces, merge entries and piece-list offsets share one
            # host-to-device copy.
            parts = [items.reshape(-1), merges.reshape(-1)]
            if wave_extra is not None:
                parts.append(wave_extra)
            flat = self._staging.to_device(np.concatenate(parts), block_tables.device)
            n_items, n_merge = num_decode_items * ops.DECODE_ITEM_INTS, num_decode_merges * ops.DECODE_ITEM_INTS
            decode_items = flat[:n_items].view(num_decode_items, ops.DECODE_ITEM_INTS)
            decode_merges = flat[n_items:n_items + n_merge].view(num_decode_merges, ops.DECODE_ITEM_INTS)
            if wave_extra is not None:
                decode_wave_extra = flat[n_items + n_merge:]
                decode_host_plan = (items, wave_extra, merges, groups)
        prefill_max_tiles = 0
        mixed_prefill_max_tiles = 0
        if common.num_prefill_seqs:
            prefill_max_tiles = ops.prefill_max_tiles(common.num_prefill_tokens, common.num_prefill_seqs,
                                                      self.num_q_heads, self.num_kv_heads)
            if one_launch:
                mixed_prefill_max_tiles = ops.mixed_prefill_max_tiles(
                    common.num_prefill_tokens, common.num_prefill_seqs, self.num_q_heads, self.num_kv_heads
                )
        return MI355XAttentionMetadata(
            query_start_loc=common.query_start_loc,
            seq_lens=common.seq_lens,
            block_tables=block_tables,
            kv_indptr=tuple(offsets.tolist()),
            num_pages=num_pages,
            num_prefill_pages=num_prefill_pages,
            decode_items=decode_items,
            num_decode_items=num_decode_items,
            num_decode_waves=num_decode_waves,
            num_decode_part_slots=num_part_slots,
            decode_merges=decode_merges,
            num_decode_merges=num_decode_merges,
            decode_wave_extra=decode_wave_extra,
            decode_waves_per_group=waves_per_group,
            decode_host_plan=decode_host_plan,
            prefill_max_tiles=prefill_max_tiles,
            mixed_prefill_max_tiles=mixed_prefill_max_tiles,
            mixed_split_reason=split_reason if mixed and not one_launch else None,
        )

    def build_plan(self, common, metadata: MI355XAttentionMetadata | None = None):
        if metadata is None:
            metadata = self.build_metadata(common)
        if not isinstance(metadata, MI355XAttentionMetadata):
            raise TypeError("MI355X attention requires MI355XAttentionMetadata")
        Route = self.route_type
        Batch = self.batch_type_enum
        # The single phase classification point for the whole batch.
        batch_type = classify_batch(common, Batch)
        if metadata.is_cacheless:
            route = Route.WARMUP
        elif batch_type is Batch.PURE_PREFILL:
            route = Route.PREFILL
        elif batch_type is Batch.PURE_DECODE:
            route = Route.DECODE
        else:
            # MIXED_UNIFIED exactly when the metadata plans one launch; the
            # capability properties then describe this batch.
            one_launch = metadata.mixed_prefill_max_tiles > 0
            route = Route.MIXED_UNIFIED if one_launch else Route.MIXED_SPLIT
            self._mixed_attention_unavailable_reason = (
                None if one_launch else metadata.mixed_split_reason or self._backend_mixed_reason()
                or "the MIXED metadata was planned for prefill + decode launches"
            )
        plan = self.plan_type(batch_type, route, common, metadata)
        self._prefill_planned_for = None  # a new step plans its prefill tiles again
        self._planned_route = route.value
        self._route_counts[route.value] += 1
        return plan

    # ---- buffers ---------------------------------------------------------------
    def _get_reusable_attention_output(self, q: torch.Tensor) -> torch.Tensor:
        required = q.size(0)
        buffer = self._output_buffer
        if (
            buffer is None
            or buffer.size(0) < required
            or buffer.shape[1:] != q.shape[1:]
            or buffer.device != q.device
            or buffer.dtype != q.dtype
        ):
            buffer = torch.empty_like(q)
            self._output_buffer = buffer
        return buffer[:required]

    def _get_prefill_workspace(self, max_tiles: int, device: torch.device) -> torch.Tensor:
        nbytes = ops.prefill_workspace_bytes(max_tiles)
        ws = self._prefill_workspace
        if ws is None or ws.numel() < nbytes or ws.device != device:
            ws = torch.empty(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
            self._prefill_workspace = ws
            self._prefill_planned_for = None
        return ws

    def _get_workspace(self, nbytes: int, device: torch.device) -> torch.Tensor | None:
        if nbytes <= 0:
            return None
        ws = self._workspace
        if ws is None or ws.numel() < nbytes or ws.device != device:
            # Zeroed once: the kernels leave their counters at zero on exit.
            ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            self._workspace = ws
        return ws

    # ---- forward ------------------------------------------------------------------
    def _validate_inputs(self, q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor) -> None:
        if q.device.type != "cuda" or q.dtype != self.dtype:
            raise ValueError("query must be a CUDA tensor with the backend dtype")
        if q.ndim != 3 or q.shape[1:] != (self.num_q_heads, self.head_dim):
            raise ValueError("query must have shape [tokens, num_q_heads, head_dim]")
        if q.stride(2) != 1:
            raise ValueError("query must have unit stride in head_dim")
        expected_tail = (self.block_size, self.num_kv_heads, self.head_dim)
        for name, cache in (("key", k_cache), ("value", v_cache)):
            if cache.device != q.device or cache.dtype != self.dtype:
                raise ValueError(f"{name} cache must share the query device and dtype")
            if cache.ndim != 4 or cache.shape[1:] != expected_tail:
                raise ValueError(f"{name} cache must have shape [pages, block_size, num_kv_heads, head_dim]")
            if cache.stride(3) != 1 or cache.stride(2) != self.head_dim or cache.stride(1) != self.num_kv_heads * self.head_dim:
                raise ValueError(f"{name} cache pages must be contiguous")
        if k_cache.shape != v_cache.shape or k_cache.stride() != v_cache.stride():
            raise ValueError("key and value caches must share shape and layout")

    def forward_with_kv_store(self, q, k, v, k_cache, v_cache, slot_mapping, plan, store=None) -> torch.Tensor:
        """The KV store of ``Attention.forward`` (``attention.py:140-141``) followed by
        :meth:`forward`, as one call.

        A DECODE step of trusted metadata planned with piece lists writes the
        new rows inside the decode launch (``mva_paged_decode_store``).  The
        model runner's slots are each sequence's last position
        (``model_runner.py:361-484``); for those the result and the caches
        are those of the store followed by the decode.  A row with any other
        slot is still written (by the kernel after the decode), so the caches
        always match the store, but this step's attention did not see it
        there; the workspace error word records it (``fused_store_error``,
        or ``check_fused_store`` to raise at once).  Every other step runs
        ``store`` (the layer's ``KVCacheStore``; the HIP store when None) and
        then :meth:`forward`.
        """
        metadata = plan.metadata if isinstance(plan, self.plan_type) else None
        if (
            self._active_graph_state is None
            and isinstance(metadata, MI355XAttentionMetadata)
            and getattr(plan.common, "trusted", False) is True
            and plan.route is self.route_type.DECODE
            and metadata.decode_wave_extra is not None
            and _has_cache(k_cache)
            and _has_cache(v_cache)
            and k is not None
            and v is not None
            and k.dim() == 3
            and k.size(0) == q.size(0)
            and k.size(0) * self.num_kv_heads <= ops.FUSED_STORE_MAX_ROWS
        ):
            self._pending_store = (k, v, slot_mapping)
            try:
                out = self.forward(q, k, v, k_cache, v_cache, plan)
            finally:
                self._pending_store = None
            if self.check_fused_store and self.fused_store_error():
                raise RuntimeError("fused KV store: a new row's slot is not its sequence's last position; "
                                   "the cache holds the row, but this step's attention did not see it there")
            return out
        (store if store is not None else ops.store_kvcache)(k, v, k_cache, v_cache, slot_mapping)
        return self.forward(q, k, v, k_cache, v_cache, plan)

    def forward(self, q, k, v, k_cache, v_cache, plan) -> torch.Tensor:
        metadata = plan_metadata(plan, MI355XAttentionMetadata, self.backend_name, self.plan_type)
        Route = self.route_type
        Batch = self.batch_type_enum
        has_k_cache = _has_cache(k_cache)
        has_v_cache = _has_cache(v_cache)
        if has_k_cache != has_v_cache:
            raise ValueError("key and value caches must both be present or absent")
        graph_state = self._active_graph_state
        if graph_state is not None:
            if not has_k_cache:
                raise RuntimeError("full decode graph requires allocated KV cache")
            self._validate_inputs(q, k_cache, v_cache)
            if graph_state.output.shape != q.shape:
                raise RuntimeError("decode graph attention output does not match query shape")
            self._run_decode_graph(q, k_cache, v_cache, graph_state)
            return graph_state.output
        route = plan.route
        if route is Route.WARMUP:
            if has_k_cache:
                raise ValueError("MI355X warmup route requires an empty KV cache")
            if not metadata.is_cacheless:
                raise ValueError("MI355X warmup route requires cacheless metadata")
            self._check_cacheless_inputs(q, k, v)
            output = self._get_reusable_attention_output(q)
            self._run_warmup(q, k, v, plan.common, output)
            return output

        expected = {
            Route.PREFILL: Batch.PURE_PREFILL,
            Route.DECODE: Batch.PURE_DECODE,
            Route.MIXED_UNIFIED: Batch.MIXED,
            Route.MIXED_SPLIT: Batch.MIXED,
        }.get(route)
        if expected is None:
            raise RuntimeError(f"invalid planned MI355X route: {route!r}")
        if plan.batch_type is not expected:
            raise ValueError("MI355X route does not match the planned BatchType")
        # The metadata fixes how a MIXED batch runs: a single launch's decode
        # plan has no merge list, a split plan's has.
        if expected is Batch.MIXED and (route is Route.MIXED_UNIFIED) != (metadata.mixed_prefill_max_tiles > 0):
            raise ValueError("MI355X MIXED route does not match the planned metadata")
        if not has_k_cache:
            raise ValueError("paged MI355X route requires an allocated KV cache")
        if metadata.is_cacheless:
            raise ValueError("paged MI355X route requires page metadata")
        self._validate_inputs(q, k_cache, v_cache)
        common = plan.common
        if q.size(0) != common.num_query_tokens:
            raise ValueError("query token count does not match the attention plan")

        output = self._get_reusable_attention_output(q)
        if route is Route.DECODE:
            self._run_decode(q, k_cache, v_cache, common, metadata, output)
            return output
        if route is Route.PREFILL:
            self._run_prefill(q, k_cache, v_cache, common, metadata, output)
            return output
        if route is Route.MIXED_SPLIT:
            if common.num_prefill_seqs:
                self._run_prefill(q, k_cache, v_cache, common, metadata, output)
            if common.num_decode_seqs:
                self._run_decode(q, k_cache, v_cache, common, metadata, output)
            return output
        self._run_mixed(q, k_cache, v_cache, common, metadata, output)
        return output

    def _run_decode(self, q, k_cache, v_cache, common, metadata: MI355XAttentionMetadata, output) -> None:
        group = self.num_q_heads // self.num_kv_heads
        ws_bytes = ops.decode_workspace_bytes(metadata.num_decode_part_slots, self.num_kv_heads, group)
        workspace = self._get_workspace(ws_bytes, q.device)
        if self._pending_store is not None:
            key, value, slot_mapping = self._pending_store
            ops.paged_decode_store(
                q, key, value, slot_mapping, k_cache, v_cache,
                metadata.block_tables, metadata.seq_lens,
                metadata.decode_items, metadata.num_decode_items, metadata.num_decode_waves,
                metadata.decode_merges, metadata.num_decode_merges, metadata.num_decode_part_slots,
                output, workspace, self.softmax_scale,
                metadata.decode_wave_extra, metadata.decode_waves_per_group, validate=False,
            )
            return
        ops.paged_decode(
            q,
            k_cache,
            v_cache,
            metadata.block_tables,
            metadata.seq_lens,
            metadata.decode_items,
            metadata.num_decode_items,
            metadata.num_decode_waves,
            metadata.decode_merges,
            metadata.num_decode_merges,
            metadata.num_decode_part_slots,
            output,
            workspace,
            self.softmax_scale,
            metadata.decode_wave_extra,
            metadata.decode_waves_per_group,
            validate=False,
        )

    def fused_store_error(self) -> bool:
        """Whether a folded decode store since the last call met a row whose
        slot was not its sequence's last position (written after the
        attention; reads the device and clears the word)."""
        if self._workspace is None:
            return False
        return ops.decode_store_error(self._workspace)

    def _run_decode_graph(self, q, k_cache, v_cache, state: MI355XFullDecodeGraphState) -> None:
        counts, items, wave_extra, merges = state.views()
        ops.paged_decode_graph(
            q, k_cache, v_cache, state.block_tables_buffer, state.seq_lens_buffer, counts, items, wave_extra,
            state.waves_per_group, merges, state.part_slot_capacity, state.output, state.workspace,
            self.softmax_scale, validate=False,
        )

    # ---- full-decode HIP graph (reference attention_backend.py:242-275, 1028-1225) ----
    def create_full_decode_graph_state(self, batch_size: int, page_indices_capacity: int, device):
        if isinstance(batch_size, bool) or not isinstance(batch_size, int):
            raise TypeError("batch_size must be an int")
        if isinstance(page_indices_capacity, bool) or not isinstance(page_indices_capacity, int):
            raise TypeError("page_indices_capacity must be an int")
        if batch_size <= 0 or page_indices_capacity < batch_size:
            raise ValueError("graph state requires positive batch and page capacity")
        graph_device = torch.device(device)
        if graph_device.type != "cuda":
            raise ValueError("full decode graph state must be on CUDA")
        groups, waves_per_group = listed_decode_groups(self.num_kv_heads, graph_device,
                                                       override=self.decode_waves_override)
        caps = graph_decode_capacities(batch_size, page_indices_capacity, self.num_kv_heads, groups)
        group = self.num_q_heads // self.num_kv_heads
        plan_ints = graph_plan_buffer_ints(caps["item_capacity"], caps["wave_capacity"], caps["merge_capacity"])
        ws_bytes = ops.decode_workspace_bytes(caps["part_slot_capacity"], self.num_kv_heads, group)
        width = max(1, page_indices_capacity // batch_size)
        return MI355XFullDecodeGraphState(
            batch_size=batch_size,
            page_indices_capacity=page_indices_capacity,
            groups=groups,
            waves_per_group=waves_per_group,
            block_tables_buffer=torch.zeros((batch_size, width), dtype=torch.int32, device=graph_device),
            seq_lens_buffer=torch.ones(batch_size, dtype=torch.int32, device=graph_device),
            plan_buffer=torch.zeros(plan_ints, dtype=torch.int32, device=graph_device),
            plan_staging=[torch.zeros(plan_ints, dtype=torch.int32, pin_memory=True) for _ in range(2)],
            staging_ready=[None, None],
            workspace=torch.zeros(ws_bytes, dtype=torch.uint8, device=graph_device),
            output=torch.empty(batch_size, self.num_q_heads, self.head_dim, dtype=self.dtype, device=graph_device),
            **caps,
        )

    def full_decode_graph_metadata_fits(self, state, plan) -> bool:
        if not isinstance(state, MI355XFullDecodeGraphState) or not isinstance(plan, self.plan_type):
            return False
        if plan.batch_type is not self.batch_type_enum.PURE_DECODE or plan.route is not self.route_type.DECODE:
            return False
        metadata = plan.metadata
        if not isinstance(metadata, MI355XAttentionMetadata) or metadata.is_cacheless:
            return False
        common = plan.common
        if common.num_prefill_seqs != 0 or common.num_prefill_tokens != 0:
            return False
        if common.num_decode_seqs != state.batch_size or common.num_decode_tokens != state.batch_size:
            return False
        bt = metadata.block_tables
        if (
            not isinstance(bt, torch.Tensor)
            or bt.dtype != torch.int32
            or bt.device.type != "cuda"
            or bt.ndim != 2
            or bt.size(0) != state.batch_size
            or bt.size(1) > state.block_tables_buffer.size(1)
        ):
            return False
        if metadata.num_pages > state.page_indices_capacity or metadata.num_prefill_pages != 0:
            return False
        for tensor in (metadata.seq_lens, common.slot_mapping):
            if (
                not isinstance(tensor, torch.Tensor)
                or tensor.dtype != torch.int32
                or tensor.device.type != "cuda"
                or tensor.ndim != 1
                or tensor.numel() != state.batch_size
            ):
                return False
        return True

    def plan_full_decode_graph(self, state, plan) -> None:
        if not self.full_decode_graph_metadata_fits(state, plan):
            raise ValueError("attention plan does not fit full decode graph state")
        metadata = plan.metadata
        host = metadata.decode_host_plan
        if host is None or host[3] != state.groups:
            counts = np.diff(np.asarray(metadata.kv_indptr, dtype=np.int64))
            items, wave_extra, _, _, merges = plan_decode_listed(counts, 0, 0, self.num_kv_heads, state.groups)
        else:
            items, wave_extra, merges, _ = host
        # Staging buffers alternate: the one refilled now was last copied two
        # steps ago, so the host waits only if it runs two steps ahead.
        k = state.staging_turn
        state.staging_turn ^= 1
        if state.staging_ready[k] is not None:
            state.staging_ready[k].synchronize()
        staging = state.plan_staging[k]
        pack_graph_decode_plan(items, wave_extra, merges, state.item_capacity, state.wave_capacity,
                               state.merge_capacity, staging.numpy())
        state.plan_buffer.copy_(staging, non_blocking=True)
        event = torch.cuda.Event()
        event.record(torch.cuda.current_stream(state.plan_buffer.device))
        state.staging_ready[k] = event
        bt = metadata.block_tables
        state.block_tables_buffer[:, : bt.size(1)].copy_(bt)
        state.seq_lens_buffer.copy_(metadata.seq_lens)
        state.plan = plan

    def activate_full_decode_graph(self, state) -> None:
        if not isinstance(state, MI355XFullDecodeGraphState):
            raise TypeError("invalid MI355X decode graph state")
        if state.plan is None:
            raise RuntimeError("decode graph state must be planned before activation")
        if self._active_graph_state is not None:
            raise RuntimeError("a decode graph state is already active")
        self._active_graph_state = state

    def deactivate_full_decode_graph(self) -> None:
        self._active_graph_state = None

    def _check_cacheless_inputs(self, q, k, v) -> None:
        # The reference's checks (attention_backend.py:1586-1600), then the
        # layout the store and prefill kernels take.
        if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
            raise ValueError("cacheless attention expects rank-3 Q/K/V")
        if k.shape != v.shape:
            raise ValueError("cacheless key and value shapes must match")
        if q.size(0) != k.size(0):
            raise ValueError("cacheless warmup requires matching query and KV token counts")
        if q.size(1) % k.size(1):
            raise ValueError("query head count must be divisible by KV head count")
        if q.shape[1:] != (self.num_q_heads, self.head_dim) or k.shape[1:] != (self.num_kv_heads, self.head_dim):
            raise ValueError("cacheless Q/K/V must have the backend's head counts and head_dim")
        for t in (q, k, v):
            if not t.is_cuda or t.dtype != self.dtype or t.stride(2) != 1:
                raise ValueError("cacheless Q/K/V must be CUDA tensors of the backend dtype, unit inner stride")

    def _run_warmup(self, q, k, v, common, output) -> None:
        """Cacheless causal varlen attention (the WARMUP route) on the gfx950
        kernels: the batch's K/V rows are stored into a temporary page pool
        with the slot_mapping store kernel, then the ragged prefill kernel
        runs with every sequence's keys equal to its queries.  Replaces the
        reference's per-sequence SDPA fallback (attention_backend.py:1556-1624),
        so memory profiling sees the serving kernels.  Like the reference, this
        one-time path reads the query offsets to the host."""
        device = q.device
        bounds = np.asarray(common.query_start_loc.cpu().tolist(), dtype=np.int64)
        q_lens = bounds[1:] - bounds[:-1]
        if q.size(0) == 0 or q_lens.size == 0:
            return
        if np.any(q_lens < 0) or bounds[0] != 0 or bounds[-1] != q.size(0):
            raise ValueError("cacheless query_start_loc must run from 0 to the token count")
        counts = np.maximum((q_lens + PAGE_SIZE - 1) // PAGE_SIZE, 1)
        first_page = np.cumsum(counts) - counts
        seq_of = np.repeat(np.arange(q_lens.size), q_lens)
        within = np.arange(q.size(0)) - np.repeat(bounds[:-1], q_lens)
        slots = (first_page[seq_of] + within // PAGE_SIZE) * PAGE_SIZE + within % PAGE_SIZE
        table = np.full((q_lens.size, int(counts.max())), -1, dtype=np.int64)
        for s_idx, (base, c) in enumerate(zip(first_page, counts)):
            table[s_idx, :c] = np.arange(base, base + c)
        host = np.concatenate([slots, table.reshape(-1), q_lens]).astype(np.int32)
        flat = self._staging.to_device(host, device)
        n_slot, n_table = slots.size, table.size
        slot_mapping = flat[:n_slot]
        block_tables = flat[n_slot:n_slot + n_table].view(table.shape)
        seq_lens = flat[n_slot + n_table:]
        pool = torch.empty((2, int(counts.sum()), PAGE_SIZE, self.num_kv_heads, self.head_dim), dtype=self.dtype,
                           device=device)
        ops.store_kvcache(k, v, pool[0], pool[1], slot_mapping)
        max_tiles = ops.prefill_max_tiles(q.size(0), q_lens.size, self.num_q_heads, self.num_kv_heads)
        ops.paged_prefill(q, pool[0], pool[1], block_tables, seq_lens, common.query_start_loc, q_lens.size,
                          max_tiles, self._get_prefill_workspace(max_tiles, device), output, self.softmax_scale)
        self._prefill_planned_for = None

    def _run_prefill(self, q, k_cache, v_cache, common, metadata: MI355XAttentionMetadata, output) -> None:
        # The tile plan depends on the batch only: the first launch for this
        # metadata builds it on the device, later layers stream it as it is
        # (the reference's FlashInfer wrapper plans once per step in build_plan,
        # nanovllm/layers/attention_backend.py:810-825, and runs per layer, :992-994).
        workspace = self._get_prefill_workspace(metadata.prefill_max_tiles, q.device)
        ops.paged_prefill(
            q,
            k_cache,
            v_cache,
            metadata.block_tables,
            metadata.seq_lens,
            metadata.query_start_loc,
            common.num_prefill_seqs,
            metadata.prefill_max_tiles,
            workspace,
            output,
            self.softmax_scale,
            planned=self._prefill_planned_for is metadata,
        )
        self._prefill_planned_for = metadata

    def _run_mixed(self, q, k_cache, v_cache, common, metadata: MI355XAttentionMetadata, output) -> None:
        group = self.num_q_heads // self.num_kv_heads
        ws_bytes = ops.decode_workspace_bytes(metadata.num_decode_part_slots, self.num_kv_heads, group)
        workspace = self._get_workspace(ws_bytes, q.device)
        ops.paged_mixed(
            q,
            k_cache,
            v_cache,
            metadata.block_tables,
            metadata.seq_lens,
            metadata.query_start_loc,
            common.num_prefill_seqs,
            metadata.mixed_prefill_max_tiles,
            metadata.decode_items,
            metadata.num_decode_items,
            metadata.num_decode_waves,
            metadata.num_decode_part_slots,
            output,
            workspace,
            self.softmax_scale,
        )


class MI355XAttentionBackend(MI355XAttentionBackendMixin, AttentionBackend):
    """gfx950 backend registered as ``"mi355x"`` (MIXED batches: one launch)."""


class MI355XSplitAttentionBackend(MI355XAttentionBackend):
    """Same kernels; MIXED batches run as prefill + decode launches ("mi355x_split")."""

    backend_name = "mi355x_split"
    default_attention_mode = "split"


def integrate(registry: Any, base: type, plan_type: type, route_type: type, batch_type_enum: type,
              common_type: type, names: tuple[str, str] = ("mi355x", "mi355x_split")) -> tuple[type, type]:
    """Build the backend on another contract's classes and register it.

    ``base`` is that contract's ``AttentionBackend`` (the reference's:
    nanovllm/layers/attention_backend.py:174-275) and the four types its
    plan, route, batch-type and metadata classes.  Two classes are
    registered under ``names``: MIXED batches in one launch, and MIXED as
    prefill + decode launches (the reference's registry passes
    ``attention_mode`` to FlashInfer only, attention_backend.py:1376-1381, so
    the mode is carried by the name).  Returns ``(unified, split)``.
    """
    family = {"plan_type": plan_type, "route_type": route_type, "batch_type_enum": batch_type_enum,
              "common_type": common_type}
    unified = type("MI355XBackend", (MI355XAttentionBackendMixin, base),
                   {"__module__": __name__, "backend_name": names[0], **family})
    split = type("MI355XSplitBackend", (unified,),
                 {"__module__": __name__, "backend_name": names[1], "default_attention_mode": "split"})
    registry.register(names[0], unified)
    registry.register(names[1], split)
    return unified, split


__all__ = [
    "MI355XAttentionBackend",
    "MI355XAttentionBackendMixin",
    "MI355XAttentionMetadata",
    "MI355XSplitAttentionBackend",
    "integrate",
    "make_decode_plan",
    "make_decode_plan_listed",
    "plan_decode_claims",
    "plan_decode_listed",
    "resident_decode_waves",
]
