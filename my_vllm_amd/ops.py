"""Validated Python entry points over the gfx950 C ABI.

Each function checks shapes, dtypes, devices and layout on the host, with the
reference's exception classes and messages, then launches the kernel on
torch's current stream.  None of them synchronizes or reads device memory.
"""

from __future__ import annotations

import torch

from . import _native

HEAD_DIM = 128
PAGE_SIZE = 16
# int32 fields per decode work item (kDecodeItemInts in csrc/paged_decode.h).
DECODE_ITEM_INTS = 8
# Longest piece one decode work item may cover (kMaxChunkPages).
MAX_CHUNK_PAGES = 128
# Query rows per prefill workgroup (kPrefillRows): G heads x 128 // G tokens.
PREFILL_ROWS = 128
# Query rows per tile of mva_paged_prefill's kernel (the MIXED kernel's
# prefill tiles have PREFILL_ROWS).
PREFILL_STREAM_ROWS = 256
# Device-built prefill tile list: header ints (tile count + per-head claim
# counters) and ints per tile record (kPrefillPlanHeaderInts / ItemInts).
PREFILL_PLAN_HEADER_INTS = 32 * 128
PREFILL_PLAN_ITEM_INTS = 16


def silu_and_mul(x: torch.Tensor) -> torch.Tensor:
    """``silu(x[..., :I]) * x[..., I:]`` into a new contiguous ``[..., I]`` tensor.

    Argument checks and messages follow the reference's compiled op
    (csrc/silu_and_mul.cpp:8-18); an empty input gives an empty output
    (csrc/silu_and_mul_kernel.cu:61-63).
    """
    if not x.is_cuda:
        raise RuntimeError("silu_and_mul expects a CUDA tensor")
    if not x.is_contiguous():
        raise RuntimeError("silu_and_mul expects a contiguous tensor")
    if x.dim() < 1:
        raise RuntimeError("silu_and_mul expects at least one dimension")
    if x.dtype not in _native.DTYPE_CODES:
        raise RuntimeError("silu_and_mul only supports float16 and bfloat16")
    width = x.size(-1)
    if width <= 0 or width % 2:
        raise RuntimeError(
            "silu_and_mul expects the last dimension to be a positive even number"
        )
    hidden = width // 2
    out = torch.empty((*x.shape[:-1], hidden), dtype=x.dtype, device=x.device)
    if out.numel() == 0:
        return out
    rows = x.numel() // width
    _native.call(
        "mva_silu_and_mul",
        x.data_ptr(),
        out.data_ptr(),
        rows,
        hidden,
        _native.dtype_code(x.dtype),
        _native.stream_handle(x.device),
    )
    return out


def _check_rows(name: str, x: torch.Tensor, hidden: int) -> None:
    if not x.is_cuda:
        raise RuntimeError(f"{name} expects a CUDA tensor")
    if x.dtype not in _native.DTYPE_CODES:
        raise RuntimeError(f"{name} only supports float16 and bfloat16")
    if x.dim() < 1 or x.size(-1) != hidden or (x.numel() and x.stride(-1) != 1):
        raise RuntimeError(f"{name} expects rows of {hidden} elements with unit stride")


def _rows_view(x: torch.Tensor) -> tuple[int, int]:
    """(rows, row stride) of ``x`` seen as ``[-1, hidden]`` without copying."""
    if x.dim() == 1:
        return 1, x.size(0)
    flat = x.reshape(-1, x.size(-1))
    if flat.data_ptr() != x.data_ptr() or (flat.size(0) > 1 and flat.stride(1) != 1):
        raise RuntimeError("rms_norm expects rows addressable with one row stride")
    return flat.size(0), flat.stride(0) if flat.size(0) > 1 else x.size(-1)


def _grouped_rows(x: torch.Tensor) -> tuple[int, int, int, int]:
    """(groups, rows per group, group stride, row stride) of ``x`` as
    ``[G, R, hidden]`` without copying: a 2-D (or mergeable) tensor is one row
    per group; ``[tokens, heads, hidden]`` views of a packed projection keep
    their token and head strides."""
    if x.dim() <= 2:
        rows, stride = _rows_view(x)
        return rows, 1, stride, stride
    lead = x.reshape(-1, x.size(-2), x.size(-1)) if x.dim() > 3 else x
    if lead.data_ptr() != x.data_ptr() or (lead.numel() and lead.stride(2) != 1):
        raise RuntimeError("rms_norm expects [..., rows, hidden] with unit inner stride")
    return lead.size(0), lead.size(1), lead.stride(0), lead.stride(1)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """RMSNorm of the last dimension (reference nanovllm/layers/layernorm.py:31-40).

    ``x`` may be a strided view such as the ``[tokens, heads, head_dim]`` query
    slice of a packed qkv projection (the reference's q_norm input); the
    result is a new contiguous tensor unless ``out`` is given.
    """
    hidden = weight.numel()
    _check_rows("rms_norm", x, hidden)
    if weight.dtype not in (x.dtype, torch.float32) or not weight.is_contiguous() or weight.device != x.device:
        raise RuntimeError("rms_norm weight must be contiguous fp32 or the input dtype on the input device")
    if out is None:
        out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    if out.shape != x.shape:
        raise RuntimeError("rms_norm output must have the input shape")
    if x.numel() == 0:
        return out
    groups, per_group, x_gs, x_rs = _grouped_rows(x)
    o_groups, o_per_group, o_gs, o_rs = _grouped_rows(out)
    if (o_groups, o_per_group) != (groups, per_group):
        raise RuntimeError("rms_norm output rows must match the input rows")
    _native.call(
        "mva_rms_norm", x.data_ptr(), x_gs, x_rs, weight.data_ptr(), out.data_ptr(), o_gs, o_rs,
        groups * per_group, per_group, hidden, float(eps), _native.dtype_code(x.dtype),
        _native.WEIGHT_DTYPE_CODES[weight.dtype], _native.stream_handle(x.device),
    )
    return out


def fused_add_rms_norm(
    x: torch.Tensor,
    residual: torch.Tensor,
    weight: torch.Tensor,
    eps: float,
    inplace: bool = False,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(rms_norm(x + residual), x + residual)`` (reference layernorm.py:42-52);
    ``inplace`` writes them into ``x`` and ``residual``."""
    hidden = weight.numel()
    _check_rows("fused_add_rms_norm", x, hidden)
    if residual.shape != x.shape or residual.dtype != x.dtype or residual.device != x.device:
        raise RuntimeError("fused_add_rms_norm expects residual with the shape and dtype of x")
    if weight.dtype not in (x.dtype, torch.float32) or not weight.is_contiguous() or weight.device != x.device:
        raise RuntimeError("rms_norm weight must be contiguous fp32 or the input dtype on the input device")
    if inplace:
        out, res_out = x, residual
    else:
        out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        res_out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    if x.numel() == 0:
        return out, res_out
    rows, x_stride = _rows_view(x)
    _, r_stride = _rows_view(residual)
    _, o_stride = _rows_view(out)
    _, ro_stride = _rows_view(res_out)
    _native.call(
        "mva_fused_add_rms_norm", x.data_ptr(), x_stride, residual.data_ptr(), r_stride, weight.data_ptr(),
        out.data_ptr(), o_stride, res_out.data_ptr(), ro_stride, rows, hidden, float(eps),
        _native.dtype_code(x.dtype), _native.WEIGHT_DTYPE_CODES[weight.dtype], _native.stream_handle(x.device),
    )
    return out, res_out


def _check_heads(name: str, t: torch.Tensor, dtype: torch.dtype, device: torch.device) -> None:
    if t.dim() != 3 or t.size(2) != HEAD_DIM or t.stride(2) != 1:
        raise ValueError(f"{name} must be [tokens, heads, {HEAD_DIM}] with unit inner stride")
    if t.dtype != dtype or t.device != device:
        raise ValueError(f"{name} must share the query dtype and device")


def qk_norm_rope_store(
    positions: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    q_norm_weight: torch.Tensor | None = None,
    k_norm_weight: torch.Tensor | None = None,
    eps: float = 1e-6,
    v: torch.Tensor | None = None,
    k_cache: torch.Tensor | None = None,
    v_cache: torch.Tensor | None = None,
    slot_mapping: torch.Tensor | None = None,
    q_out: torch.Tensor | None = None,
    k_out: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-head q/k RMSNorm (when weights are given), neox RoPE and, when a
    cache is given, the slot_mapping store of the rotated k and of v, in one
    launch.  The reference runs these as separate ops
    (nanovllm/models/qwen3.py:96-100, nanovllm/layers/attention.py:140-141).

    ``q``/``k``/``v`` are ``[T, heads, 128]`` views (a packed qkv projection
    works); outputs default to writing ``q`` and ``k`` in place.
    ``cos_sin_cache`` is the RotaryEmbedding buffer, ``[max_pos, (1,) 128]``
    fp32 (cos | sin); ``positions`` int64 ``[T]``.  Returns ``(q_out, k_out)``.
    """
    if not q.is_cuda:
        raise RuntimeError("qk_norm_rope_store expects CUDA tensors")
    dtype, device = q.dtype, q.device
    _check_heads("query", q, dtype, device)
    _check_heads("key", k, dtype, device)
    num_tokens = q.size(0)
    if k.size(0) != num_tokens or positions.shape != (num_tokens,) or positions.dtype != torch.int64:
        raise ValueError("positions must be int64 [tokens] and key must have the query's token count")
    if positions.device != device:
        raise ValueError("positions must be on the query device")
    if not positions.is_contiguous():
        positions = positions.contiguous()  # the kernel indexes it densely
    table = cos_sin_cache.reshape(cos_sin_cache.size(0), -1)
    if table.dtype != torch.float32 or table.size(1) != HEAD_DIM or not table.is_contiguous() or table.device != device:
        raise ValueError(f"cos_sin_cache must be contiguous fp32 [max_position, {HEAD_DIM}] on the query device")
    q_out = q if q_out is None else q_out
    k_out = k if k_out is None else k_out
    if q_out.shape != q.shape or q_out.stride() != q.stride() or k_out.shape != k.shape or k_out.stride() != k.stride():
        raise ValueError("outputs must match the inputs' shape and strides")
    weight_code = 0
    if (q_norm_weight is None) != (k_norm_weight is None):
        raise ValueError("give both q and k norm weights or neither")
    if q_norm_weight is not None:
        for w in (q_norm_weight, k_norm_weight):
            if w.numel() != HEAD_DIM or not w.is_contiguous() or w.device != device or w.dtype not in (dtype, torch.float32):
                raise ValueError(f"norm weights must be contiguous [{HEAD_DIM}] fp32 or the query dtype")
        if q_norm_weight.dtype != k_norm_weight.dtype:
            raise ValueError("q and k norm weights must share a dtype")
        weight_code = _native.WEIGHT_DTYPE_CODES[q_norm_weight.dtype]
    store = k_cache is not None
    if store:
        if v is None or v_cache is None or slot_mapping is None:
            raise ValueError("the KV store needs v, v_cache and slot_mapping")
        _check_heads("value", v, dtype, device)
        num_kv = k.size(1)
        for cache in (k_cache, v_cache):
            if (cache.dtype != dtype or cache.device != device or cache.dim() != 4 or cache.size(2) != num_kv
                    or cache.size(3) != HEAD_DIM or not cache.is_contiguous()):
                raise ValueError("caches must be contiguous [pages, page, num_kv_heads, 128] in the query dtype")
        if slot_mapping.dtype not in (torch.int32, torch.int64) or slot_mapping.numel() != num_tokens:
            raise ValueError("slot_mapping must be int32/int64 with one slot per token")
        if slot_mapping.device != device:
            raise ValueError("slot_mapping must be on the query device")
        if slot_mapping.dim() != 1 or not slot_mapping.is_contiguous():
            slot_mapping = slot_mapping.reshape(-1).contiguous()  # the kernel indexes it densely
    if num_tokens == 0:
        return q_out, k_out
    _native.call(
        "mva_qk_norm_rope_store",
        q.data_ptr(), q_out.data_ptr(), q.stride(0), q.stride(1), q.size(1),
        k.data_ptr(), k_out.data_ptr(), k.stride(0), k.stride(1),
        v.data_ptr() if store else 0, v.stride(0) if store else 0, v.stride(1) if store else 0, k.size(1),
        positions.data_ptr(), table.data_ptr(), table.size(0), HEAD_DIM,
        q_norm_weight.data_ptr() if q_norm_weight is not None else 0,
        k_norm_weight.data_ptr() if k_norm_weight is not None else 0, weight_code, float(eps),
        k_cache.data_ptr() if store else 0, v_cache.data_ptr() if store else 0,
        k_cache.size(0) * k_cache.size(1) if store else 0,
        slot_mapping.data_ptr() if store else 0, int(store and slot_mapping.dtype == torch.int64),
        num_tokens, HEAD_DIM, _native.dtype_code(dtype), _native.stream_handle(device),
    )
    return q_out, k_out


def rotary_embedding(positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor, cos_sin_cache: torch.Tensor,
                     head_size: int = HEAD_DIM) -> tuple[torch.Tensor, torch.Tensor]:
    """Neox RoPE into new tensors (nanovllm/layers/rotary_embedding.py:41-51);
    ``query``/``key`` are ``[T, heads * head_size]`` or ``[T, heads, head_size]``."""
    if head_size != HEAD_DIM:
        raise ValueError(f"rotary embedding supports head_size {HEAD_DIM}")
    q3 = query.view(query.size(0), -1, HEAD_DIM)
    k3 = key.view(key.size(0), -1, HEAD_DIM)
    q_out = torch.empty_like(q3)
    k_out = torch.empty_like(k3)
    if q_out.stride() != q3.stride() or k_out.stride() != k3.stride():
        q3, k3 = q3.contiguous(), k3.contiguous()
    qk_norm_rope_store(positions, q3, k3, cos_sin_cache, q_out=q_out, k_out=k_out)
    return q_out.view(query.shape), k_out.view(key.shape)


def store_kvcache(
    key: torch.Tensor,
    value: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
) -> None:
    """Scatter K/V rows into the paged cache by ``slot_mapping`` (``< 0`` = skip).

    Layout contract of the reference's store (nanovllm/layers/attention.py:34-41):
    ``key``/``value`` are ``[N, Hkv, D]`` with unit element stride and head
    stride ``D`` (the token stride is free: V is a view into a packed qkv
    projection); the caches are contiguous ``[P, page, Hkv, D]``.
    """
    if key.dim() != 3 or value.shape != key.shape:
        raise ValueError("key and value must both have shape [tokens, num_kv_heads, head_dim]")
    num_tokens, num_heads, head_dim = key.shape
    row_elems = num_heads * head_dim
    if slot_mapping.numel() != num_tokens:
        raise ValueError("slot_mapping must contain one slot per token")
    if slot_mapping.dtype not in (torch.int32, torch.int64):
        raise TypeError("slot_mapping must be int32 or int64")
    if key.stride(-1) != 1 or value.stride(-1) != 1:
        raise ValueError("key/value must have unit stride in the head dimension")
    if key.stride(1) != head_dim or value.stride(1) != head_dim:
        raise ValueError("key/value heads must be packed (stride(1) == head_dim)")
    for name, cache in (("k_cache", k_cache), ("v_cache", v_cache)):
        if not cache.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
        if cache.dtype != key.dtype:
            raise TypeError(f"{name} dtype {cache.dtype} does not match key dtype {key.dtype}")
        if cache.numel() % row_elems or (cache.dim() >= 2 and cache.stride(1) != row_elems):
            raise ValueError(f"{name} rows must hold num_kv_heads * head_dim elements")
        if cache.device != key.device:
            raise ValueError(f"{name} must be on the key's device")
    if v_cache.shape != k_cache.shape:
        raise ValueError("k_cache and v_cache shapes differ")
    if value.dtype != key.dtype:
        raise TypeError("key and value dtypes differ")
    if not key.is_cuda or not slot_mapping.is_cuda or slot_mapping.device != key.device:
        raise RuntimeError("store_kvcache expects CUDA tensors on one device")
    if slot_mapping.dim() != 1 or not slot_mapping.is_contiguous():
        slot_mapping = slot_mapping.reshape(-1).contiguous()  # the kernel indexes it densely
    if num_tokens == 0:
        return
    _native.call(
        "mva_kv_store",
        key.data_ptr(),
        key.stride(0),
        value.data_ptr(),
        value.stride(0),
        k_cache.data_ptr(),
        v_cache.data_ptr(),
        k_cache.numel() // row_elems,
        slot_mapping.data_ptr(),
        1 if slot_mapping.dtype == torch.int64 else 0,
        num_tokens,
        row_elems,
        _native.dtype_code(key.dtype),
        _native.stream_handle(key.device),
    )


def decode_workspace_bytes(num_part_slots: int, num_kv_heads: int, group: int) -> int:
    """Workspace bytes of a decode (or MIXED) launch with ``num_part_slots`` split-K slots."""
    nbytes = int(_native.query("mva_decode_workspace_bytes", num_part_slots, num_kv_heads, group))
    if nbytes < 0:
        raise ValueError("invalid decode workspace arguments")
    return nbytes


# Byte offset of the fused store's error word in a decode workspace
# (MVA_DECODE_STORE_ERROR_OFFSET in include/my_vllm_amd.h).
DECODE_STORE_ERROR_OFFSET = 4224


# (token, KV head) rows a fused store launch takes (its per-row flags).
FUSED_STORE_MAX_ROWS = 65536


def decode_store_error(workspace: torch.Tensor, clear: bool = True) -> bool:
    """Whether a :func:`paged_decode_store` launch on ``workspace`` met a row
    whose slot is not its sequence's last position (the row was written after
    the attention read the cache).  Reads the device, so it synchronizes with
    the stream; ``clear`` resets the word."""
    word = workspace[DECODE_STORE_ERROR_OFFSET:DECODE_STORE_ERROR_OFFSET + 4].view(torch.int32)
    flagged = bool(word.item() != 0)
    if flagged and clear:
        word.zero_()
    return flagged


def decode_merge_list(items):
    """The merge entries of a decode plan: chunk 0 of every split segment.

    ``items`` is the int32 ``[n, 8]`` piece array (numpy); the result has the
    same format and lists each (sequence, KV head) cut into more than one
    piece exactly once.
    """
    return items[(items[:, 3] == 0) & (items[:, 4] > 1)]


def paged_decode(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    items: torch.Tensor,
    num_items: int,
    num_waves: int,
    merges: torch.Tensor | None,
    num_merges: int,
    num_part_slots: int,
    out: torch.Tensor,
    workspace: torch.Tensor | None,
    softmax_scale: float,
    wave_extra: torch.Tensor | None = None,
    waves_per_group: int = 1,
    *,
    validate: bool = True,
) -> None:
    """Launch the paged GQA decode kernel over prepared pieces.

    ``q``/``out`` are ``[T, Hq, D]`` views (rows addressed by the pieces'
    ``q_row``); caches ``[P, page, Hkv, D]``; ``items`` int32 ``[n, 8]``,
    run by ``num_waves`` (``1 <= num_waves <= n``) wavefronts, ``waves_per_group``
    to a workgroup.  With ``wave_extra`` (int32 ``[num_waves + 1]``) wavefront
    ``w`` runs piece ``w`` and then pieces ``wave_extra[w]:wave_extra[w + 1]``;
    without it, wavefronts claim pieces from workspace counters.
    ``merges`` (see :func:`decode_merge_list`) lists the split segments whose
    partials the follow-up merge kernel combines.
    """
    if validate:
        _check_paged(q, out, k_cache, v_cache,
                     (("block_tables", block_tables), ("seq_lens", seq_lens), ("items", items),
                      ("merges", merges), ("wave_extra", wave_extra)), (("workspace", workspace),))
    num_q_heads, head_dim = q.shape[1], q.shape[2]
    num_pages, page_size, num_kv_heads = k_cache.shape[0], k_cache.shape[1], k_cache.shape[2]
    ws_ptr = workspace.data_ptr() if workspace is not None else 0
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _native.call(
        "mva_paged_decode",
        q.data_ptr(), q.stride(0), q.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(), num_pages, k_cache.stride(0), k_cache.stride(1),
        block_tables.data_ptr(), block_tables.stride(0), seq_lens.data_ptr(),
        items.data_ptr(), num_items, num_waves,
        wave_extra.data_ptr() if wave_extra is not None else 0, int(waves_per_group),
        merges.data_ptr() if merges is not None else 0, num_merges, num_part_slots,
        out.data_ptr(), out.stride(0), out.stride(1),
        ws_ptr, ws_bytes,
        num_q_heads, num_kv_heads, head_dim, page_size, float(softmax_scale),
        _native.dtype_code(q.dtype), _native.stream_handle(q.device),
    )


def paged_decode_store(
    q: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    items: torch.Tensor,
    num_items: int,
    num_waves: int,
    merges: torch.Tensor | None,
    num_merges: int,
    num_part_slots: int,
    out: torch.Tensor,
    workspace: torch.Tensor | None,
    softmax_scale: float,
    wave_extra: torch.Tensor,
    waves_per_group: int = 1,
    *,
    validate: bool = True,
) -> None:
    """:func:`store_kvcache` of this step's ``key``/``value`` and :func:`paged_decode`
    in one launch (piece lists only).

    A new row whose slot is its sequence's last position lies in the last
    page, which only one piece per KV head reads; that piece's wavefront
    writes the row before reading any page.  Any other row with a slot >= 0
    (a slot elsewhere, or a row no piece names) is written by the merge
    kernel that always follows, after the attention has read the cache, and
    sets the workspace word at :data:`DECODE_STORE_ERROR_OFFSET` (see
    :func:`decode_store_error`).  So the caches always end as
    :func:`store_kvcache` leaves them.  At most :data:`FUSED_STORE_MAX_ROWS`
    (token, KV head) rows.  ``key``/``value`` are ``[T, Hkv, D]`` with unit
    inner stride; ``slot_mapping`` int32/int64 ``[T]`` (``< 0`` = skip).
    """
    if validate:
        _check_paged(q, out, k_cache, v_cache,
                     (("block_tables", block_tables), ("seq_lens", seq_lens), ("items", items),
                      ("merges", merges), ("wave_extra", wave_extra)), (("workspace", workspace),))
    num_q_heads, head_dim = q.shape[1], q.shape[2]
    num_pages, page_size, num_kv_heads = k_cache.shape[0], k_cache.shape[1], k_cache.shape[2]
    num_tokens = key.shape[0]
    # The kernel dereferences these pointers: they must be device memory on
    # the query's GPU (as store_kvcache requires).
    for name, t in (("key", key), ("value", value), ("slot_mapping", slot_mapping)):
        if not t.is_cuda or t.device != q.device:
            raise RuntimeError(f"paged_decode_store expects {name} as a CUDA tensor on the query's device")
    if key.shape != value.shape or key.dim() != 3 or key.shape[1:] != (num_kv_heads, head_dim):
        raise ValueError("key and value must be [T, num_kv_heads, head_dim]")
    if key.dtype != q.dtype or value.dtype != q.dtype:
        raise TypeError("key and value must have the query dtype")
    if key.stride(-1) != 1 or value.stride(-1) != 1:
        raise ValueError("key and value need unit stride in the last dimension")
    if slot_mapping.numel() != num_tokens or slot_mapping.dtype not in (torch.int32, torch.int64):
        raise ValueError("slot_mapping must be int32/int64 with one slot per token")
    if slot_mapping.dim() != 1 or not slot_mapping.is_contiguous():
        slot_mapping = slot_mapping.reshape(-1).contiguous()  # the kernel indexes it densely
    ws_ptr = workspace.data_ptr() if workspace is not None else 0
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _native.call(
        "mva_paged_decode_store",
        q.data_ptr(), q.stride(0), q.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(), num_pages, k_cache.stride(0), k_cache.stride(1),
        block_tables.data_ptr(), block_tables.stride(0), seq_lens.data_ptr(),
        items.data_ptr(), num_items, num_waves,
        wave_extra.data_ptr(), int(waves_per_group),
        merges.data_ptr() if merges is not None else 0, num_merges, num_part_slots,
        out.data_ptr(), out.stride(0), out.stride(1),
        ws_ptr, ws_bytes,
        key.data_ptr(), key.stride(0), key.stride(1),
        value.data_ptr(), value.stride(0), value.stride(1),
        slot_mapping.data_ptr(), 1 if slot_mapping.dtype == torch.int64 else 0, num_tokens,
        num_q_heads, num_kv_heads, head_dim, page_size, float(softmax_scale),
        _native.dtype_code(q.dtype), _native.stream_handle(q.device),
    )


def paged_decode_graph(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    counts: torch.Tensor,
    items: torch.Tensor,
    wave_extra: torch.Tensor,
    waves_per_group: int,
    merges: torch.Tensor,
    num_part_slots: int,
    out: torch.Tensor,
    workspace: torch.Tensor,
    softmax_scale: float,
    *,
    validate: bool = True,
) -> None:
    """Fixed-shape decode launch for HIP graph capture.

    ``counts`` (int32 ``[3]`` on the device) holds this step's
    ``{num_items, num_waves, num_merges}``; ``items`` ``[item_capacity, 8]``,
    ``wave_extra`` ``[wave_capacity + 1]`` and ``merges`` ``[merge_capacity, 8]``
    hold the piece-list plan.  Grids are sized by the capacities, so every
    pointer and size stays fixed from one step to the next.
    """
    if min(counts.numel(), 3) != 3 or wave_extra.numel() < 2:
        raise ValueError("graph decode needs 3 counts and at least one wavefront")
    if validate:
        _check_paged(q, out, k_cache, v_cache,
                     (("block_tables", block_tables), ("seq_lens", seq_lens), ("counts", counts), ("items", items),
                      ("wave_extra", wave_extra), ("merges", merges)), (("workspace", workspace),))
    num_q_heads, head_dim = q.shape[1], q.shape[2]
    num_pages, page_size, num_kv_heads = k_cache.shape[0], k_cache.shape[1], k_cache.shape[2]
    _native.call(
        "mva_paged_decode_graph",
        q.data_ptr(), q.stride(0), q.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(), num_pages, k_cache.stride(0), k_cache.stride(1),
        block_tables.data_ptr(), block_tables.stride(0), seq_lens.data_ptr(),
        counts.data_ptr(),
        items.data_ptr(), items.shape[0], wave_extra.data_ptr(), wave_extra.numel() - 1, int(waves_per_group),
        merges.data_ptr(), merges.shape[0], num_part_slots,
        out.data_ptr(), out.stride(0), out.stride(1),
        workspace.data_ptr(), workspace.numel() * workspace.element_size(),
        num_q_heads, num_kv_heads, head_dim, page_size, float(softmax_scale),
        _native.dtype_code(q.dtype), _native.stream_handle(q.device),
    )


def _check_paged(q, out, k_cache, v_cache, int32_arrays=(), buffers=()) -> None:
    """The checks the C ABI cannot make: every pointer it gets is device memory
    on the query's GPU, the metadata arrays are int32 and dense (the block
    table's rows may be strided: its row stride crosses the ABI), and the V
    cache has the K cache's shape and strides (only the K strides cross the
    ABI).  Shapes, alignment and head counts are checked there.  The attention
    backend, which checks the query and caches itself on every forward and
    builds the work lists, calls the ops with ``validate=False``: on a
    launch-bound decode step these checks are a visible share of the host
    time."""
    device = q.device
    if not q.is_cuda:
        raise RuntimeError("paged attention expects CUDA tensors")
    for name, t in (("out", out), ("k_cache", k_cache), ("v_cache", v_cache)):
        if t.device != device:
            raise RuntimeError(f"paged attention: {name} must be on the query's device")
        if t.dtype != q.dtype:
            raise TypeError(f"paged attention: {name} must have the query dtype")
    if v_cache.shape != k_cache.shape or v_cache.stride() != k_cache.stride() or k_cache.dim() != 4:
        raise ValueError("paged attention: k_cache and v_cache must be [pages, page, Hkv, D] of one layout")
    if k_cache.stride(3) != 1 or k_cache.stride(2) != k_cache.size(3):
        raise ValueError("paged attention: cache rows must be packed heads of unit-stride elements")
    for name, t in int32_arrays:
        if t is None:
            continue
        dense = t.stride(-1) == 1 if name == "block_tables" else t.is_contiguous()
        if t.device != device or t.dtype != torch.int32 or not dense:
            raise ValueError(f"paged attention: {name} must be a dense int32 CUDA tensor on the query's device")
    for name, t in buffers:
        if t is not None and (t.device != device or not t.is_contiguous()):
            raise ValueError(f"paged attention: {name} must be a contiguous CUDA tensor on the query's device")


def _paged_args(q, k_cache, v_cache, block_tables, seq_lens):
    return (
        q.data_ptr(), q.stride(0), q.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.shape[0], k_cache.stride(0), k_cache.stride(1),
        block_tables.data_ptr(), block_tables.stride(0), seq_lens.data_ptr(),
    )


def _tail_args(q, k_cache, softmax_scale):
    return (
        q.shape[1], k_cache.shape[2], q.shape[2], k_cache.shape[1], float(softmax_scale),
        _native.dtype_code(q.dtype), _native.stream_handle(q.device),
    )


def prefill_max_tiles(num_prefill_tokens: int, num_prefill_seqs: int, num_q_heads: int, num_kv_heads: int) -> int:
    """Bound on the query tiles of a prefill batch: sum(ceil(q_s / tile)) <=
    tokens // tile + sequences."""
    tile = PREFILL_STREAM_ROWS // (num_q_heads // num_kv_heads)
    return num_prefill_tokens // tile + num_prefill_seqs


def mixed_prefill_max_tiles(num_prefill_tokens: int, num_prefill_seqs: int, num_q_heads: int,
                            num_kv_heads: int) -> int:
    """Bound on the 128-row query tiles of a MIXED launch's prefill part."""
    tile = PREFILL_ROWS // (num_q_heads // num_kv_heads)
    return num_prefill_tokens // tile + num_prefill_seqs


# Prefill sequences and KV heads one MIXED launch takes (kMixedPrefillSeqsMax,
# kMixedPrefillMaxHeads); larger MIXED batches run as prefill + decode.
MIXED_PREFILL_SEQS_MAX = 1024
MIXED_MAX_KV_HEADS = 64
# Split-K (partial slot, KV head) pairs one MIXED launch merges
# (kArrivalCounters).
MIXED_ARRIVAL_COUNTERS = 65536


def prefill_workspace_bytes(max_tiles: int) -> int:
    nbytes = int(_native.query("mva_prefill_workspace_bytes", max_tiles))
    if nbytes < 0:
        raise ValueError("invalid prefill tile capacity")
    return nbytes


# Byte offset of the prefill plan's dropped-tile count in a prefill workspace
# (MVA_PREFILL_DROPPED_TILES_OFFSET in include/my_vllm_amd.h).
PREFILL_DROPPED_TILES_OFFSET = 4


def prefill_dropped_tiles(workspace: torch.Tensor) -> int:
    """Tiles of the last :func:`paged_prefill` launch on ``workspace`` beyond
    its ``max_tiles`` (not run; 0 when the bound held).  Reads the device, so
    it synchronizes with the stream."""
    off = PREFILL_DROPPED_TILES_OFFSET
    return int(workspace[off:off + 4].view(torch.int32).item())


def paged_prefill(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    query_start_loc: torch.Tensor,
    num_seqs: int,
    max_tiles: int,
    workspace: torch.Tensor,
    out: torch.Tensor,
    softmax_scale: float,
    *,
    validate: bool = True,
    planned: bool = False,
) -> None:
    """Launch the ragged causal prefill over the first ``num_seqs`` sequences.

    The query tiles are planned on the device from ``query_start_loc`` and
    ``seq_lens`` into ``workspace`` (at least
    ``prefill_workspace_bytes(max_tiles)`` bytes); ``max_tiles`` must bound
    the tile count (see :func:`prefill_max_tiles`): tiles beyond it are not
    run and counted at :data:`PREFILL_DROPPED_TILES_OFFSET`
    (:func:`prefill_dropped_tiles`).  With ``planned=True`` the launch
    streams the plan that :func:`paged_prefill_plan` (or an earlier launch)
    left in ``workspace`` for the same batch metadata, and plans nothing.
    """
    if validate:
        _check_paged(q, out, k_cache, v_cache,
                     (("block_tables", block_tables), ("seq_lens", seq_lens), ("query_start_loc", query_start_loc)),
                     (("workspace", workspace),))
    _native.call(
        "mva_paged_prefill_run" if planned else "mva_paged_prefill",
        *_paged_args(q, k_cache, v_cache, block_tables, seq_lens),
        query_start_loc.data_ptr(), int(num_seqs), int(max_tiles),
        workspace.data_ptr(), workspace.numel() * workspace.element_size(),
        out.data_ptr(), out.stride(0), out.stride(1),
        *_tail_args(q, k_cache, softmax_scale),
    )


def paged_prefill_plan(
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    query_start_loc: torch.Tensor,
    num_seqs: int,
    max_tiles: int,
    workspace: torch.Tensor,
    num_pages: int,
    num_q_heads: int,
    num_kv_heads: int,
) -> None:
    """Build the tile list of a prefill batch into ``workspace`` on the
    current stream of the workspace's device, once for the layers of a step;
    each layer then calls :func:`paged_prefill` with ``planned=True``.  Plans
    and launches on one workspace must not overlap."""
    for name, t in (("block_tables", block_tables), ("seq_lens", seq_lens), ("query_start_loc", query_start_loc)):
        if t.device != workspace.device or t.dtype != torch.int32:
            raise RuntimeError(f"{name} must be an int32 tensor on the workspace's device")
    if seq_lens.stride(0) != 1 or query_start_loc.stride(0) != 1 or block_tables.stride(1) != 1:
        raise RuntimeError("seq_lens, query_start_loc and block table rows must be dense")
    _native.call(
        "mva_paged_prefill_plan",
        block_tables.data_ptr(), block_tables.stride(0), int(num_pages),
        seq_lens.data_ptr(), query_start_loc.data_ptr(), int(num_seqs), int(max_tiles),
        workspace.data_ptr(), workspace.numel() * workspace.element_size(),
        int(num_q_heads), int(num_kv_heads), _native.stream_handle(workspace.device),
    )


def paged_mixed(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    query_start_loc: torch.Tensor,
    num_prefill_seqs: int,
    max_prefill_tiles: int,
    decode_items: torch.Tensor | None,
    num_decode_items: int,
    num_decode_waves: int,
    num_part_slots: int,
    out: torch.Tensor,
    workspace: torch.Tensor,
    softmax_scale: float,
    *,
    validate: bool = True,
) -> None:
    """One launch: prefill tiles write ``out[:P]``, decode pieces write ``out[P:]``.

    The prefill tiles of the leading ``num_prefill_seqs`` sequences are
    derived on the device; ``max_prefill_tiles`` bounds them (see
    :func:`mixed_prefill_max_tiles`).  Split decode segments are merged
    inside the launch (no merge list).  ``workspace`` is the decode
    workspace.
    """
    if validate:
        _check_paged(q, out, k_cache, v_cache,
                     (("block_tables", block_tables), ("seq_lens", seq_lens), ("query_start_loc", query_start_loc),
                      ("decode_items", decode_items)), (("workspace", workspace),))
    _native.call(
        "mva_paged_mixed",
        *_paged_args(q, k_cache, v_cache, block_tables, seq_lens),
        query_start_loc.data_ptr(), int(num_prefill_seqs), int(max_prefill_tiles),
        decode_items.data_ptr() if decode_items is not None else 0, num_decode_items, num_decode_waves,
        num_part_slots,
        out.data_ptr(), out.stride(0), out.stride(1),
        workspace.data_ptr(), workspace.numel() * workspace.element_size(),
        *_tail_args(q, k_cache, softmax_scale),
    )
