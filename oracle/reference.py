"""CPU restatement of the reference's native paths (test infrastructure only).

Every function names the reference code it restates.  Inputs are torch CPU
tensors (or numpy arrays for the integer helpers); arithmetic is fp32.
"""

from __future__ import annotations

from math import sqrt

import numpy as np
import torch
import torch.nn.functional as F


# ---------------------------------------------------------------------------
# SiLU-and-mul
# ---------------------------------------------------------------------------

def silu_and_mul_eager(x: torch.Tensor) -> torch.Tensor:
    """``x, y = x.chunk(2, -1); F.silu(x) * y`` evaluated eagerly.

    Restates nanovllm/layers/activation.py:34-37 without ``torch.compile``:
    in eager torch the bf16/fp16 ``F.silu`` result is rounded to the storage
    type before the multiply (two roundings).
    """
    a, b = x.chunk(2, -1)
    return F.silu(a) * b


def silu_and_mul_fused(x: torch.Tensor) -> torch.Tensor:
    """fp32 ``g / (1 + exp(-g)) * u`` rounded once to the storage type.

    Restates the reference's compiled kernel (csrc/silu_and_mul_kernel.cu:26-29)
    and the fused (compiled) native path: one rounding of the fp32 product.
    """
    a, b = x.float().chunk(2, -1)
    return (a / (1.0 + torch.exp(-a)) * b).to(x.dtype)


# ---------------------------------------------------------------------------
# RMSNorm / fused residual-add RMSNorm
# ---------------------------------------------------------------------------

def rms_scaled(x32: torch.Tensor, eps: float, dtype: torch.dtype) -> torch.Tensor:
    """The row scaled by its fp32 reciprocal RMS and rounded to ``dtype``
    (the intermediate of nanovllm/layers/layernorm.py:35-38, before the
    weight multiply)."""
    r = torch.rsqrt(x32.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (x32 * r).to(dtype)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``T(T(x32 * rsqrt(mean(x32^2) + eps)) * w)`` with fp32 statistics.

    Restates nanovllm/layers/layernorm.py:31-40: the scaled row is rounded to
    the storage type, then multiplied by the weight (fp32 product, rounded
    once more).
    """
    x32 = x.float()
    r = torch.rsqrt(x32.pow(2).mean(dim=-1, keepdim=True) + eps)
    return ((x32 * r).to(x.dtype).float() * weight.float()).to(x.dtype)


def fused_add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    """``(rms_norm of the fp32 sum, T(sum))``.

    Restates nanovllm/layers/layernorm.py:42-52: the statistics use the fp32
    sum ``x + residual``, not the rounded residual that is returned.
    """
    s32 = x.float() + residual.float()
    r = torch.rsqrt(s32.pow(2).mean(dim=-1, keepdim=True) + eps)
    return ((s32 * r).to(x.dtype).float() * weight.float()).to(x.dtype), s32.to(x.dtype)


# ---------------------------------------------------------------------------
# Rotary embedding and the fused attention prologue
# ---------------------------------------------------------------------------

def rope_cos_sin_cache(rotary_dim: int, max_position: int, base: float) -> torch.Tensor:
    """``[max_position, 1, rotary_dim]`` fp32 cos | sin table
    (nanovllm/layers/rotary_embedding.py:30-35)."""
    inv_freq = 1.0 / (base ** (torch.arange(0, rotary_dim, 2, dtype=torch.float) / rotary_dim))
    freqs = torch.einsum("i,j -> ij", torch.arange(max_position, dtype=torch.float), inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1).unsqueeze_(1)


def rope(x: torch.Tensor, positions: torch.Tensor, cos_sin_cache: torch.Tensor) -> torch.Tensor:
    """Neox rotation of ``x [T, H, D]``: halves x1, x2 -> (x1 c - x2 s, x2 c + x1 s),
    fp32 products rounded once (rotary_embedding.py:7-15, 41-51)."""
    cos, sin = cos_sin_cache[positions].chunk(2, dim=-1)  # [T, 1, D/2]
    x1, x2 = torch.chunk(x.float(), 2, dim=-1)
    return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(x.dtype)


def qk_norm_rope(q, k, positions, cos_sin_cache, q_norm_weight=None, k_norm_weight=None, eps=1e-6):
    """q_norm / k_norm (per head) then RoPE, as Qwen3Attention.forward runs
    them (nanovllm/models/qwen3.py:96-100)."""
    if q_norm_weight is not None:
        q = rms_norm(q, q_norm_weight, eps)
        k = rms_norm(k, k_norm_weight, eps)
    return rope(q, positions, cos_sin_cache), rope(k, positions, cos_sin_cache)


# ---------------------------------------------------------------------------
# slot_mapping KV store
# ---------------------------------------------------------------------------

def kv_store(
    key: np.ndarray,
    value: np.ndarray,
    k_cache: np.ndarray,
    v_cache: np.ndarray,
    slot_mapping: np.ndarray,
) -> None:
    """In-place scatter of ``key[t]``/``value[t]`` to cache row ``slot_mapping[t]``.

    Restates nanovllm/layers/attention.py:69-85 (``index_copy_`` of the rows
    with ``slot >= 0``) on numpy arrays of any dtype (bit copy).  ``key`` is
    ``[N, H, D]``; caches are viewed as ``[-1, H, D]``.
    """
    n, h, d = key.shape
    if slot_mapping.size != n:
        raise ValueError("slot_mapping must contain one slot per token")
    flat_k = k_cache.reshape(-1, h, d)
    flat_v = v_cache.reshape(-1, h, d)
    valid = slot_mapping >= 0
    slots = slot_mapping[valid].astype(np.int64)
    flat_k[slots] = key[valid]
    flat_v[slots] = value[valid]


def kv_store_index_copy(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                        slot_mapping: torch.Tensor) -> None:
    """The same scatter in torch, as the reference's CPU path runs it:
    ``index_copy_`` of the rows whose slot is ``>= 0`` into the caches viewed
    as ``[-1, H, D]`` (nanovllm/layers/attention.py:69-85).  Timed as the
    store's CPU baseline; pinned to ``kv_store`` by the tests."""
    if slot_mapping.numel() != key.shape[0]:
        raise ValueError("slot_mapping must contain one slot per token")
    h, d = key.shape[-2:]
    keep = slot_mapping >= 0
    rows = slot_mapping[keep].long()
    k_cache.view(-1, h, d).index_copy_(0, rows, key[keep])
    v_cache.view(-1, h, d).index_copy_(0, rows, value[keep])


# ---------------------------------------------------------------------------
# Paged / ragged attention
# ---------------------------------------------------------------------------

def paged_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    query_lengths: list[int],
    kv_lengths: list[int],
) -> torch.Tensor:
    """fp32 paged causal attention over NHD pages, bottom-right aligned.

    Restates the reference's test oracle ``_paged_attention_reference``
    (tests/test_attention_backend.py:660-699), reading pages from dense
    ``block_tables`` rows: query ``i`` of sequence ``s`` sits at absolute
    position ``kv_s - q_s + i`` and sees keys ``j <= kv_s - q_s + i``
    (:686-693); GQA repeats each KV head over ``Hq / Hkv`` query heads.
    Returns fp32 ``[T, Hq, D]``.
    """
    page = k_cache.shape[1]
    group = q.shape[1] // k_cache.shape[2]
    outputs = []
    start = 0
    for s, (q_len, kv_len) in enumerate(zip(query_lengths, kv_lengths)):
        n_pages = (kv_len + page - 1) // page
        pages = block_tables[s, :n_pages].long()
        keys = k_cache[pages].flatten(0, 1)[:kv_len].float()
        values = v_cache[pages].flatten(0, 1)[:kv_len].float()
        keys = keys.repeat_interleave(group, dim=1)
        values = values.repeat_interleave(group, dim=1)
        query = q[start : start + q_len].float()
        scores = torch.einsum("qhd,khd->hqk", query, keys) / sqrt(q.shape[-1])
        q_pos = torch.arange(kv_len - q_len, kv_len)
        k_pos = torch.arange(kv_len)
        mask = k_pos[None, :] <= q_pos[:, None]
        scores.masked_fill_(~mask[None], -torch.inf)
        probs = torch.softmax(scores, dim=-1)
        outputs.append(torch.einsum("hqk,khd->qhd", probs, values))
        start += q_len
    return torch.cat(outputs)


def ragged_attention(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, lengths: list[int]
) -> torch.Tensor:
    """fp32 cacheless causal varlen attention (query length == key length).

    Restates ``_ragged_attention_reference``
    (tests/test_attention_backend.py:702-734).  Returns fp32 ``[T, Hq, D]``.
    """
    group = q.shape[1] // k.shape[1]
    outputs = []
    start = 0
    for length in lengths:
        query = q[start : start + length].float()
        keys = k[start : start + length].float().repeat_interleave(group, dim=1)
        values = v[start : start + length].float().repeat_interleave(group, dim=1)
        scores = torch.einsum("qhd,khd->hqk", query, keys) / sqrt(q.shape[-1])
        mask = torch.arange(length)[None, :] <= torch.arange(length)[:, None]
        scores.masked_fill_(~mask[None], -torch.inf)
        outputs.append(torch.einsum("hqk,khd->qhd", torch.softmax(scores, dim=-1), values))
        start += length
    return torch.cat(outputs)


def attention_partial(q_row: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, scale: float):
    """Normalised output and natural-log sum-exp of one query over a key range.

    The split-K building block: ``o = softmax(scale q.K) V`` and
    ``lse = log(sum exp(scale q.K))`` (fp32; ``q_row`` ``[D]``, keys/values ``[N, D]``).
    """
    scores = keys.float() @ q_row.float() * scale
    lse = torch.logsumexp(scores, dim=0)
    probs = torch.exp(scores - lse)
    return probs @ values.float(), lse


def lse_merge(outputs: list[torch.Tensor], lses: list[torch.Tensor]) -> torch.Tensor:
    """Combine split-K partials: sum_i exp(lse_i - max) o_i / sum_i exp(lse_i - max)."""
    lse = torch.stack(lses)
    weights = torch.exp(lse - lse.max())
    return (weights[:, None] * torch.stack(outputs)).sum(0) / weights.sum()


# ---------------------------------------------------------------------------
# Metadata helpers
# ---------------------------------------------------------------------------

def classify_batch(num_prefill_seqs: int, num_decode_seqs: int) -> str:
    """Restates ``_classify_batch`` (nanovllm/layers/attention_backend.py:1484-1491)."""
    if num_prefill_seqs == 0:
        if num_decode_seqs <= 0:
            raise ValueError("pure decode batch must contain decode requests")
        return "pure_decode"
    if num_decode_seqs == 0:
        return "pure_prefill"
    return "mixed"


def page_csr(block_tables: np.ndarray, seq_lens: list[int], block_size: int, num_prefill_seqs: int):
    """Dense block tables -> page CSR, as the reference builds it for FlashInfer.

    Restates nanovllm/layers/attention_backend.py:725-761: ``kv_indptr`` from
    ``ceil(seq_len / block_size)``, ``page_indices`` = row prefixes of
    ``block_tables``, ``last_page_len = (seq_len - 1) % block_size + 1``.
    Returns ``(kv_indptr, page_indices, last_page_len, num_pages, num_prefill_pages)``.
    """
    counts = [(n + block_size - 1) // block_size for n in seq_lens]
    kv_indptr = [0]
    for c in counts:
        kv_indptr.append(kv_indptr[-1] + c)
    page_indices = [int(block_tables[s][j]) for s, c in enumerate(counts) for j in range(c)]
    last_page_len = [(n - 1) % block_size + 1 for n in seq_lens]
    return kv_indptr, page_indices, last_page_len, kv_indptr[-1], kv_indptr[num_prefill_seqs]


def slot_mapping_for(
    block_table: list[int], num_cached_tokens: int, num_context_tokens: int, block_size: int
) -> list[int]:
    """Cache slots of a sequence's new tokens ``[num_cached_tokens, num_context_tokens)``.

    Restates the slot loop of ModelRunner.prepare_model_input
    (nanovllm/engine/model_runner.py:405-419): slot = page * block_size + offset.
    """
    return [
        block_table[pos // block_size] * block_size + pos % block_size
        for pos in range(num_cached_tokens, num_context_tokens)
    ]


def split_page_csr(query_start_loc: list[int], kv_indptr: list[int], page_indices: list[int],
                   last_page_len: list[int], num_prefill_seqs: int, num_prefill_pages: int):
    """MIXED_SPLIT slicing of the page CSR into a prefill part and a decode part.

    Restates nanovllm/layers/attention_backend.py:858-889: the prefill plan
    takes the first ``num_prefill_seqs + 1`` offsets and the first
    ``num_prefill_pages`` pages; the decode plan takes the rest, with its
    ``kv_indptr`` re-based by ``num_prefill_pages`` (:874-876).
    """
    p = num_prefill_seqs
    prefill = {
        "qo_indptr": list(query_start_loc[: p + 1]),
        "kv_indptr": list(kv_indptr[: p + 1]),
        "page_indices": list(page_indices[:num_prefill_pages]),
        "last_page_len": list(last_page_len[:p]),
    }
    decode = {
        "kv_indptr": [x - num_prefill_pages for x in kv_indptr[p:]],
        "page_indices": list(page_indices[num_prefill_pages:]),
        "last_page_len": list(last_page_len[p:]),
    }
    return prefill, decode
