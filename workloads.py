"""Seeded synthetic batches for the hot path's benchmark configurations
(used by the tests, the smoke check and bench.py; not part of the package).

A batch is what the reference's ModelRunner would hand to the attention layer
for one step (nanovllm/engine/model_runner.py:361-484): packed queries, new
K/V rows with their ``slot_mapping``, and a paged KV cache whose pages are a
random permutation of a pool sized to the total context.  Every sequence's
``seq_len`` includes its new tokens; the new tokens occupy positions
``[seq_len - q_len, seq_len)``.  Prefill sequences come first.

Values are drawn from N(0, 1) with a seeded ``torch.Generator``.  Small batches
are drawn on the CPU (so the CPU oracle sees identical bits); multi-GB batches
can be drawn directly on the GPU (``rng_device="cuda"``).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from my_vllm_amd.contract import CommonAttentionMetadata

PAGE_SIZE = 16
HEAD_DIM = 128


@dataclass
class PagedBatch:
    common: CommonAttentionMetadata
    q: torch.Tensor  # [T, Hq, D]
    k_new: torch.Tensor  # [T, Hkv, D]
    v_new: torch.Tensor  # [T, Hkv, D]
    k_cache: torch.Tensor  # [P, 16, Hkv, D]
    v_cache: torch.Tensor
    query_lengths: list[int]
    kv_lengths: list[int]
    block_counts: tuple[int, ...]
    block_tables_host: np.ndarray  # [S, W] int32


def _randn(shape, gen: torch.Generator, dtype, device, rng_device: str) -> torch.Tensor:
    t = torch.randn(shape, generator=gen, dtype=torch.float32, device=rng_device).to(dtype)
    return t.to(device)


def make_paged_batch(
    seed: int,
    query_lengths: list[int],
    kv_lengths: list[int],
    num_prefill_seqs: int,
    num_q_heads: int,
    num_kv_heads: int,
    dtype: torch.dtype = torch.bfloat16,
    device: str | torch.device = "cpu",
    rng_device: str = "cpu",
    head_dim: int = HEAD_DIM,
    extra_pages: int = 0,
) -> PagedBatch:
    """Build one step's batch (see module docstring); pages permuted with `seed`."""
    if len(query_lengths) != len(kv_lengths):
        raise ValueError("query_lengths and kv_lengths differ in length")
    if any(q <= 0 or q > kv for q, kv in zip(query_lengths, kv_lengths)):
        raise ValueError("every sequence needs 0 < q_len <= kv_len")
    if any(q != 1 for q in query_lengths[num_prefill_seqs:]):
        raise ValueError("decode sequences have exactly one query token")
    gen = torch.Generator(device=rng_device)
    gen.manual_seed(seed)
    np_rng = np.random.default_rng(seed)
    counts = [(kv + PAGE_SIZE - 1) // PAGE_SIZE for kv in kv_lengths]
    num_pages = sum(counts) + extra_pages
    perm = np_rng.permutation(num_pages).astype(np.int32)
    width = max(counts)
    bt = np.full((len(counts), width), -1, dtype=np.int32)
    pos = 0
    for s, c in enumerate(counts):
        bt[s, :c] = perm[pos : pos + c]
        pos += c
    slots = []
    for s, (q_len, kv_len) in enumerate(zip(query_lengths, kv_lengths)):
        for p in range(kv_len - q_len, kv_len):
            slots.append(int(bt[s, p // PAGE_SIZE]) * PAGE_SIZE + p % PAGE_SIZE)
    total_q = sum(query_lengths)
    q = _randn((total_q, num_q_heads, head_dim), gen, dtype, device, rng_device)
    k_new = _randn((total_q, num_kv_heads, head_dim), gen, dtype, device, rng_device)
    v_new = _randn((total_q, num_kv_heads, head_dim), gen, dtype, device, rng_device)
    k_cache = _randn((num_pages, PAGE_SIZE, num_kv_heads, head_dim), gen, dtype, device, rng_device)
    v_cache = _randn((num_pages, PAGE_SIZE, num_kv_heads, head_dim), gen, dtype, device, rng_device)
    qsl = np.concatenate(([0], np.cumsum(query_lengths))).astype(np.int32)
    dev = torch.device(device)
    common = CommonAttentionMetadata(
        num_prefill_seqs=num_prefill_seqs,
        num_decode_seqs=len(query_lengths) - num_prefill_seqs,
        num_prefill_tokens=int(sum(query_lengths[:num_prefill_seqs])),
        num_decode_tokens=int(sum(query_lengths[num_prefill_seqs:])),
        query_start_loc=torch.from_numpy(qsl).to(dev),
        seq_lens=torch.tensor(kv_lengths, dtype=torch.int32, device=dev),
        slot_mapping=torch.tensor(slots, dtype=torch.int32, device=dev),
        block_tables=torch.from_numpy(bt).to(dev),
        max_q_len=max(query_lengths),
        max_kv_len=max(kv_lengths),
        block_counts=tuple(counts),
        num_kv_blocks=sum(counts),
        num_prefill_kv_blocks=sum(counts[:num_prefill_seqs]),
        trusted=True,
    )
    return PagedBatch(
        common=common,
        q=q,
        k_new=k_new,
        v_new=v_new,
        k_cache=k_cache,
        v_cache=v_cache,
        query_lengths=list(query_lengths),
        kv_lengths=list(kv_lengths),
        block_counts=tuple(counts),
        block_tables_host=bt,
    )


# ---------------------------------------------------------------------------
# The benchmark configurations (integer draws use numpy's seeded generator).
# ---------------------------------------------------------------------------

def silu_input(tokens: int = 4096, width: int = 6144, seed: int = 0, dtype=torch.bfloat16,
               device="cpu", rng_device="cpu") -> torch.Tensor:
    """SiLU-and-mul input ``[tokens, width]`` ~ N(0, 1) (Qwen3-0.6B MLP: 4096 x 6144)."""
    gen = torch.Generator(device=rng_device)
    gen.manual_seed(seed)
    return _randn((tokens, width), gen, dtype, device, rng_device)


def decode_lengths(seed: int, batch: int, lo: int, hi: int) -> list[int]:
    """Context lengths uniform in [lo, hi] (inclusive)."""
    return [int(x) for x in np.random.default_rng(seed).integers(lo, hi + 1, size=batch)]


def config_decode_small(seed: int = 1, **kw) -> PagedBatch:
    """KV store + PURE_DECODE at Qwen3-0.6B shape: 16 Q / 8 KV heads, 64 seqs, ctx U[128, 2048]."""
    ctx = decode_lengths(seed, 64, 128, 2048)
    return make_paged_batch(seed, [1] * 64, ctx, 0, 16, 8, **kw)


def prefill_lengths(seed: int, num_seqs: int = 16) -> tuple[list[int], list[int]]:
    """New-token counts U[64, 2048] and cached prefixes 16*U[0, 64] per sequence."""
    rng = np.random.default_rng(seed)
    q = [int(x) for x in rng.integers(64, 2048 + 1, size=num_seqs)]
    prefix = [16 * int(x) for x in rng.integers(0, 64 + 1, size=num_seqs)]
    return q, [a + b for a, b in zip(q, prefix)]


def config_prefill(seed: int = 2, **kw) -> PagedBatch:
    """PURE_PREFILL with prefix cache at Qwen3-8B shape: 32 Q / 8 KV heads, 16 seqs."""
    q, kv = prefill_lengths(seed)
    return make_paged_batch(seed, q, kv, len(q), 32, 8, **kw)


def mixed_lengths(seed: int, budget: int = 8192) -> tuple[list[int], list[int], int]:
    """4 prefill chunks (q U[512, 2048] over existing ctx U[0, 8192]) + 256 decodes
    (ctx U[512, 8192]); chunk draws are repeated until sum(q) + 256 <= budget."""
    rng = np.random.default_rng(seed)
    while True:
        q = [int(x) for x in rng.integers(512, 2048 + 1, size=4)]
        if sum(q) + 256 <= budget:
            break
    existing = [int(x) for x in rng.integers(0, 8192 + 1, size=4)]
    dec = [int(x) for x in rng.integers(512, 8192 + 1, size=256)]
    q_lens = q + [1] * 256
    kv_lens = [a + b for a, b in zip(q, existing)] + dec
    return q_lens, kv_lens, 4


def config_mixed(seed: int = 3, **kw) -> PagedBatch:
    """MIXED chunked-prefill batch at Qwen3-8B shape, token budget 8192."""
    q, kv, num_prefill = mixed_lengths(seed)
    return make_paged_batch(seed, q, kv, num_prefill, 32, 8, **kw)


def config_long_decode(seed: int = 4, batch: int = 128, **kw) -> PagedBatch:
    """Long-context decode at Qwen3-32B shape: 64 Q / 8 KV heads, ctx U[8192, 32768]."""
    ctx = decode_lengths(seed, batch, 8192, 32768)
    return make_paged_batch(seed, [1] * batch, ctx, 0, 64, 8, **kw)
