"""The numpy statement of the decode planners, kept as the specification
that the library's native planners (``mva_decode_plan_claims`` /
``mva_decode_plan_listed``, behind ``attention_backend.make_decode_plan`` and
``make_decode_plan_listed``) must reproduce row for row.  Test code only."""

from __future__ import annotations

import numpy as np

DECODE_ITEM_INTS = 8
MAX_CHUNK_PAGES = 128


def claims_plan_spec(
    block_counts: np.ndarray | tuple[int, ...],
    first_seq: int,
    first_q_row: int,
    num_kv_heads: int,
    num_waves: int,
    pieces_per_wave: float = 1.5,
    min_piece_pages: int = 4,
    max_piece_pages: int = MAX_CHUNK_PAGES,
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
    launch.
    """
    counts = np.asarray(block_counts, dtype=np.int64)
    if counts.size == 0:
        return np.zeros((0, DECODE_ITEM_INTS), np.int32), 0, 0
    if np.any(counts <= 0):
        raise ValueError("every decode sequence needs at least one page")
    if not 1 <= min_piece_pages <= max_piece_pages <= MAX_CHUNK_PAGES:
        raise ValueError("piece length bounds must satisfy 1 <= min <= max <= 128")
    seg_len = np.repeat(counts, num_kv_heads)
    nseg = seg_len.size
    total = int(seg_len.sum())
    target = max(1, int(num_waves * max(1.0, float(pieces_per_wave))))
    piece = int(np.clip(-(-total // target), min_piece_pages, max_piece_pages))
    nchunks = (seg_len + piece - 1) // piece
    seg_of = np.repeat(np.arange(nseg), nchunks)
    first_piece = np.cumsum(nchunks) - nchunks
    chunk = np.arange(int(nchunks.sum())) - np.repeat(first_piece, nchunks)
    n_of = nchunks[seg_of]
    len_of = seg_len[seg_of]
    # Near-equal cut of L pages into n pieces: piece k covers [k*L//n, (k+1)*L//n).
    begin = (chunk * len_of) // n_of
    end = ((chunk + 1) * len_of) // n_of
    # Every KV head of a sequence has the same length and so the same cut:
    # partial slots are numbered per sequence.
    seq_split = np.where(nchunks[::num_kv_heads] > 1, nchunks[::num_kv_heads], 0)
    seq_base = np.cumsum(seq_split) - seq_split
    items = np.zeros((seg_of.size, DECODE_ITEM_INTS), dtype=np.int32)
    items[:, 0] = first_seq + seg_of // num_kv_heads
    items[:, 1] = begin
    items[:, 2] = end
    items[:, 3] = chunk
    items[:, 4] = n_of
    items[:, 5] = seq_base[seg_of // num_kv_heads]
    items[:, 6] = first_q_row + seg_of // num_kv_heads
    items[:, 7] = seg_of % num_kv_heads
    order = np.argsort(-(end - begin), kind="stable")
    items = items[order]
    waves = max(1, min(int(num_waves), items.shape[0]))
    return items, waves, int(seq_split.sum())


def listed_plan_spec(
    block_counts: np.ndarray | tuple[int, ...],
    first_seq: int,
    first_q_row: int,
    num_kv_heads: int,
    num_groups: int,
    max_piece_pages: int = MAX_CHUNK_PAGES,
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
    order, at rows ``wave_extra[w] .. wave_extra[w + 1] - 1``.
    """
    counts = np.asarray(block_counts, dtype=np.int64)
    if counts.size == 0:
        return np.zeros((0, DECODE_ITEM_INTS), np.int32), np.zeros(1, np.int32), 0, 0
    if np.any(counts <= 0):
        raise ValueError("every decode sequence needs at least one page")
    if not 1 <= max_piece_pages <= MAX_CHUNK_PAGES:
        raise ValueError("piece length must be in [1, 128] pages")
    hkv = int(num_kv_heads)
    offsets = np.concatenate(([0], np.cumsum(counts)))
    total = int(offsets[-1])
    groups = max(1, min(int(num_groups), total))
    bounds = (np.arange(groups + 1, dtype=np.int64) * total) // groups
    # Breakpoints of both partitions: every interval lies in one range and
    # one sequence.
    cuts = np.union1d(bounds, offsets)
    starts, ends = cuts[:-1], cuts[1:]
    group_of = np.searchsorted(bounds, starts, side="right") - 1
    seq_of = np.searchsorted(offsets, starts, side="right") - 1
    lengths = ends - starts
    ncut = (lengths + max_piece_pages - 1) // max_piece_pages
    iv = np.repeat(np.arange(starts.size), ncut)
    k = np.arange(iv.size) - np.repeat(np.cumsum(ncut) - ncut, ncut)
    p_begin = starts[iv] + (k * lengths[iv]) // ncut[iv]
    p_end = starts[iv] + ((k + 1) * lengths[iv]) // ncut[iv]
    piece_group = group_of[iv]
    piece_seq = seq_of[iv]
    per_seq = np.bincount(piece_seq, minlength=counts.size)
    chunk = np.arange(iv.size) - (np.cumsum(per_seq) - per_seq)[piece_seq]
    split = np.where(per_seq > 1, per_seq, 0)
    part_base = np.cumsum(split) - split
    pieces = np.zeros((iv.size, hkv, DECODE_ITEM_INTS), dtype=np.int32)
    pieces[:, :, 0] = (first_seq + piece_seq)[:, None]
    pieces[:, :, 1] = (p_begin - offsets[piece_seq])[:, None]
    pieces[:, :, 2] = (p_end - offsets[piece_seq])[:, None]
    pieces[:, :, 3] = chunk[:, None]
    pieces[:, :, 4] = per_seq[piece_seq][:, None]
    pieces[:, :, 5] = part_base[piece_seq][:, None]
    pieces[:, :, 6] = (first_q_row + piece_seq)[:, None]
    pieces[:, :, 7] = np.arange(hkv)[None, :]
    wave_of = (piece_group[:, None] * hkv + np.arange(hkv)[None, :]).reshape(-1)
    pieces = pieces.reshape(-1, DECODE_ITEM_INTS)
    order = np.argsort(wave_of, kind="stable")  # page order within a wavefront
    pieces, wave_of = pieces[order], wave_of[order]
    waves = groups * hkv
    per_wave = np.bincount(wave_of, minlength=waves)
    first = np.cumsum(per_wave) - per_wave
    is_first = np.zeros(pieces.shape[0], dtype=bool)
    is_first[first] = True
    items = np.concatenate([pieces[first], pieces[~is_first]])
    wave_extra = waves + np.concatenate(([0], np.cumsum(per_wave - 1)))
    return items, wave_extra.astype(np.int32), waves, int(split.sum())


def merge_list_spec(items: np.ndarray) -> np.ndarray:
    """Chunk 0 of every split segment, in item order."""
    return items[(items[:, 3] == 0) & (items[:, 4] > 1)]
