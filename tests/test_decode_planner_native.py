"""The library's host-side decode planners (mva_decode_plan_listed /
mva_decode_plan_claims) against their numpy statement (tests/_decode_plan_spec.py):
identical items, piece-list offsets, wave counts, partial slots and merge
lists, row for row, over random batches and the edge cases of both cuts.
No GPU: the planners are host code of the library."""

import numpy as np
import pytest

from my_vllm_amd import _native, ops
from my_vllm_amd.attention_backend import (
    make_decode_plan,
    make_decode_plan_listed,
    plan_decode_claims,
    plan_decode_listed,
)
from tests._decode_plan_spec import claims_plan_spec, listed_plan_spec, merge_list_spec


def _batch(rng):
    n = int(rng.choice([1, 2, 3, 7, 64, 129, 300]))
    hi = int(rng.choice([1, 2, 9, 128, 129, 700, 2048]))
    return rng.integers(1, hi + 1, size=n, dtype=np.int64)


@pytest.mark.parametrize("seed", range(40))
def test_listed_plan_matches_the_numpy_statement(seed):
    rng = np.random.default_rng(1000 + seed)
    counts = _batch(rng)
    hkv = int(rng.choice([1, 2, 3, 8]))
    groups = int(rng.choice([1, 5, 256, 2048, 100000]))
    max_piece = int(rng.choice([1, 3, 64, 128]))
    first_seq, first_q_row = int(rng.integers(0, 50)), int(rng.integers(0, 5000))
    items, wave_extra, waves, slots, merges = plan_decode_listed(counts, first_seq, first_q_row, hkv, groups,
                                                                 max_piece)
    e_items, e_extra, e_waves, e_slots = listed_plan_spec(counts, first_seq, first_q_row, hkv, groups, max_piece)
    assert np.array_equal(items, e_items) and items.dtype == np.int32
    assert np.array_equal(wave_extra, e_extra) and wave_extra.dtype == np.int32
    assert (waves, slots) == (e_waves, e_slots)
    assert np.array_equal(merges, merge_list_spec(e_items))
    assert np.array_equal(ops.decode_merge_list(items), merges)
    got = make_decode_plan_listed(counts, first_seq, first_q_row, hkv, groups, max_piece)
    assert all(np.array_equal(a, b) for a, b in zip(got[:2], (e_items, e_extra))) and got[2:] == (e_waves, e_slots)


@pytest.mark.parametrize("seed", range(40))
def test_claims_plan_matches_the_numpy_statement(seed):
    rng = np.random.default_rng(2000 + seed)
    counts = _batch(rng)
    hkv = int(rng.choice([1, 2, 3, 8]))
    waves = int(rng.choice([1, 4, 64, 1280, 1536, 100000]))
    per_wave = float(rng.choice([0.5, 1.0, 1.5, 2.0, 3.3]))
    lo = int(rng.choice([1, 2, 4, 16]))
    hi = int(rng.choice([lo, 64, 128]))
    first_seq, first_q_row = int(rng.integers(0, 50)), int(rng.integers(0, 5000))
    items, nw, slots, merges = plan_decode_claims(counts, first_seq, first_q_row, hkv, waves, per_wave, lo, hi)
    e_items, e_nw, e_slots = claims_plan_spec(counts, first_seq, first_q_row, hkv, waves, per_wave, lo, hi)
    assert np.array_equal(items, e_items) and items.dtype == np.int32
    assert (nw, slots) == (e_nw, e_slots)
    assert np.array_equal(merges, merge_list_spec(e_items))
    got = make_decode_plan(counts, first_seq, first_q_row, hkv, waves, per_wave, lo, hi)
    assert np.array_equal(got[0], e_items) and got[1:] == (e_nw, e_slots)


def test_headline_and_long_context_batches_match():
    from workloads import decode_lengths

    for seed, n, lo, hi, hkv in ((1, 64, 128, 2048, 8), (4, 128, 8192, 32768, 8), (3, 256, 512, 8192, 8)):
        counts = np.asarray([(c + 15) // 16 for c in decode_lengths(seed, n, lo, hi)], dtype=np.int64)
        a = plan_decode_listed(counts, 4, 9, hkv, 256)
        b = listed_plan_spec(counts, 4, 9, hkv, 256)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1]) and a[2:4] == b[2:4]
        c = plan_decode_claims(counts, 4, 9, hkv, 1280)
        d = claims_plan_spec(counts, 4, 9, hkv, 1280)
        assert np.array_equal(c[0], d[0]) and c[1:3] == d[1:3]


def test_planners_refuse_bad_input_like_the_statement():
    for planner in (lambda c: plan_decode_listed(c, 0, 0, 8, 256), lambda c: plan_decode_claims(c, 0, 0, 8, 64)):
        with pytest.raises(ValueError):
            planner(np.array([3, 0, 2]))
        with pytest.raises(ValueError):
            planner(np.array([-1]))
    with pytest.raises(ValueError):
        plan_decode_listed(np.array([3]), 0, 0, 8, 256, max_piece_pages=129)
    with pytest.raises(ValueError):
        plan_decode_claims(np.array([3]), 0, 0, 8, 64, 1.5, 8, 4)
    empty = plan_decode_listed(np.zeros(0, np.int64), 0, 0, 8, 256)
    assert empty[0].shape == (0, 8) and np.array_equal(empty[1], [0]) and empty[2:4] == (0, 0)
    empty = plan_decode_claims(np.zeros(0, np.int64), 0, 0, 8, 64)
    assert empty[0].shape == (0, 8) and empty[1:3] == (0, 0)
    # Capacities the C ABI checks itself.
    counts = np.array([40, 7], np.int64)
    items = np.empty((1, 8), np.int32)
    extra = np.empty(17, np.int32)
    out = np.zeros(4, np.int64)
    with pytest.raises(RuntimeError, match="capacity"):
        _native.call("mva_decode_plan_listed", counts.ctypes.data, 2, 0, 0, 8, 2, 128, items.ctypes.data, 1,
                     extra.ctypes.data, extra.size, 0, 0, out.ctypes.data)
    with pytest.raises(RuntimeError, match="wave_extra"):
        _native.call("mva_decode_plan_listed", counts.ctypes.data, 2, 0, 0, 8, 2, 128, items.ctypes.data, 1,
                     extra.ctypes.data, 4, 0, 0, out.ctypes.data)
    with pytest.raises(RuntimeError, match="capacity"):
        _native.call("mva_decode_plan_claims", counts.ctypes.data, 2, 0, 0, 8, 64, 1.5, 4, 128,
                     items.ctypes.data, 1, 0, 0, out.ctypes.data)


def test_planners_refuse_indices_beyond_int32():
    # Sequence and query-row indices are int32 in the pieces: the last
    # sequence may sit at 2^31-1 but not past it.
    top = 2**31 - 1
    counts = np.array([3, 5], np.int64)
    for first_seq, first_q_row in ((top, 0), (0, top), (top - 1, top + 5)):
        with pytest.raises(RuntimeError, match="int32 range"):
            plan_decode_claims(counts, first_seq, first_q_row, 8, 16)
        with pytest.raises(RuntimeError, match="int32 range"):
            plan_decode_listed(counts, first_seq, first_q_row, 8, 16)
    items, _, _, _ = plan_decode_claims(counts, top - 1, top - 1, 8, 16)
    assert items[:, 0].max() == top and items[:, 6].max() == top
    items, _, _, _, _ = plan_decode_listed(counts, top - 1, top - 1, 8, 16)
    assert items[:, 0].max() == top and items[:, 6].max() == top


def test_claims_planner_refuses_more_than_int32_pieces():
    # 3 segments of 2^31-1 pages at 64 KV heads and 128-page pieces: about
    # 3.2e9 pieces.  Refused before anything is written (a 1-row buffer).
    top = 2**31 - 1
    counts = np.full(3, top, np.int64)
    items = np.zeros((1, ops.DECODE_ITEM_INTS), np.int32)
    out = np.zeros(4, np.int64)
    with pytest.raises(RuntimeError, match="2\\^31-1 pieces"):
        _native.call("mva_decode_plan_claims", counts.ctypes.data, 3, 0, 0, 64, 1, 1.0, 1, 128,
                     items.ctypes.data, 1 << 40, 0, 0, out.ctypes.data)
    assert not items.any() and not out.any()
