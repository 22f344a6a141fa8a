"""CPU: the oracle's integer functions against the reference's known-answer vectors.

The vectors live in tests/golden/reference_kats.json (written by
tests/golden/make_golden.py, each with the reference test it comes from).
Brute-force cases pin the KV store beyond the single known answer.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from my_vllm_amd.contract import BatchType, CommonAttentionMetadata
from oracle.reference import classify_batch, kv_store, page_csr, slot_mapping_for, split_page_csr

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def test_kv_store_reference_known_answer():
    kat = KATS["kv_store"]
    key = np.arange(kat["key"]["arange_from"], kat["key"]["arange_to"], dtype=np.float32).reshape(kat["key"]["shape"])
    value = key + kat["value_offset"]
    k_cache = np.full(kat["cache_shape"], kat["cache_fill"], dtype=np.float32)
    v_cache = np.full(kat["cache_shape"], kat["cache_fill"], dtype=np.float32)
    expected_k, expected_v = k_cache.copy(), v_cache.copy()
    rows = key.shape[1:]
    for row, token in kat["writes"]:
        expected_k.reshape(-1, *rows)[row] = key[token]
        expected_v.reshape(-1, *rows)[row] = value[token]
    kv_store(key, value, k_cache, v_cache, np.array(kat["slot_mapping"], dtype=np.int64))
    np.testing.assert_array_equal(k_cache, expected_k)
    np.testing.assert_array_equal(v_cache, expected_v)


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("slot_dtype", [np.int32, np.int64])
def test_kv_store_matches_brute_force(seed, slot_dtype):
    rng = np.random.default_rng(seed)
    pages, page, heads, dim, tokens = 5, 4, 2, 3, 9
    key = rng.standard_normal((tokens, heads, dim)).astype(np.float32)
    value = rng.standard_normal((tokens, heads, dim)).astype(np.float32)
    slots = rng.permutation(pages * page)[:tokens].astype(slot_dtype)
    slots[rng.random(tokens) < 0.3] = -1
    k_cache = rng.standard_normal((pages, page, heads, dim)).astype(np.float32)
    v_cache = rng.standard_normal((pages, page, heads, dim)).astype(np.float32)
    expected_k, expected_v = k_cache.copy(), v_cache.copy()
    for t in range(tokens):
        s = int(slots[t])
        if s < 0:
            continue
        for h in range(heads):
            for d in range(dim):
                expected_k[s // page, s % page, h, d] = key[t, h, d]
                expected_v[s // page, s % page, h, d] = value[t, h, d]
    kv_store(key, value, k_cache, v_cache, slots)
    np.testing.assert_array_equal(k_cache, expected_k)
    np.testing.assert_array_equal(v_cache, expected_v)


def test_kv_store_rejects_wrong_slot_count():
    key = np.zeros((3, 1, 2), np.float32)
    with pytest.raises(ValueError, match="one slot per token"):
        kv_store(key, key, np.zeros((2, 2, 1, 2), np.float32), np.zeros((2, 2, 1, 2), np.float32), np.zeros(2))


def test_page_csr_reference_known_answer():
    kat = KATS["page_csr"]
    kv_indptr, page_indices, last_page_len, num_pages, num_prefill_pages = page_csr(
        np.array(kat["block_tables"]), kat["kv_lengths"], 16, kat["num_prefill_seqs"]
    )
    assert kv_indptr == kat["kv_indptr"]
    assert page_indices == kat["page_indices"]
    assert last_page_len == kat["last_page_len"]
    assert num_pages == kat["num_pages"]
    assert num_prefill_pages == kat["num_prefill_pages"]


def test_last_page_len_is_never_zero():
    # docs/operator-audit.md:94-95: a full last page has length 16, not 0.
    _, _, last, _, _ = page_csr(np.array([[0], [1], [2, 3]], dtype=object), [16, 1, 32], 16, 0)
    assert last == [16, 1, 16]


def test_split_csr_reference_known_answer():
    kat = KATS["split_csr"]
    qsl = np.concatenate(([0], np.cumsum(kat["query_lengths"]))).tolist()
    bt = np.array(KATS["page_csr"]["block_tables"])
    kv_indptr, page_indices, last_page_len, _, num_prefill_pages = page_csr(
        bt, kat["kv_lengths"], 16, kat["num_prefill_seqs"]
    )
    prefill, decode = split_page_csr(qsl, kv_indptr, page_indices, last_page_len, kat["num_prefill_seqs"],
                                     num_prefill_pages)
    assert prefill == kat["prefill"]
    assert decode == kat["decode"]


@pytest.mark.parametrize("case", KATS["slot_mapping"], ids=lambda c: c["source"].split(":")[-1])
def test_slot_mapping_reference_known_answers(case):
    slots, qsl, seq_lens = [], [0], []
    for block_table, cached, context in case["sequences"]:
        slots += slot_mapping_for(block_table, cached, context, 16)
        qsl.append(qsl[-1] + context - cached)
        seq_lens.append(context)
    assert slots == case["slot_mapping"]
    assert qsl == case["query_start_loc"]
    assert seq_lens == case["seq_lens"]
    counts = [(n + 15) // 16 for n in seq_lens]
    assert counts == case["block_counts"]
    width = max(len(bt) for bt, _, _ in case["sequences"])
    padded = [bt + [-1] * (width - len(bt)) for bt, _, _ in case["sequences"]]
    assert padded == case["block_tables"]


@pytest.mark.parametrize("prefill,decode,expected", KATS["classify"]["cases"])
def test_classification_reference_known_answers(prefill, decode, expected):
    assert classify_batch(prefill, decode) == expected
    assert BatchType(expected).value == expected


def test_classification_rejects_empty_batch():
    with pytest.raises(ValueError):
        classify_batch(0, 0)


def test_common_metadata_totals_known_answer():
    kat = KATS["common_totals"]
    q, kv, p = kat["query_lengths"], kat["kv_lengths"], kat["num_prefill_seqs"]
    qsl = np.concatenate(([0], np.cumsum(q))).tolist()
    common = CommonAttentionMetadata(
        num_prefill_seqs=p,
        num_decode_seqs=len(q) - p,
        num_prefill_tokens=sum(q[:p]),
        num_decode_tokens=sum(q[p:]),
        query_start_loc=torch.tensor(qsl, dtype=torch.int32),
        seq_lens=torch.tensor(kv, dtype=torch.int32),
        slot_mapping=torch.arange(qsl[-1], dtype=torch.int32),
        max_q_len=max(q),
        max_kv_len=max(kv),
        block_counts=tuple((n + 15) // 16 for n in kv),
    )
    assert common.num_prefill_tokens == kat["num_prefill_tokens"]
    assert common.num_decode_tokens == kat["num_decode_tokens"]
    assert common.num_seqs == kat["num_seqs"]
    assert common.num_query_tokens == kat["num_query_tokens"]
    assert common.query_start_loc.tolist() == kat["query_start_loc"]
    assert list(common.block_counts) == kat["block_counts"]
    assert (common.max_q_len, common.max_kv_len) == (kat["max_q_len"], kat["max_kv_len"])
    with pytest.raises(Exception):
        common.num_prefill_seqs = 3  # frozen for one runtime step


def test_golden_fixture_is_current():
    # The committed fixture is exactly what the generator writes.
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", Path(__file__).parent / "golden" / "make_golden.py")
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    assert module.KATS == KATS


@pytest.mark.parametrize("seed", range(3))
def test_torch_index_copy_store_equals_the_numpy_store(seed):
    # The torch form timed as the store's CPU baseline writes the same bits.
    from oracle.reference import kv_store_index_copy

    rng = np.random.default_rng(seed)
    n, h, d, pages = 37, 2, 8, 5
    key = rng.integers(-2**15, 2**15, size=(n, h, d), dtype=np.int16)
    value = rng.integers(-2**15, 2**15, size=(n, h, d), dtype=np.int16)
    slots = rng.permutation(pages * 16)[:n].astype(np.int32)
    slots[rng.random(n) < 0.2] = -1
    kc = rng.integers(-2**15, 2**15, size=(pages, 16, h, d), dtype=np.int16)
    vc = kc.copy()
    kt, vt = torch.from_numpy(kc.copy()), torch.from_numpy(vc.copy())
    kv_store(key, value, kc, vc, slots)
    kv_store_index_copy(torch.from_numpy(key), torch.from_numpy(value), kt, vt, torch.from_numpy(slots))
    assert np.array_equal(kt.numpy(), kc) and np.array_equal(vt.numpy(), vc)
