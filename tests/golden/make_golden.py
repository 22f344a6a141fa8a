"""Writes tests/golden/reference_kats.json: known-answer vectors of the hot path.

The values are the literal inputs and expected outputs of the reference's own
tests (transcribed, with file:line citations); nothing from the reference is
imported or executed.  Run from the repository root:

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
from pathlib import Path

KATS = {
    # tests/test_custom_op_dispatch.py:75-95 (KVCacheStore ignores negative slots)
    "kv_store": {
        "source": "tests/test_custom_op_dispatch.py:75-95",
        "key": {"arange_from": 1, "arange_to": 25, "shape": [3, 2, 4]},
        "value_offset": 100,
        "cache_shape": [2, 2, 2, 4],
        "cache_fill": -1.0,
        "slot_mapping": [3, -1, 0],
        # flattened cache row <- token
        "writes": [[3, 0], [0, 2]],
    },
    # tests/test_attention_backend.py:280-299 with _phase_case (:596-641):
    # q (5, 1), kv (21, 13), one prefill sequence, pages numbered in order.
    "page_csr": {
        "source": "tests/test_attention_backend.py:280-299, :596-641",
        "query_lengths": [5, 1],
        "kv_lengths": [21, 13],
        "num_prefill_seqs": 1,
        "block_tables": [[0, 1], [2, -1]],
        "kv_indptr": [0, 2, 3],
        "page_indices": [0, 1, 2],
        "last_page_len": [5, 13],
        "num_pages": 3,
        "num_prefill_pages": 2,
    },
    # tests/test_attention_registry.py:311-328 (MIXED_SPLIT slices the CSR:
    # prefill plan gets qo_indptr, kv_indptr, page_indices, last_page_len;
    # decode plan gets kv_indptr re-based to the decode pages).
    "split_csr": {
        "source": "tests/test_attention_registry.py:311-328",
        "query_lengths": [5, 1],
        "kv_lengths": [21, 13],
        "num_prefill_seqs": 1,
        "prefill": {"qo_indptr": [0, 5], "kv_indptr": [0, 2], "page_indices": [0, 1], "last_page_len": [5]},
        "decode": {"kv_indptr": [0, 1], "page_indices": [2], "last_page_len": [13]},
    },
    # tests/test_attention_registry.py:36-54 (CommonAttentionMetadata totals)
    "common_totals": {
        "source": "tests/test_attention_registry.py:36-54",
        "query_lengths": [5, 1, 1],
        "kv_lengths": [21, 13, 18],
        "num_prefill_seqs": 1,
        "num_prefill_tokens": 5,
        "num_decode_tokens": 2,
        "num_seqs": 3,
        "num_query_tokens": 7,
        "query_start_loc": [0, 5, 6, 7],
        "block_counts": [2, 1, 2],
        "max_q_len": 5,
        "max_kv_len": 21,
    },
    # tests/test_model_runner_metadata.py slot_mapping / seq_lens cases:
    # each sequence is (block_table, num_cached_tokens, num_context_tokens).
    "slot_mapping": [
        {
            "source": "tests/test_model_runner_metadata.py:138-187",
            "sequences": [[[7, 4], 16, 19], [[9], 0, 5]],
            "query_start_loc": [0, 3, 8],
            "seq_lens": [19, 5],
            "slot_mapping": [64, 65, 66, 144, 145, 146, 147, 148],
            "block_tables": [[7, 4], [9, -1]],
            "block_counts": [2, 1],
        },
        {
            "source": "tests/test_model_runner_metadata.py:219-255",
            "sequences": [[[2], 0, 3], [[4, 5], 17, 18]],
            "query_start_loc": [0, 3, 4],
            "seq_lens": [3, 18],
            "slot_mapping": [32, 33, 34, 81],
            "block_tables": [[2, -1], [4, 5]],
            "block_counts": [1, 2],
        },
        {
            "source": "tests/test_model_runner_metadata.py:311-349",
            "sequences": [[[3, 4], 16, 17]],
            "query_start_loc": [0, 1],
            "seq_lens": [17],
            "slot_mapping": [64],
            "block_tables": [[3, 4]],
            "block_counts": [2],
        },
    ],
    # tests/test_model_runner_metadata.py:48-87 and :351-374 (classification):
    # (num_prefill_seqs, num_decode_seqs) -> batch type
    "classify": {
        "source": "tests/test_model_runner_metadata.py:48-87, :351-374",
        "cases": [[2, 0, "pure_prefill"], [0, 2, "pure_decode"], [1, 1, "mixed"]],
    },
    # tests/test_custom_cuda_silu.py:30-31 shapes and :53-66 error messages
    "silu": {
        "source": "tests/test_custom_cuda_silu.py:30-31, :53-66",
        "shapes": [[18], [31, 64], [2, 3, 14], [0, 16]],
        "errors": {
            "cpu": "CUDA",
            "non_contiguous": "contiguous",
            "scalar": "at least one dimension",
            "dtype": "only supports float16 and bfloat16",
            "odd": "positive even number",
        },
    },
}


def main() -> None:
    out = Path(__file__).resolve().parent / "reference_kats.json"
    out.write_text(json.dumps(KATS, indent=1) + "\n")
    print(f"wrote {out}")


if __name__ == "__main__":
    main()
