"""MIXED batches: single-launch (MIXED_UNIFIED) and split (MIXED_SPLIT) routes.

Both routes run the same prefill code, so the prefill rows must be bitwise
identical; the split route's decode half runs the piece-list schedule (a
different split-K partition than the single launch's claims), so decode
rows agree within the attention tolerance.  Both are checked against the
fp32 oracle (2e-2 / 1e-2).
The split route writes ``out[:P]`` and ``out[P:]`` of one buffer without
concatenation.
"""

import pytest
import torch

from my_vllm_amd.attention_backend import AttentionRoute
from my_vllm_amd.context import BatchType
from my_vllm_amd.workloads import config_mixed, make_paged_batch
from tests._util import assert_attention_close
from tests.test_gpu_prefill import expected, run_backend

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("waves", ["3", "2048", "100000"])
def test_mixed_unified_and_split_match(gpu, monkeypatch, waves):
    monkeypatch.setenv("MVA_DECODE_WAVES", waves)
    q = [5, 130, 1, 1, 1, 1]
    kv = [21, 400, 13, 18, 1500, 3000]
    batch = make_paged_batch(83, q, kv, 2, 32, 8)
    out_u, plan_u = run_backend(batch, gpu, mode="unified")
    out_u = out_u.clone()
    out_s, plan_s = run_backend(batch, gpu, mode="split")
    assert plan_u.batch_type is BatchType.MIXED and plan_u.route is AttentionRoute.MIXED_UNIFIED
    assert plan_s.route is AttentionRoute.MIXED_SPLIT
    prefill_rows = sum(q[:2])
    assert torch.equal(out_u[:prefill_rows], out_s[:prefill_rows])
    torch.testing.assert_close(out_u.float(), out_s.float(), atol=2e-2, rtol=1e-2)
    ref = expected(batch)
    assert_attention_close(out_u, ref)
    assert_attention_close(out_s, ref)


def test_all_single_token_mixed_batch(gpu):
    # A prefill sequence with q == 1 stays on the prefill path (reference
    # tests/test_model_runner_metadata.py:351-374).
    batch = make_paged_batch(89, [1, 1], [1, 17], 1, 16, 8)
    out, plan = run_backend(batch, gpu)
    assert plan.batch_type is BatchType.MIXED
    assert_attention_close(out, expected(batch))


def test_qwen3_8b_mixed_configuration(gpu):
    batch = config_mixed(seed=3)
    out, plan = run_backend(batch, gpu)
    assert plan.route is AttentionRoute.MIXED_UNIFIED
    seqs = [0, 1, 2, 3, 4, 100, 259]
    exp, rows = expected(batch, seqs)
    assert_attention_close(out.cpu()[rows], exp)
