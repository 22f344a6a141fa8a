"""Full-decode HIP graph: capture once, replay over different decode batches.

Mirrors the reference's capture/replay flow (nanovllm/engine/model_runner.py:
631-742: plan the capture batch, activate the state, capture, then per step
``plan_full_decode_graph`` + replay).  Every replay is checked against the
fp32 oracle (2e-2 abs / 1e-2 rel) and bit-for-bit against the eager decode
path, with eager work and synchronizations between replays.
"""

import pytest
import torch

from my_vllm_amd.attention_backend import MI355XAttentionBackend
from my_vllm_amd.contract import AttentionRoute
from my_vllm_amd.contract import CommonAttentionMetadata
from workloads import decode_lengths, make_paged_batch
from oracle.reference import paged_attention
from tests._util import assert_attention_close

pytestmark = pytest.mark.gpu


def _on(common, device):
    return type(common)(**{**common.__dict__,
                           "query_start_loc": common.query_start_loc.to(device),
                           "seq_lens": common.seq_lens.to(device),
                           "slot_mapping": common.slot_mapping.to(device),
                           "block_tables": common.block_tables.to(device)})


@pytest.mark.parametrize("hq,hkv,batch,width", [(16, 8, 6, 160), (32, 8, 33, 40), (8, 2, 3, 300), (12, 3, 4, 64)])
def test_decode_graph_replays_match_eager_and_oracle(gpu, hq, hkv, batch, width):
    backend = MI355XAttentionBackend(hq, hkv, 128, 16, torch.bfloat16)
    pages = batch * width
    state = backend.create_full_decode_graph_state(batch, pages, gpu)
    k_cache = torch.zeros(pages, 16, hkv, 128, dtype=torch.bfloat16, device=gpu)
    v_cache = torch.zeros_like(k_cache)
    q_static = torch.zeros(batch, hq, 128, dtype=torch.bfloat16, device=gpu)
    empty = q_static.new_empty((0, hkv, 128))

    # Capture batch as the model runner builds it: one page each, page 0.
    capture = CommonAttentionMetadata(
        num_prefill_seqs=0, num_decode_seqs=batch, num_prefill_tokens=0, num_decode_tokens=batch,
        query_start_loc=torch.arange(batch + 1, dtype=torch.int32, device=gpu),
        seq_lens=torch.ones(batch, dtype=torch.int32, device=gpu),
        slot_mapping=torch.full((batch,), -1, dtype=torch.int32, device=gpu),
        block_tables=torch.zeros((batch, 1), dtype=torch.int32, device=gpu),
        max_q_len=1, max_kv_len=1, block_counts=(1,) * batch, num_kv_blocks=batch, num_prefill_kv_blocks=0,
        trusted=True)
    plan = backend.build_plan(capture)
    backend.plan_full_decode_graph(state, plan)
    backend.activate_full_decode_graph(state)
    try:
        out = backend.forward(q_static, empty, empty, k_cache, v_cache, plan)
        assert out.data_ptr() == state.output.data_ptr()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            backend.forward(q_static, empty, empty, k_cache, v_cache, plan)
        torch.cuda.synchronize()
    finally:
        backend.deactivate_full_decode_graph()

    for step, seed in enumerate((11, 12, 13, 14)):
        # Contexts up to the per-request page capacity, incl. one-page and full rows.
        ctx = decode_lengths(seed, batch, 1, width * 16)
        ctx[0] = width * 16
        ctx[-1] = 1
        b = make_paged_batch(seed, [1] * batch, ctx, 0, hq, hkv)
        common = _on(b.common, gpu)
        k_cache.zero_()
        v_cache.zero_()
        k_cache[: b.k_cache.shape[0]].copy_(b.k_cache)
        v_cache[: b.v_cache.shape[0]].copy_(b.v_cache)
        q_static.copy_(b.q)
        step_plan = backend.build_plan(common)
        assert step_plan.route is AttentionRoute.DECODE
        assert backend.full_decode_graph_metadata_fits(state, step_plan)
        backend.plan_full_decode_graph(state, step_plan)
        graph.replay()
        got = state.output.clone()
        torch.cuda.synchronize()
        # Eager work between replays.
        x = torch.randn(256, 256, device=gpu)
        (x @ x).sum().item()
        eager = backend.forward(q_static, empty, empty, k_cache, v_cache, step_plan)
        assert torch.equal(got, eager), f"replay {step} differs from the eager launch"
        expected = paged_attention(b.q, b.k_cache, b.v_cache, b.common.block_tables, [1] * batch, ctx)
        assert_attention_close(got, expected)


def test_decode_graph_state_rejects_plans_that_do_not_fit(gpu):
    backend = MI355XAttentionBackend(16, 8, 128, 16, torch.bfloat16)
    state = backend.create_full_decode_graph_state(4, 4 * 8, gpu)
    wrong_batch = make_paged_batch(3, [1] * 3, [5, 9, 30], 0, 16, 8)
    assert not backend.full_decode_graph_metadata_fits(state, backend.build_plan(_on(wrong_batch.common, gpu)))
    too_long = make_paged_batch(4, [1] * 4, [5, 9, 30, 16 * 8 + 1], 0, 16, 8)
    assert not backend.full_decode_graph_metadata_fits(state, backend.build_plan(_on(too_long.common, gpu)))
    mixed = make_paged_batch(5, [3, 1, 1, 1], [20, 9, 30, 7], 1, 16, 8)
    assert not backend.full_decode_graph_metadata_fits(state, backend.build_plan(_on(mixed.common, gpu)))
    ok = make_paged_batch(6, [1] * 4, [5, 9, 30, 128], 0, 16, 8)
    assert backend.full_decode_graph_metadata_fits(state, backend.build_plan(_on(ok.common, gpu)))
    with pytest.raises(RuntimeError, match="planned before activation"):
        backend.activate_full_decode_graph(backend.create_full_decode_graph_state(4, 32, gpu))
