"""MIXED batches: single-launch (MIXED_UNIFIED) and split (MIXED_SPLIT) routes.

Both routes run the same prefill code, so the prefill rows must be bitwise
identical; the split route's decode half runs the piece-list schedule (a
different split-K partition than the single launch's claims), so decode
rows agree within the attention tolerance.  Both are checked against the
fp32 oracle (2e-2 / 1e-2).
The split route writes ``out[:P]`` and ``out[P:]`` of one buffer without
concatenation.  GQA ratios 1, 3 and 8 and fp16 run on both routes.
"""

import pytest
import torch

from my_vllm_amd.contract import AttentionRoute
from my_vllm_amd.contract import BatchType
from workloads import config_mixed, make_paged_batch
from tests._util import assert_attention_close, set_decode_planning
from tests.test_gpu_prefill import expected, run_backend

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("waves", ["3", "2048", "100000"])
def test_mixed_unified_and_split_match(gpu, monkeypatch, waves):
    set_decode_planning(monkeypatch, waves=waves)
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


@pytest.mark.parametrize("mode", ["unified", "split"])
@pytest.mark.parametrize("hq,hkv", [(8, 8), (12, 4), (64, 8), (6, 3), (16, 1)])
def test_mixed_gqa_ratios(gpu, mode, hq, hkv):
    # G = 1, 3, 8, 2 and 16: the prefill tile of one launch holds 128 // G
    # tokens of every query head of a KV head; decode wavefronts cover G heads
    # each.  3 and 1 KV heads give prefill pools that are not a multiple of
    # the 8 XCDs.
    batch = make_paged_batch(97, [70, 33, 1, 1, 1], [70, 290, 9, 700, 2100], 2, hq, hkv)
    out, plan = run_backend(batch, gpu, mode=mode)
    assert plan.batch_type is BatchType.MIXED
    assert_attention_close(out, expected(batch))


@pytest.mark.parametrize("mode", ["unified", "split"])
def test_mixed_fp16(gpu, mode):
    batch = make_paged_batch(101, [40, 1, 1], [57, 333, 1200], 1, 32, 8, dtype=torch.float16)
    out, _ = run_backend(batch, gpu, dtype=torch.float16, mode=mode)
    assert out.dtype == torch.float16
    assert_attention_close(out, expected(batch))


@pytest.mark.parametrize("mode", ["unified", "split"])
@pytest.mark.parametrize("case", range(3))
def test_reference_numeric_cases(gpu, mode, case):
    # The reference's paged pure/MIXED numeric cases
    # (tests/test_attention_backend.py:367-418): Hq=16, Hkv=4, seeds 307+i,
    # both attention modes; case 2 is its MIXED batch ((5, 1), (21, 13), 1).
    q_lens, kv_lens, num_prefill = [((5, 3), (21, 13), 2), ((1, 1), (21, 13), 0), ((5, 1), (21, 13), 1)][case]
    batch = make_paged_batch(307 + case, list(q_lens), list(kv_lens), num_prefill, 16, 4)
    out, plan = run_backend(batch, gpu, mode=mode)
    route = {0: AttentionRoute.PREFILL, 1: AttentionRoute.DECODE,
             2: AttentionRoute.MIXED_UNIFIED if mode == "unified" else AttentionRoute.MIXED_SPLIT}[case]
    assert plan.route is route
    assert out.shape == batch.q.shape and out.dtype == torch.bfloat16
    assert_attention_close(out, expected(batch))


def test_mixed_many_prefill_sequences_device_tiles(gpu):
    # 150 prefill sequences: the single launch orders their tiles on the
    # device across several 64-sequence scan chunks, sequences with equal
    # contexts included; prefill rows match the split route bit for bit.
    import numpy as np

    rng = np.random.default_rng(17)
    q = [int(x) for x in rng.integers(1, 40, size=150)]
    kv = [n + int(rng.choice([0, 16, 37, 200])) for n in q]
    q += [1] * 20
    kv += [int(x) for x in rng.integers(1, 600, size=20)]
    batch = make_paged_batch(97, q, kv, 150, 16, 4)
    out_u, plan_u = run_backend(batch, gpu, mode="unified")
    out_u = out_u.clone()
    assert plan_u.route is AttentionRoute.MIXED_UNIFIED and plan_u.metadata.mixed_prefill_max_tiles > 0
    out_s, _ = run_backend(batch, gpu, mode="split")
    rows = sum(q[:150])
    assert torch.equal(out_u[:rows], out_s[:rows])
    assert_attention_close(out_u, expected(batch))


def test_mixed_launch_leaves_its_counters_clear(gpu):
    # The prefill pool's claim and exit counters (and the decode claims) are
    # back at zero after every launch, so the next launch on the same
    # workspace starts from tile 0.
    from my_vllm_amd import ops
    from my_vllm_amd.attention_backend import MI355XAttentionBackend
    from tests.test_gpu_prefill import to_device

    batch = make_paged_batch(101, [70, 300, 1, 1, 1], [70, 900, 40, 700, 2000], 2, 32, 8)
    backend = MI355XAttentionBackend(32, 8, 128, 16, torch.bfloat16)
    common, qd, kc, vc = to_device(batch, gpu)
    plan = backend.build_plan(common)
    empty = qd.new_empty((0, 8, 128))
    first = backend.forward(qd, empty, empty, kc, vc, plan).clone()
    again = backend.forward(qd, empty, empty, kc, vc, plan)
    torch.cuda.synchronize()
    assert torch.equal(first, again)
    sched = ops.decode_workspace_bytes(0, 1, 1)
    assert int(backend._workspace[:sched].view(torch.int32).abs().sum().item()) == 0
    assert_attention_close(again, expected(batch))


def test_mixed_in_launch_merges_flush_a_long_list(gpu, monkeypatch):
    # One decode wavefront runs 640 split pieces (40 sequences x 8 KV heads x
    # 2 chunks): its list of pieces awaiting arrival fills (64 entries) and
    # is flushed ten times; every segment is still merged exactly once.
    set_decode_planning(monkeypatch, waves=1)
    q = [40] + [1] * 40
    kv = [300] + [2080] * 40
    batch = make_paged_batch(103, q, kv, 1, 16, 8)
    out, plan = run_backend(batch, gpu)
    assert plan.route is AttentionRoute.MIXED_UNIFIED
    assert plan.metadata.num_decode_items == 640 and plan.metadata.num_decode_merges == 0
    assert_attention_close(out, expected(batch))


def test_mixed_beyond_one_launch_runs_prefill_then_decode(gpu):
    # More prefill sequences than one MIXED launch orders (1024): the unified
    # backend plans MIXED_SPLIT, says why, and runs prefill + decode launches
    # (reference attention_backend.py:626-663, 858-890).
    from my_vllm_amd import ops
    from my_vllm_amd.attention_backend import MI355XAttentionBackend
    from tests.test_gpu_prefill import to_device

    n = ops.MIXED_PREFILL_SEQS_MAX + 3
    q = [2] * n + [1, 1]
    kv = [9] * n + [300, 40]
    batch = make_paged_batch(107, q, kv, n, 16, 8)
    backend = MI355XAttentionBackend(16, 8, 128, 16, torch.bfloat16)
    common, qd, kc, vc = to_device(batch, gpu)
    plan = backend.build_plan(common)
    assert plan.route is AttentionRoute.MIXED_SPLIT and plan.metadata.mixed_prefill_max_tiles == 0
    assert backend.mixed_attention_available is False
    assert f"at most {ops.MIXED_PREFILL_SEQS_MAX} prefill sequences" in backend.mixed_attention_unavailable_reason
    assert dict(backend.route_counts)["mixed_split"] == 1 and dict(backend.route_counts)["mixed_unified"] == 0
    empty = qd.new_empty((0, 8, 128))
    out = backend.forward(qd, empty, empty, kc, vc, plan)
    assert_attention_close(out, expected(batch))
    # A batch within the limits on the same backend runs as one launch again.
    small = make_paged_batch(108, [5, 1], [21, 13], 1, 16, 8)
    common, qd, kc, vc = to_device(small, gpu)
    plan = backend.build_plan(common)
    assert plan.route is AttentionRoute.MIXED_UNIFIED and backend.mixed_attention_available
    assert backend.mixed_attention_unavailable_reason is None
    assert_attention_close(backend.forward(qd, empty, empty, kc, vc, plan), expected(small))


def test_mixed_after_decode_steps_on_one_workspace(gpu, monkeypatch):
    # A decode step with many split-K partial slots, then MIXED steps with
    # fewer, then a decode step, all on one backend and workspace: the MIXED
    # launch's arrival counters must not see the earlier partials, and every
    # step matches the oracle.
    from my_vllm_amd.attention_backend import MI355XAttentionBackend
    from tests.test_gpu_prefill import to_device

    backend = MI355XAttentionBackend(32, 8, 128, 16, torch.bfloat16)
    batches = [
        make_paged_batch(111, [1] * 40, [1500 + 37 * i for i in range(40)], 0, 32, 8),
        make_paged_batch(112, [30, 1, 1, 1], [300, 900, 2100, 40], 1, 32, 8),
        make_paged_batch(113, [7, 20, 1, 1], [7, 500, 3000, 1000], 2, 32, 8),
        make_paged_batch(114, [1] * 12, [800 + 90 * i for i in range(12)], 0, 32, 8),
    ]
    for b in batches:
        # Default decode planning (many ranges, many partial slots); few
        # decode wavefronts in the MIXED launches (few partial slots).
        if b.common.num_prefill_seqs:
            set_decode_planning(monkeypatch, waves=64)
        else:
            set_decode_planning(monkeypatch)
        common, qd, kc, vc = to_device(b, gpu)
        plan = backend.build_plan(common)
        empty = qd.new_empty((0, 8, 128))
        out = backend.forward(qd, empty, empty, kc, vc, plan)
        assert_attention_close(out, expected(b))


def test_many_launches_keep_the_counters_consistent(gpu):
    # 120 back-to-back launches on one backend: MIXED (prefill pool claims,
    # in-launch merges), DECODE (claim counters, merge kernel) and PREFILL in
    # turn; the counters each launch leaves at zero are what the next one
    # starts from, so every output must stay equal to its first.
    from my_vllm_amd.attention_backend import MI355XAttentionBackend
    from tests.test_gpu_prefill import to_device

    backend = MI355XAttentionBackend(32, 8, 128, 16, torch.bfloat16)
    batches = [
        make_paged_batch(121, [64, 9, 1, 1, 1], [300, 9, 1500, 40, 2600], 2, 32, 8),
        make_paged_batch(122, [1] * 20, [100 + 150 * i for i in range(20)], 0, 32, 8),
        make_paged_batch(123, [200, 31], [700, 31], 2, 32, 8),
    ]
    steps = []
    for b in batches:
        common, qd, kc, vc = to_device(b, gpu)
        plan = backend.build_plan(common)
        steps.append((qd, kc, vc, plan))
    empty = steps[0][0].new_empty((0, 8, 128))
    firsts = [backend.forward(qd, empty, empty, kc, vc, plan).clone() for qd, kc, vc, plan in steps]
    for i in range(120):
        qd, kc, vc, plan = steps[i % 3]
        out = backend.forward(qd, empty, empty, kc, vc, plan)
        if i % 30 < 3:
            assert torch.equal(out, firsts[i % 3]), f"launch {i} differs"
    for b, first in zip(batches, firsts):
        assert_attention_close(first, expected(b))


def test_mixed_untrusted_metadata_matches_trusted(gpu):
    # The untrusted path validates the metadata on the device side first;
    # the launch itself is the same, so the rows are bit-identical.
    batch = make_paged_batch(125, [40, 300, 1, 1], [100, 300, 70, 900], 2, 32, 8)
    a, _ = run_backend(batch, gpu, trusted=True)
    a = a.clone()
    b, plan = run_backend(batch, gpu, trusted=False)
    assert plan.route is AttentionRoute.MIXED_UNIFIED
    assert torch.equal(a, b)


def test_mixed_output_only_8_byte_aligned_matches_aligned(gpu):
    # The single launch's prefill rows are stored 16 bytes per lane when the
    # output and its strides are 16-byte aligned and 8 bytes otherwise; an
    # output view 8 bytes past an aligned buffer takes the second path and
    # must give the same bits (its decode rows as well).
    from my_vllm_amd import ops
    from my_vllm_amd.attention_backend import MI355XAttentionBackend
    from tests.test_gpu_prefill import to_device

    batch = make_paged_batch(157, [70, 300, 1, 1, 1], [70, 900, 40, 700, 2000], 2, 32, 8)
    backend = MI355XAttentionBackend(32, 8, 128, 16, torch.bfloat16)
    common, qd, kc, vc = to_device(batch, gpu)
    plan = backend.build_plan(common)
    assert plan.route is AttentionRoute.MIXED_UNIFIED
    md = plan.metadata
    ws = backend._get_workspace(ops.decode_workspace_bytes(md.num_decode_part_slots, 8, 4), qd.device)
    outs = []
    for shift in (0, 4):
        flat = torch.full((qd.numel() + 8,), float("nan"), dtype=qd.dtype, device=gpu)
        out = flat[shift:shift + qd.numel()].view(qd.shape)
        assert (out.data_ptr() % 16 == 0) == (shift == 0)
        ops.paged_mixed(qd, kc, vc, md.block_tables, md.seq_lens, md.query_start_loc, common.num_prefill_seqs,
                        md.mixed_prefill_max_tiles, md.decode_items, md.num_decode_items, md.num_decode_waves,
                        md.num_decode_part_slots, out, ws, backend.softmax_scale)
        outs.append(out.clone())
    assert torch.equal(outs[0], outs[1])
    assert_attention_close(outs[0], expected(batch))
