"""Paged GQA decode (DECODE route) on gfx950 vs the fp32 oracle.

Tolerance: 2e-2 absolute / 1e-2 relative of the fp32-accumulated oracle
(tests/_util.py).  Cases cover the reference's shapes (16 Q / 4 KV heads,
contexts 21 and 13), the Qwen3-0.6B decode configuration, GQA ratios 1..16,
split-K with in-launch merging, page/sequence-end edges, NaN-poisoned stale
cache rows, fp16, and repeated launches over one workspace.
"""

import pytest
import torch

import numpy as np

from my_vllm_amd import ops
from my_vllm_amd.attention_backend import (
    MI355XAttentionBackend,
    _to_device,
    make_decode_plan,
    make_decode_plan_listed,
)
from my_vllm_amd.contract import AttentionRoute, BatchType
from workloads import config_decode_small, decode_lengths, make_paged_batch
from oracle.reference import paged_attention
from tests._util import assert_attention_close, set_decode_planning

pytestmark = pytest.mark.gpu


def _to(batch, device):
    c = batch.common
    common = type(c)(**{**c.__dict__,
                        "query_start_loc": c.query_start_loc.to(device),
                        "seq_lens": c.seq_lens.to(device),
                        "slot_mapping": c.slot_mapping.to(device),
                        "block_tables": c.block_tables.to(device)})
    return common, batch.q.to(device), batch.k_cache.to(device), batch.v_cache.to(device)


def _run(batch, device, dtype=torch.bfloat16):
    hq, hkv = batch.q.shape[1], batch.k_cache.shape[2]
    backend = MI355XAttentionBackend(hq, hkv, 128, 16, dtype)
    common, q, kc, vc = _to(batch, device)
    plan = backend.build_plan(common)
    assert plan.batch_type is BatchType.PURE_DECODE and plan.route is AttentionRoute.DECODE
    empty = q.new_empty((0, hkv, 128))
    out = backend.forward(q, empty, empty, kc, vc, plan)
    assert out.shape == q.shape and out.dtype == dtype
    return out, backend, plan, (q, kc, vc, empty)


def _expected(batch):
    return paged_attention(batch.q, batch.k_cache, batch.v_cache, batch.common.block_tables,
                           batch.query_lengths, batch.kv_lengths)


def test_reference_shapes(gpu):
    batch = make_paged_batch(307, [1, 1], [21, 13], 0, 16, 4)
    out, *_ = _run(batch, gpu)
    assert_attention_close(out, _expected(batch))


@pytest.mark.parametrize("schedule", ["listed", "claims"])
def test_qwen3_0p6b_decode_configuration(gpu, monkeypatch, schedule):
    set_decode_planning(monkeypatch, schedule=schedule)
    batch = config_decode_small(seed=1)
    out, backend, plan, _ = _run(batch, gpu)
    assert (plan.metadata.decode_wave_extra is not None) == (schedule == "listed")
    assert_attention_close(out, _expected(batch))


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 8), (32, 8), (64, 8), (16, 1), (12, 3)])
def test_gqa_ratios(gpu, hq, hkv):
    ctx = decode_lengths(41, 9, 1, 700)
    batch = make_paged_batch(41, [1] * 9, ctx, 0, hq, hkv)
    out, *_ = _run(batch, gpu)
    assert_attention_close(out, _expected(batch))


@pytest.mark.parametrize("schedule", ["listed", "claims"])
@pytest.mark.parametrize("waves", [1, 7, 64, 2048, 100000])
def test_split_k_merge(gpu, monkeypatch, waves, schedule):
    # Claims: the piece length follows the wave count: 1 wave claims every
    # piece (128-page pieces) itself; 100000 waves give 4-page pieces and one
    # wavefront per piece.  Piece lists: waves / 8 page ranges (at least
    # one), down to one page per range.
    set_decode_planning(monkeypatch, waves=waves, schedule=schedule)
    ctx = [1, 16, 17, 255, 256, 257, 1000, 3001, 4096, 2049]
    batch = make_paged_batch(43, [1] * len(ctx), ctx, 0, 32, 8)
    out, backend, plan, args = _run(batch, gpu)
    assert plan.metadata.num_decode_part_slots > 0
    expected = _expected(batch)
    assert_attention_close(out, expected)
    first = out.clone()
    # The last wavefront resets the claim counters: a second launch is identical.
    q, kc, vc, empty = args
    again = backend.forward(q, empty, empty, kc, vc, plan)
    assert torch.equal(again, first)


@pytest.mark.parametrize("waves,per_wave,min_pages", [(1, 1, 1), (3, 8, 1), (64, 2, 1), (5000, 64, 1), (40, 4, 2)])
def test_piece_plans_through_c_abi(gpu, waves, per_wave, min_pages):
    # One-page pieces, one-page sequences and single-piece wavefronts exercise
    # every branch of the page stream across piece boundaries; a second launch
    # checks that the claim counters were reset.
    ctx = [1, 16, 17, 40, 1, 300, 33, 2049, 5, 640]
    hq, hkv = 32, 8
    batch = make_paged_batch(61, [1] * len(ctx), ctx, 0, hq, hkv)
    common, q, kc, vc = _to(batch, gpu)
    counts = np.asarray([(n + 15) // 16 for n in ctx])
    items, nw, slots = make_decode_plan(counts, 0, 0, hkv, waves, per_wave, min_pages)
    assert nw == min(waves, items.shape[0])
    ws = torch.zeros(ops.decode_workspace_bytes(slots, hkv, hq // hkv), dtype=torch.uint8, device=gpu)
    out = torch.full_like(q, float("nan"))
    scale = 128 ** -0.5
    merges = ops.decode_merge_list(items)
    args = (q, kc, vc, common.block_tables, common.seq_lens, _to_device(items, gpu), items.shape[0], nw,
            _to_device(merges, gpu), merges.shape[0], slots, out, ws, scale)
    ops.paged_decode(*args)
    first = out.clone()
    assert_attention_close(first, _expected(batch))
    ops.paged_decode(*args)
    assert torch.equal(out, first)
    assert int(ws[:8].view(torch.int32).abs().sum().item()) == 0


@pytest.mark.parametrize(
    "hq,hkv,groups,max_piece",
    [(32, 8, 1, 128), (32, 8, 7, 3), (32, 8, 256, 128), (16, 4, 100, 1), (8, 2, 33, 5), (8, 1, 13, 128),
     (12, 3, 50, 2), (16, 8, 100000, 128), (128, 8, 40, 7)],
)
def test_piece_lists_through_c_abi(gpu, hq, hkv, groups, max_piece):
    # Equal page ranges per workgroup (one wavefront per KV head when the
    # head count divides 8), one-page and 3-page pieces, ranges of one page,
    # one range over the whole batch; a second launch must be identical and
    # leave the claim counters untouched.
    ctx = [1, 16, 17, 40, 1, 300, 33, 2049, 5, 640]
    batch = make_paged_batch(71, [1] * len(ctx), ctx, 0, hq, hkv)
    common, q, kc, vc = _to(batch, gpu)
    counts = np.asarray([(n + 15) // 16 for n in ctx])
    items, wave_extra, nw, slots = make_decode_plan_listed(counts, 0, 0, hkv, groups, max_piece)
    per_group = hkv if hkv in (1, 2, 4, 8) else 1
    ws = torch.zeros(ops.decode_workspace_bytes(slots, hkv, hq // hkv), dtype=torch.uint8, device=gpu)
    out = torch.full_like(q, float("nan"))
    merges = ops.decode_merge_list(items)
    args = (q, kc, vc, common.block_tables, common.seq_lens, _to_device(items, gpu), items.shape[0], nw,
            _to_device(merges, gpu) if len(merges) else None, merges.shape[0], slots, out, ws, 128 ** -0.5)
    extra = _to_device(wave_extra, gpu)
    ops.paged_decode(*args, wave_extra=extra, waves_per_group=per_group)
    first = out.clone()
    assert_attention_close(first, _expected(batch))
    ops.paged_decode(*args, wave_extra=extra, waves_per_group=per_group)
    assert torch.equal(out, first)
    sched_bytes = ops.decode_workspace_bytes(0, 1, 1)  # the scheduler area alone
    assert int(ws[:sched_bytes].view(torch.int32).abs().sum().item()) == 0


def test_claim_schedule_rejects_multi_wave_groups(gpu):
    batch = make_paged_batch(73, [1, 1], [40, 7], 0, 16, 8)
    common, q, kc, vc = _to(batch, gpu)
    items, nw, slots = make_decode_plan(np.asarray([3, 1]), 0, 0, 8, 64)
    ws = torch.zeros(ops.decode_workspace_bytes(slots, 8, 2), dtype=torch.uint8, device=gpu)
    with pytest.raises(RuntimeError, match="one wavefront per workgroup"):
        ops.paged_decode(q, kc, vc, common.block_tables, common.seq_lens, _to_device(items, gpu), items.shape[0],
                         nw, None, 0, slots, torch.empty_like(q), ws, 128 ** -0.5, waves_per_group=8)


@pytest.mark.parametrize("hq,hkv", [(8, 8), (24, 8), (40, 8), (128, 8)])
def test_merge_of_one_page_pieces_for_every_group_shape(gpu, hq, hkv):
    # One-page pieces cut a 2049-token context into 129 chunks: merges with
    # more than 64 chunks and several staged batches, for G = 1, 3, 5 and 16
    # (odd G stages one spare row per batch, which must stay inside the
    # merge scratch).
    ctx = [2049, 300, 17, 1]
    batch = make_paged_batch(67, [1] * len(ctx), ctx, 0, hq, hkv)
    common, q, kc, vc = _to(batch, gpu)
    counts = np.asarray([(n + 15) // 16 for n in ctx])
    items, nw, slots = make_decode_plan(counts, 0, 0, hkv, 5000, 64, 1)
    assert int(items[:, 4].max()) == 129
    ws = torch.zeros(ops.decode_workspace_bytes(slots, hkv, hq // hkv), dtype=torch.uint8, device=gpu)
    out = torch.full_like(q, float("nan"))
    merges = ops.decode_merge_list(items)
    args = (q, kc, vc, common.block_tables, common.seq_lens, _to_device(items, gpu), items.shape[0], nw,
            _to_device(merges, gpu), merges.shape[0], slots, out, ws, 128 ** -0.5)
    ops.paged_decode(*args)
    first = out.clone()
    assert_attention_close(first, _expected(batch))
    ops.paged_decode(*args)
    assert torch.equal(out, first)


def test_stale_nan_rows_past_seq_len_do_not_leak(gpu, monkeypatch):
    set_decode_planning(monkeypatch, waves=100000)
    ctx = [5, 16, 33, 300, 129]
    batch = make_paged_batch(47, [1] * len(ctx), ctx, 0, 16, 8, extra_pages=3)
    bt = batch.common.block_tables
    for s, kv in enumerate(ctx):
        last = int(bt[s, (kv - 1) // 16])
        batch.k_cache[last, (kv - 1) % 16 + 1:] = float("nan")
        batch.v_cache[last, (kv - 1) % 16 + 1:] = float("nan")
    used = set(bt[bt >= 0].tolist())
    for p in range(batch.k_cache.shape[0]):
        if p not in used:
            batch.k_cache[p] = float("nan")
            batch.v_cache[p] = float("nan")
    out, *_ = _run(batch, gpu)
    assert_attention_close(out, _expected(batch))


def test_fp16(gpu):
    ctx = decode_lengths(53, 17, 1, 1500)
    batch = make_paged_batch(53, [1] * 17, ctx, 0, 32, 8, dtype=torch.float16)
    out, *_ = _run(batch, gpu, dtype=torch.float16)
    assert_attention_close(out, _expected(batch))


def test_one_key_context_returns_v_exactly(gpu):
    batch = make_paged_batch(59, [1, 1, 1], [1, 1, 1], 0, 16, 8)
    out, *_ = _run(batch, gpu)
    bt = batch.common.block_tables
    expected = torch.stack([batch.v_cache[int(bt[s, 0]), 0] for s in range(3)])  # [3, Hkv, D]
    expected = expected.repeat_interleave(2, dim=1)
    assert torch.equal(out.cpu(), expected)


def test_backend_supports_this_gpu(gpu):
    caps = dict(num_q_heads=16, num_kv_heads=8, head_dim=128, block_size=16, dtype=torch.bfloat16, device=gpu)
    assert MI355XAttentionBackend.support_reason(**caps) is None
    assert MI355XAttentionBackend.supports(**caps) is True


def test_one_backend_replans_many_steps_through_its_staging_ring(gpu):
    # Nine decode steps of different batches planned back to back on one
    # backend, without synchronizing: the work lists go through the
    # backend's ring of pinned staging buffers (four), each reused only after
    # its previous copy; every step's output matches the oracle.
    backend = MI355XAttentionBackend(16, 8, 128, 16, torch.bfloat16)
    steps = []
    for k in range(9):
        n = 3 + k
        batch = make_paged_batch(400 + k, [1] * n, [40 + 97 * i + 13 * k for i in range(n)], 0, 16, 8)
        common, q, kc, vc = _to(batch, gpu)
        plan = backend.build_plan(common)
        empty = q.new_empty((0, 8, 128))
        out = backend.forward(q, empty, empty, kc, vc, plan).clone()
        steps.append((batch, out))
    torch.cuda.synchronize()
    for batch, out in steps:
        assert_attention_close(out, _expected(batch))


def test_raw_op_rejects_foreign_and_mistyped_tensors(gpu):
    """The raw op refuses, before any launch, the tensors the C ABI cannot
    check: host metadata, int64 metadata, and a V cache laid out unlike K."""
    batch = make_paged_batch(62, [1, 1], [40, 17], 0, 16, 8)
    common, q, kc, vc = _to(batch, gpu)
    counts = np.asarray([3, 2])
    items, nw, slots = make_decode_plan(counts, 0, 0, 8, 4, 1, 1)
    ws = torch.zeros(ops.decode_workspace_bytes(slots, 8, 2), dtype=torch.uint8, device=gpu)
    out = torch.zeros_like(q)
    merges = ops.decode_merge_list(items)
    good = dict(q=q, k_cache=kc, v_cache=vc, block_tables=common.block_tables, seq_lens=common.seq_lens,
                items=_to_device(items, gpu), num_items=items.shape[0], num_waves=nw,
                merges=_to_device(merges, gpu), num_merges=merges.shape[0], num_part_slots=slots, out=out,
                workspace=ws, softmax_scale=128 ** -0.5)
    bad = [
        {"seq_lens": common.seq_lens.cpu()},
        {"block_tables": common.block_tables.to(torch.int64)},
        {"items": _to_device(items, gpu).t().contiguous().t()},
        {"v_cache": vc.transpose(0, 1).contiguous().transpose(0, 1)},
        {"out": out.to(torch.float16)},
    ]
    for change in bad:
        with pytest.raises((ValueError, TypeError, RuntimeError)):
            ops.paged_decode(**{**good, **change})
    ops.paged_decode(**good)
    assert_attention_close(out, _expected(batch))
