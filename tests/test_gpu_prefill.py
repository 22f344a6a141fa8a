"""Ragged causal chunked prefill (PREFILL route) on gfx950 vs the fp32 oracle.

Tolerance 2e-2 absolute / 1e-2 relative (tests/_util.py).  Cases: the
reference's shapes, the Qwen3-8B prefill-with-prefix configuration (a subset
of its sequences is checked on the CPU), GQA ratios 1..16 including 3, a
single-token chunk with a long context, unaligned prefixes, NaN-poisoned
stale rows, fp16, trusted vs untrusted metadata, and the cacheless warmup.
"""

import dataclasses

import pytest
import torch

from my_vllm_amd import ops
from my_vllm_amd.attention_backend import MI355XAttentionBackend
from my_vllm_amd.contract import AttentionRoute
from my_vllm_amd.contract import BatchType
from workloads import config_prefill, make_paged_batch
from oracle.reference import paged_attention, ragged_attention
from tests._util import assert_attention_close

pytestmark = pytest.mark.gpu


def to_device(batch, device, trusted=True):
    c = batch.common
    common = type(c)(**{**c.__dict__,
                        "query_start_loc": c.query_start_loc.to(device),
                        "seq_lens": c.seq_lens.to(device),
                        "slot_mapping": c.slot_mapping.to(device),
                        "block_tables": c.block_tables.to(device),
                        "trusted": trusted})
    return common, batch.q.to(device), batch.k_cache.to(device), batch.v_cache.to(device)


def run_backend(batch, device, dtype=torch.bfloat16, trusted=True, mode="unified"):
    hq, hkv = batch.q.shape[1], batch.k_cache.shape[2]
    backend = MI355XAttentionBackend(hq, hkv, 128, 16, dtype, attention_mode=mode)
    common, q, kc, vc = to_device(batch, device, trusted)
    plan = backend.build_plan(common)
    empty = q.new_empty((0, hkv, 128))
    out = backend.forward(q, empty, empty, kc, vc, plan)
    assert out.shape == q.shape and out.dtype == dtype
    return out, plan


def expected(batch, seqs=None):
    if seqs is None:
        return paged_attention(batch.q, batch.k_cache, batch.v_cache, batch.common.block_tables,
                               batch.query_lengths, batch.kv_lengths)
    rows, parts = [], []
    starts = [0]
    for n in batch.query_lengths:
        starts.append(starts[-1] + n)
    for s in seqs:
        bt = batch.common.block_tables[s:s + 1]
        q = batch.q[starts[s]:starts[s + 1]]
        parts.append(paged_attention(q, batch.k_cache, batch.v_cache, bt,
                                     [batch.query_lengths[s]], [batch.kv_lengths[s]]))
        rows.extend(range(starts[s], starts[s + 1]))
    return torch.cat(parts), rows


def test_reference_shapes(gpu):
    batch = make_paged_batch(307, [5, 3], [21, 13], 2, 16, 4)
    out, plan = run_backend(batch, gpu)
    assert plan.batch_type is BatchType.PURE_PREFILL and plan.route is AttentionRoute.PREFILL
    assert_attention_close(out, expected(batch))


def test_qwen3_8b_prefill_with_prefix_configuration(gpu):
    batch = config_prefill(seed=2)
    out, _ = run_backend(batch, gpu)
    longest = max(range(16), key=lambda s: batch.kv_lengths[s])
    seqs = sorted({0, 7, 15, longest})
    exp, rows = expected(batch, seqs)
    assert_attention_close(out.cpu()[rows], exp)


# (80, 80): more KV heads than a wavefront has lanes, so a workgroup whose
# own queue is exhausted reads the other heads' claim counters in two rounds.
@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 8), (32, 8), (64, 8), (128, 8), (12, 4), (16, 1), (80, 80)])
def test_gqa_ratios(gpu, hq, hkv):
    q = [1, 37, 130, 64]
    kv = [1, 37 + 16 * 3, 130 + 5, 64 + 200]
    batch = make_paged_batch(61, q, kv, 4, hq, hkv)
    out, _ = run_backend(batch, gpu)
    assert_attention_close(out, expected(batch))


def test_edge_lengths(gpu):
    # single-token chunk over a long context, unaligned prefixes, exact tile
    # and page multiples, q == kv (no prefix)
    q = [1, 7, 32, 33, 96, 257, 64, 500]
    kv = [2049, 7, 32 + 16, 33 + 1, 96 + 63, 257 + 1000, 64 + 64, 500 + 17]
    batch = make_paged_batch(67, q, kv, len(q), 32, 8)
    out, _ = run_backend(batch, gpu)
    assert_attention_close(out, expected(batch))


def test_untrusted_metadata_matches_trusted(gpu):
    batch = make_paged_batch(71, [40, 300, 3], [100, 300, 70], 3, 32, 8)
    a, _ = run_backend(batch, gpu, trusted=True)
    a = a.clone()
    b, _ = run_backend(batch, gpu, trusted=False)
    assert torch.equal(a, b)
    assert_attention_close(b, expected(batch))


def test_stale_nan_rows_past_seq_len_do_not_leak(gpu):
    q = [20, 70, 5]
    kv = [40, 75, 150]
    batch = make_paged_batch(73, q, kv, 3, 16, 8, extra_pages=2)
    bt = batch.common.block_tables
    for s, n in enumerate(kv):
        last = int(bt[s, (n - 1) // 16])
        batch.k_cache[last, (n - 1) % 16 + 1:] = float("nan")
        batch.v_cache[last, (n - 1) % 16 + 1:] = float("nan")
    used = set(bt[bt >= 0].tolist())
    for p in range(batch.k_cache.shape[0]):
        if p not in used:
            batch.k_cache[p] = float("nan")
            batch.v_cache[p] = float("nan")
    out, _ = run_backend(batch, gpu)
    assert_attention_close(out, expected(batch))


def test_fp16(gpu):
    batch = make_paged_batch(79, [100, 17], [180, 17], 2, 32, 8, dtype=torch.float16)
    out, _ = run_backend(batch, gpu, dtype=torch.float16)
    assert_attention_close(out, expected(batch))


def test_cacheless_warmup_route(gpu):
    torch.manual_seed(223)
    lengths = [3, 1]
    q = torch.randn(4, 16, 128).bfloat16()
    k = torch.randn(4, 4, 128).bfloat16()
    v = torch.randn(4, 4, 128).bfloat16()
    from my_vllm_amd.contract import CommonAttentionMetadata

    common = CommonAttentionMetadata(
        num_prefill_seqs=2, num_decode_seqs=0, num_prefill_tokens=4, num_decode_tokens=0,
        query_start_loc=torch.tensor([0, 3, 4], dtype=torch.int32, device=gpu),
        seq_lens=torch.tensor(lengths, dtype=torch.int32, device=gpu),
        slot_mapping=torch.full((4,), -1, dtype=torch.int32, device=gpu),
        block_tables=None, max_q_len=3, max_kv_len=3, trusted=True)
    backend = MI355XAttentionBackend(16, 4, 128, 16, torch.bfloat16)
    plan = backend.build_plan(common)
    assert plan.route is AttentionRoute.WARMUP
    empty = torch.empty(0, device=gpu)
    out = backend.forward(q.to(gpu), k.to(gpu), v.to(gpu), empty, empty, plan)
    assert_attention_close(out, ragged_attention(q, k, v, lengths))


@pytest.mark.parametrize("lengths,hq,hkv", [([1, 15, 16, 17, 300], 32, 8), ([2049, 5], 16, 4), ([64], 8, 8), ([33, 1, 1], 16, 1)])
def test_cacheless_warmup_runs_the_prefill_kernel(gpu, lengths, hq, hkv):
    from my_vllm_amd.contract import CommonAttentionMetadata

    g = torch.Generator().manual_seed(sum(lengths) + hq)
    total = sum(lengths)
    q = torch.randn(total, hq, 128, generator=g).bfloat16()
    kv = torch.randn(total, 2 * hkv, 128, generator=g).bfloat16()  # packed k|v: strided views
    k, v = kv[:, :hkv], kv[:, hkv:]
    qsl = [0]
    for n in lengths:
        qsl.append(qsl[-1] + n)
    common = CommonAttentionMetadata(
        num_prefill_seqs=len(lengths), num_decode_seqs=0, num_prefill_tokens=total, num_decode_tokens=0,
        query_start_loc=torch.tensor(qsl, dtype=torch.int32, device=gpu),
        seq_lens=torch.tensor(lengths, dtype=torch.int32, device=gpu),
        slot_mapping=torch.full((total,), -1, dtype=torch.int32, device=gpu),
        block_tables=None, max_q_len=max(lengths), max_kv_len=max(lengths), trusted=True)
    backend = MI355XAttentionBackend(hq, hkv, 128, 16, torch.bfloat16)
    plan = backend.build_plan(common)
    assert plan.route is AttentionRoute.WARMUP
    empty = torch.empty(0, device=gpu)
    kvd = kv.to(gpu)
    out = backend.forward(q.to(gpu), kvd[:, :hkv], kvd[:, hkv:], empty, empty, plan)
    assert out.data_ptr() == backend._get_reusable_attention_output(q.to(gpu)).data_ptr()
    assert_attention_close(out, ragged_attention(q, k.contiguous(), v.contiguous(), lengths))


def _expected_tiles(q_lens, kv_lens, tile, tail=0):
    """The tile list the device planner must write: sequences by context
    length (longest first, ties by index), each sequence's tiles by key count
    (largest first), then the last ``tail`` tiles (at most 1024) by key count
    (largest first, ties in order), as {seq, t0, q0, q_len, kv, ntiles, full,
    npages} and the page-table slots of the first two 64-key tiles' 8 pages
    (clamped to the last needed page)."""
    starts = [0]
    for n in q_lens:
        starts.append(starts[-1] + n)
    rows = []
    for s in sorted(range(len(q_lens)), key=lambda i: (-kv_lens[i], i)):
        q, kv = q_lens[s], kv_lens[s]
        if q <= 0 or kv < q:
            continue
        nt = -(-q // tile)
        for j in range(nt):
            t0 = (nt - 1 - j) * tile
            kv_end = kv - q + min(t0 + tile, q)
            ntiles = -(-kv_end // 64)
            npages = -(-kv_end // 16)
            rows.append([s, t0, starts[s], q, kv, ntiles, min((kv - q + t0 + 1) // 64, ntiles), npages]
                        + [min(i, npages - 1) for i in range(8)])
    k = min(len(rows), tail, 1024)
    if k > 1:
        rows = rows[:-k] + sorted(rows[-k:], key=lambda r: -r[5])  # stable: ties keep their order
    return rows


@pytest.mark.parametrize("hq,hkv", [(32, 8), (16, 1), (12, 4)])
def test_device_tile_plan_is_exact(gpu, hq, hkv):
    # Exact tiles from the device's query offsets: no tile past a sequence's
    # queries, ordered as the host restatement orders them.
    q = [1, 37, 130, 64, 700, 3, 700]
    kv = [1, 37 + 16 * 9, 130, 64 + 80, 2000, 3, 700]
    batch = make_paged_batch(131, q, kv, len(q), hq, hkv)
    out, plan = run_backend(batch, gpu)
    assert_attention_close(out, expected(batch))
    # run_backend drops the backend; plan again on a kept one to read its workspace.
    backend = MI355XAttentionBackend(hq, hkv, 128, 16, torch.bfloat16)
    common, qd, kc, vc = to_device(batch, gpu)
    p = backend.build_plan(common)
    empty = qd.new_empty((0, hkv, 128))
    backend.forward(qd, empty, empty, kc, vc, p)
    torch.cuda.synchronize()
    backend_ws = backend._prefill_workspace.view(torch.int32).cpu()
    tile = ops.PREFILL_STREAM_ROWS // (hq // hkv)
    # The launch's workgroups per KV head: one per CU, at most one per tile bound.
    per_head = min(torch.cuda.get_device_properties(gpu).multi_processor_count // hkv, p.metadata.prefill_max_tiles)
    want = _expected_tiles(q, kv, tile, tail=3 * max(per_head, 1))
    assert int(backend_ws[0]) == len(want) <= p.metadata.prefill_max_tiles
    assert ops.prefill_dropped_tiles(backend._prefill_workspace) == 0
    head, rec = ops.PREFILL_PLAN_HEADER_INTS, ops.PREFILL_PLAN_ITEM_INTS
    got = backend_ws[head:head + rec * len(want)].view(-1, rec).tolist()
    # Page slots -> the sequence's page ids.
    bt = batch.common.block_tables
    want = [r[:8] + [int(bt[r[0], i]) for i in r[8:]] for r in want]
    assert got == want


def test_undersized_tile_bound_is_reported(gpu):
    # A max_tiles below the batch's tile count (a host bound that disagrees
    # with the device's query offsets): the tiles past it are not run, their
    # rows keep the buffer's contents, and the plan reports how many.
    q = [300, 37, 130, 64]
    kv = [300 + 48, 37, 130, 64]
    batch = make_paged_batch(139, q, kv, len(q), 32, 8)
    common, qd, kc, vc = to_device(batch, gpu)
    tile = ops.PREFILL_STREAM_ROWS // 4
    n_tiles = len(_expected_tiles(q, kv, tile))
    ws = torch.empty(ops.prefill_workspace_bytes(n_tiles), dtype=torch.uint8, device=gpu)
    for cap, dropped in ((n_tiles, 0), (n_tiles - 3, 3), (1, n_tiles - 1)):
        out = torch.full_like(qd, float("nan"))
        ops.paged_prefill(qd, kc, vc, common.block_tables, common.seq_lens, common.query_start_loc, len(q), cap,
                          ws, out, 128 ** -0.5)
        assert ops.prefill_dropped_tiles(ws) == dropped
        stale = torch.isnan(out.float()).all(dim=2)  # [tokens, heads]
        assert bool(stale.any()) == (dropped > 0)
        ref = expected(batch)
        done = ~stale.cpu()
        torch.testing.assert_close(out.float().cpu()[done], ref[done], atol=2e-2, rtol=1e-2)


def test_more_sequences_than_the_planner_sorts(gpu):
    # 2100 short prefill sequences, more than the planner sorts (2048): the
    # device plans them in batch order, in two rounds; every row is still
    # computed once.
    import numpy as np

    rng = np.random.default_rng(23)
    n = 2100
    q = [int(x) for x in rng.integers(1, 6, size=n)]
    kv = [x + int(rng.integers(0, 40)) for x in q]
    batch = make_paged_batch(137, q, kv, n, 8, 8)
    out, plan = run_backend(batch, gpu)
    assert plan.route is AttentionRoute.PREFILL
    seqs = [0, 1, 1000, 2047, 2048, 2049, n - 1]
    exp, rows = expected(batch, seqs)
    assert_attention_close(out.cpu()[rows], exp)
    # Rows of every sequence are written (no NaN from the backend's buffer).
    assert bool(torch.isfinite(out.float()).all())


def test_tiles_of_other_kv_heads_run_with_their_own_heads(gpu):
    # Many one-tile items and more workgroups than one head's items: the
    # workgroups whose own queue empties first take other heads' tiles, which
    # must read that head's K/V and write that head's output columns.
    q = [3, 1, 2, 4, 1, 5, 2, 1, 3, 2, 6, 1]
    kv = [x + 16 * (i % 5) + 7 for i, x in enumerate(q)]
    batch = make_paged_batch(149, q, kv, len(q), 32, 8)
    for _ in range(3):
        out, _ = run_backend(batch, gpu)
        assert_attention_close(out, expected(batch))



@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_output_only_8_byte_aligned_matches_aligned(gpu, dtype):
    # The kernel stores 16 bytes per lane when the output and its strides are
    # 16-byte aligned and 8 bytes otherwise; an output view 8 bytes past an
    # aligned buffer takes the second path and must give the same bits.
    q = [300, 37, 130, 64, 1]
    kv = [300 + 48, 37, 130 + 16, 64, 90]
    batch = make_paged_batch(151, q, kv, len(q), 32, 8, dtype=dtype)
    common, qd, kc, vc = to_device(batch, gpu)
    tile = ops.PREFILL_STREAM_ROWS // 4
    n_tiles = len(_expected_tiles(q, kv, tile))
    ws = torch.empty(ops.prefill_workspace_bytes(n_tiles), dtype=torch.uint8, device=gpu)
    outs = []
    for shift in (0, 4):
        flat = torch.full((qd.numel() + 8,), float("nan"), dtype=dtype, device=gpu)
        out = flat[shift:shift + qd.numel()].view(qd.shape)
        assert (out.data_ptr() % 16 == 0) == (shift == 0)
        ops.paged_prefill(qd, kc, vc, common.block_tables, common.seq_lens, common.query_start_loc, len(q), n_tiles,
                          ws, out, 128 ** -0.5)
        outs.append(out.clone())
    assert torch.equal(outs[0], outs[1])
    assert_attention_close(outs[0].cpu(), expected(batch))


@pytest.mark.parametrize("hq,hkv", [(32, 8), (12, 4), (16, 1)])
def test_padded_output_rows_match_contiguous(gpu, hq, hkv):
    # Output rows at a padded, 16-byte aligned stride: the whole-line output
    # stores address every row through the token and head strides, give the
    # contiguous launch's bits and leave the padding untouched.
    q = [300, 37, 130, 64, 1]
    kv = [300 + 48, 37, 130 + 16, 64, 90]
    batch = make_paged_batch(163, q, kv, len(q), hq, hkv)
    common, qd, kc, vc = to_device(batch, gpu)
    tile = ops.PREFILL_STREAM_ROWS // (hq // hkv)
    n_tiles = len(_expected_tiles(q, kv, tile))
    ws = torch.empty(ops.prefill_workspace_bytes(n_tiles), dtype=torch.uint8, device=gpu)
    ref = torch.empty_like(qd)
    ops.paged_prefill(qd, kc, vc, common.block_tables, common.seq_lens, common.query_start_loc, len(q), n_tiles,
                      ws, ref, 128 ** -0.5)
    padded = torch.full((qd.shape[0], hq, 136), float("nan"), dtype=qd.dtype, device=gpu)
    out = padded[..., :128]
    assert out.data_ptr() % 16 == 0 and (out.stride(0) * 2) % 16 == 0 and (out.stride(1) * 2) % 16 == 0
    ops.paged_prefill(qd, kc, vc, common.block_tables, common.seq_lens, common.query_start_loc, len(q), n_tiles,
                      ws, out, 128 ** -0.5)
    assert torch.equal(out, ref)
    assert bool(torch.isnan(padded[..., 128:]).all())
    assert_attention_close(out.cpu(), expected(batch))


def _layers(seed, q, kv, hq, hkv, n, num_prefill=None):
    """n batches with one step's lengths and pages and each layer's own
    queries and cache values."""
    base = make_paged_batch(seed, q, kv, len(q) if num_prefill is None else num_prefill, hq, hkv)
    out = [base]
    for i in range(1, n):
        g = torch.Generator().manual_seed(seed * 100 + i)
        new = lambda t: torch.randn(t.shape, generator=g).to(t.dtype)  # noqa: E731
        out.append(dataclasses.replace(base, q=new(base.q), k_cache=new(base.k_cache), v_cache=new(base.v_cache)))
    return out


@pytest.mark.parametrize("hq,hkv,dtype", [(32, 8, torch.bfloat16), (16, 1, torch.bfloat16), (12, 4, torch.float16)])
def test_one_plan_serves_every_layer(gpu, hq, hkv, dtype):
    # One device plan, then a run per layer with that layer's queries and
    # caches: each run gives the bits of a launch that plans for itself, and
    # leaves the claim counters and the exit count at zero for the next.
    q = [300, 37, 130, 64, 1, 700]
    kv = [300 + 48, 37, 130 + 16, 64, 90, 900]
    layers = _layers(170, q, kv, hq, hkv, 3)
    common, _, _, _ = to_device(layers[0], gpu)
    tile = ops.PREFILL_STREAM_ROWS // (hq // hkv)
    n_tiles = len(_expected_tiles(q, kv, tile))
    ws = torch.empty(ops.prefill_workspace_bytes(n_tiles), dtype=torch.uint8, device=gpu)
    ws_fresh = torch.empty_like(ws)
    num_pages = layers[0].k_cache.shape[0]
    ops.paged_prefill_plan(common.block_tables, common.seq_lens, common.query_start_loc, len(q), n_tiles, ws,
                           num_pages, hq, hkv)
    scale = 128 ** -0.5
    for batch in layers:
        _, qd, kc, vc = (x.to(dtype) if torch.is_tensor(x) else x for x in to_device(batch, gpu))
        out = torch.full_like(qd, float("nan"))
        ops.paged_prefill(qd, kc, vc, common.block_tables, common.seq_lens, common.query_start_loc, len(q), n_tiles,
                          ws, out, scale, planned=True)
        ref = torch.full_like(qd, float("nan"))
        ops.paged_prefill(qd, kc, vc, common.block_tables, common.seq_lens, common.query_start_loc, len(q), n_tiles,
                          ws_fresh, ref, scale)
        assert torch.equal(out, ref)
        header = ws[:ops.PREFILL_PLAN_HEADER_INTS * 4].view(torch.int32).cpu()
        assert int(header[0]) == n_tiles and int(header[1]) == 0
        assert int(header[16]) == 0  # exit count
        lines = header[32:].view(-1, 32)[:, 0]
        assert int(lines.abs().sum()) == 0  # claim counters
        want = expected(dataclasses.replace(batch, q=batch.q.to(dtype), k_cache=batch.k_cache.to(dtype),
                                            v_cache=batch.v_cache.to(dtype)))
        assert_attention_close(out.cpu(), want)


def test_backend_plans_prefill_tiles_once_per_step(gpu):
    # The PREFILL route plans on its first layer and streams that plan on the
    # next; a new step (build_plan) plans again, also for a batch whose
    # lengths differ.
    hq, hkv = 32, 8
    backend = MI355XAttentionBackend(hq, hkv, 128, 16, torch.bfloat16)
    for step, (q, kv) in enumerate([([300, 37, 130], [348, 37, 146]), ([64, 700], [64, 900])]):
        layers = _layers(180 + step, q, kv, hq, hkv, 2)
        common, _, _, _ = to_device(layers[0], gpu)
        plan = backend.build_plan(common)
        assert backend._prefill_planned_for is None
        for batch in layers:
            _, qd, kc, vc = to_device(batch, gpu)
            empty = qd.new_empty((0, hkv, 128))
            out = backend.forward(qd, empty, empty, kc, vc, plan).clone()
            assert backend._prefill_planned_for is plan.metadata
            assert_attention_close(out.cpu(), expected(batch))


def test_split_mixed_route_reuses_the_prefill_plan_across_layers(gpu):
    # MIXED_SPLIT: the prefill half plans on the first layer and streams the
    # same plan on the next; both layers match the oracle, decode rows too.
    hq, hkv = 32, 8
    q = [300, 37, 130, 1, 1, 1]
    kv = [348, 37, 146, 90, 700, 17]
    backend = MI355XAttentionBackend(hq, hkv, 128, 16, torch.bfloat16, attention_mode="split")
    layers = _layers(190, q, kv, hq, hkv, 2, num_prefill=3)
    common, _, _, _ = to_device(layers[0], gpu)
    plan = backend.build_plan(common)
    assert plan.route is AttentionRoute.MIXED_SPLIT
    for batch in layers:
        _, qd, kc, vc = to_device(batch, gpu)
        empty = qd.new_empty((0, hkv, 128))
        out = backend.forward(qd, empty, empty, kc, vc, plan).clone()
        assert backend._prefill_planned_for is plan.metadata
        assert_attention_close(out.cpu(), expected(batch))
