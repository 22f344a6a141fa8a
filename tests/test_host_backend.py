"""CPU: host-side logic of the MI355X backend (no kernel launches).

Covers the reference contract the backend mirrors (registry, validation,
classification, plan routes, trusted planning without device reads) and the
work-list planners the kernels consume.  Metadata tensors stay on the CPU
through the ``require_device_metadata`` seam; nothing here calls a kernel.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from my_vllm_amd import ops
from my_vllm_amd.attention_backend import (
    MI355XAttentionBackend,
    MI355XAttentionMetadata,
    MI355XSplitAttentionBackend,
    decode_schedule,
    integrate,
    make_decode_plan,
    make_decode_plan_listed,
)
from my_vllm_amd.contract import AttentionBackend, AttentionPlan, AttentionRoute, BatchType, CommonAttentionMetadata
from tests import _foreign_contract as foreign

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


class HostBackend(MI355XAttentionBackend):
    require_device_metadata = False


class HostSplitBackend(MI355XSplitAttentionBackend):
    require_device_metadata = False


def _common(q_lens, kv_lens, num_prefill, *, trusted=False, cache=True):
    qsl = [0]
    for n in q_lens:
        qsl.append(qsl[-1] + n)
    counts = tuple((n + 15) // 16 for n in kv_lens)
    bt = None
    if cache:
        width, rows, page = max(counts), [], 0
        for c in counts:
            rows.append(list(range(page, page + c)) + [-1] * (width - c))
            page += c
        bt = torch.tensor(rows, dtype=torch.int32)
    return CommonAttentionMetadata(
        num_prefill_seqs=num_prefill,
        num_decode_seqs=len(q_lens) - num_prefill,
        num_prefill_tokens=sum(q_lens[:num_prefill]),
        num_decode_tokens=sum(q_lens[num_prefill:]),
        query_start_loc=torch.tensor(qsl, dtype=torch.int32),
        seq_lens=torch.tensor(kv_lens, dtype=torch.int32),
        slot_mapping=torch.arange(qsl[-1], dtype=torch.int32),
        block_tables=bt,
        max_q_len=max(q_lens),
        max_kv_len=max(kv_lens),
        block_counts=counts if cache else (),
        num_kv_blocks=sum(counts) if cache else 0,
        num_prefill_kv_blocks=sum(counts[:num_prefill]) if cache else 0,
        trusted=trusted,
    )


def test_page_csr_known_answer_through_backend_metadata():
    kat = KATS["page_csr"]
    backend = HostBackend(16, 4, 128, 16, torch.bfloat16)
    md = backend.build_metadata(_common(kat["query_lengths"], kat["kv_lengths"], kat["num_prefill_seqs"]))
    assert isinstance(md, MI355XAttentionMetadata)
    assert list(md.kv_indptr) == kat["kv_indptr"]
    assert md.num_pages == kat["num_pages"]
    assert md.num_prefill_pages == kat["num_prefill_pages"]


@pytest.mark.parametrize(
    "q_lens,kv_lens,num_prefill,batch,route,split_route",
    [
        ((5, 3), (21, 13), 2, BatchType.PURE_PREFILL, AttentionRoute.PREFILL, AttentionRoute.PREFILL),
        ((1, 1), (21, 13), 0, BatchType.PURE_DECODE, AttentionRoute.DECODE, AttentionRoute.DECODE),
        ((5, 1), (21, 13), 1, BatchType.MIXED, AttentionRoute.MIXED_UNIFIED, AttentionRoute.MIXED_SPLIT),
        ((1, 1), (1, 17), 1, BatchType.MIXED, AttentionRoute.MIXED_UNIFIED, AttentionRoute.MIXED_SPLIT),
    ],
)
@pytest.mark.parametrize("trusted", [False, True])
def test_plan_routes(q_lens, kv_lens, num_prefill, batch, route, split_route, trusted):
    # Reference cases: tests/test_attention_backend.py:367-418 shapes and the
    # all-single-token MIXED batch of tests/test_model_runner_metadata.py:351-374.
    common = _common(q_lens, kv_lens, num_prefill, trusted=trusted)
    plan = HostBackend(16, 4, 128, 16, torch.bfloat16).build_plan(common)
    assert isinstance(plan, AttentionPlan)
    assert plan.batch_type is batch and plan.route is route and plan.common is common
    split = HostSplitBackend(16, 4, 128, 16, torch.bfloat16).build_plan(common)
    assert split.batch_type is batch and split.route is split_route


def test_cacheless_batch_plans_warmup():
    plan = HostBackend(16, 4, 128, 16, torch.bfloat16).build_plan(_common((3, 1), (3, 1), 2, cache=False))
    assert plan.route is AttentionRoute.WARMUP and plan.metadata.is_cacheless


def test_trusted_planning_reads_no_device_values(monkeypatch):
    # Trusted metadata is planned from host ints only (reference
    # tests/test_attention_backend.py:529-553): no .item()/.cpu()/.tolist().
    common = _common((5, 1, 1), (21, 13, 300), 1, trusted=True)
    backend = HostBackend(16, 4, 128, 16, torch.bfloat16)

    def forbidden(*args, **kwargs):
        raise AssertionError("device read during trusted planning")

    for name in ("item", "cpu", "tolist", "numpy"):
        monkeypatch.setattr(torch.Tensor, name, forbidden)
    plan = backend.build_plan(common)
    monkeypatch.undo()
    assert plan.route is AttentionRoute.MIXED_UNIFIED
    assert plan.metadata.num_decode_items > 0 and plan.metadata.mixed_prefill_max_tiles > 0


def test_validation_errors_follow_the_reference():
    backend = HostBackend(16, 4, 128, 16, torch.bfloat16)
    good = _common((5, 1), (21, 13), 1)
    with pytest.raises(TypeError):
        backend.build_plan(object())
    bad_decode = _common((5, 2), (21, 13), 1)
    with pytest.raises(ValueError, match="one query token"):
        backend.build_plan(bad_decode)
    wrong_dtype = CommonAttentionMetadata(**{**good.__dict__, "seq_lens": good.seq_lens.long()})
    with pytest.raises(TypeError, match="int32"):
        backend.build_plan(wrong_dtype)
    device_backend = MI355XAttentionBackend(16, 4, 128, 16, torch.bfloat16)
    with pytest.raises(ValueError, match="CUDA"):
        device_backend.build_plan(good)


def test_forward_rejects_foreign_plans_and_mismatched_caches():
    backend = HostBackend(16, 4, 128, 16, torch.bfloat16)
    plan = backend.build_plan(_common((1, 1), (21, 13), 0))
    q = torch.zeros(2, 16, 128, dtype=torch.bfloat16)
    cache = torch.zeros(4, 16, 4, 128, dtype=torch.bfloat16)
    empty = q.new_empty((0, 4, 128))
    with pytest.raises(TypeError):
        backend.forward(q, empty, empty, cache, cache, object())
    foreign = AttentionPlan(plan.batch_type, plan.route, plan.common, object())
    with pytest.raises(TypeError):
        backend.forward(q, empty, empty, cache, cache, foreign)
    with pytest.raises(ValueError):
        backend.forward(q, empty, empty, cache, empty, plan)


def test_constructor_contract():
    with pytest.raises(ValueError):
        MI355XAttentionBackend(16, 4, 64, 16, torch.bfloat16)
    with pytest.raises(ValueError):
        MI355XAttentionBackend(16, 4, 128, 32, torch.bfloat16)
    with pytest.raises(TypeError):
        MI355XAttentionBackend(16, 4, 128, 16, torch.float32)
    with pytest.raises(ValueError):
        MI355XAttentionBackend(16, 5, 128, 16, torch.bfloat16)
    backend = MI355XAttentionBackend(16, 4, 128, 16, torch.float16)
    assert backend.softmax_scale == pytest.approx(128 ** -0.5)


def test_support_reason_names_the_missing_capability():
    reason = MI355XAttentionBackend.support_reason(
        num_q_heads=16, num_kv_heads=4, head_dim=128, block_size=16, dtype=torch.bfloat16, device="cpu"
    )
    assert isinstance(reason, str) and reason
    assert MI355XAttentionBackend.supports(num_q_heads=16, num_kv_heads=4, head_dim=64, block_size=16,
                                           dtype=torch.bfloat16, device="cpu") is False


def test_backend_is_an_attention_backend_with_reference_capability_contract():
    assert issubclass(MI355XAttentionBackend, AttentionBackend)
    caps = dict(num_q_heads=16, num_kv_heads=4, head_dim=128, block_size=16, dtype=torch.bfloat16, device="cpu")
    assert type(MI355XAttentionBackend.supports(**caps)) is bool
    assert MI355XSplitAttentionBackend.default_attention_mode == "split"


def _foreign_backends(registry_name: str):
    class Registry(foreign.ForeignRegistry):
        backends = {}

    unified, split = integrate(Registry, foreign.ForeignBackendBase, foreign.ForeignPlan, foreign.ForeignRoute,
                               foreign.ForeignBatchType, foreign.ForeignCommon,
                               names=(registry_name, registry_name + "_split"))
    return Registry, unified, split


def test_integrate_registers_both_modes_in_a_foreign_registry():
    registry, unified, split = _foreign_backends("mi355x")
    assert registry.backends == {"mi355x": unified, "mi355x_split": split}
    assert issubclass(unified, foreign.ForeignBackendBase) and issubclass(split, unified)
    supported, reason = registry.support("mi355x", num_q_heads=16, num_kv_heads=4, head_dim=128, block_size=16,
                                         dtype=torch.bfloat16, device="cpu")
    assert supported is False and isinstance(reason, str) and reason  # no gfx950 in a CPU process
    with pytest.raises(ValueError):
        integrate(registry, foreign.ForeignBackendBase, foreign.ForeignPlan, foreign.ForeignRoute,
                  foreign.ForeignBatchType, foreign.ForeignCommon)  # names taken


@pytest.mark.parametrize(
    "q_lens,kv_lens,num_prefill,batch,unified_route,split_route",
    [
        ((1, 1), (21, 13), 0, "PURE_DECODE", "DECODE", "DECODE"),
        ((5, 3), (21, 13), 2, "PURE_PREFILL", "PREFILL", "PREFILL"),
        ((5, 1), (21, 13), 1, "MIXED", "MIXED_UNIFIED", "MIXED_SPLIT"),
    ],
)
def test_foreign_family_plans_return_the_foreign_classes(q_lens, kv_lens, num_prefill, batch, unified_route,
                                                         split_route):
    _, unified, split = _foreign_backends("f")
    common = foreign.to_foreign(_common(q_lens, kv_lens, num_prefill, trusted=True))
    for cls, route in ((unified, unified_route), (split, split_route)):
        host_cls = type("Host", (cls,), {"require_device_metadata": False})
        plan = host_cls(16, 4, 128, 16, torch.bfloat16).build_plan(common)
        assert type(plan) is foreign.ForeignPlan
        assert plan.batch_type is foreign.ForeignBatchType[batch] and plan.route is foreign.ForeignRoute[route]
    with pytest.raises(TypeError):
        type("Host", (unified,), {"require_device_metadata": False})(16, 4, 128, 16, torch.bfloat16).build_plan(
            _common(q_lens, kv_lens, num_prefill, trusted=True))  # this package's class is foreign to it


def _record_launches(monkeypatch, backend):
    calls = []
    monkeypatch.setattr(type(backend), "_validate_inputs", lambda self, q, kc, vc: None)
    for name in ("paged_decode", "paged_decode_store", "store_kvcache"):
        monkeypatch.setattr(ops, name, lambda *a, _n=name, **k: calls.append(_n))
    monkeypatch.setattr(type(backend), "_get_workspace", lambda self, nbytes, device: None)
    return calls


@pytest.mark.parametrize("family", ["own", "foreign"])
@pytest.mark.parametrize("trusted", [True, False])
def test_fused_store_path_is_taken_for_trusted_piece_list_decode(monkeypatch, family, trusted):
    # forward_with_kv_store folds the store into the decode launch for the
    # backend's own plan class and for a foreign family alike, and only for
    # trusted (model-runner) metadata; otherwise the store runs first.
    if family == "own":
        cls = HostBackend
        common = _common((1, 1, 1), (21, 13, 300), 0, trusted=trusted)
    else:
        _, unified, _ = _foreign_backends("g")
        cls = type("Host", (unified,), {"require_device_metadata": False})
        common = foreign.to_foreign(_common((1, 1, 1), (21, 13, 300), 0, trusted=trusted))
    backend = cls(16, 4, 128, 16, torch.bfloat16)
    plan = backend.build_plan(common)
    assert plan.metadata.decode_wave_extra is not None  # piece lists
    calls = _record_launches(monkeypatch, backend)
    q = torch.zeros(3, 16, 128, dtype=torch.bfloat16)
    kv = torch.zeros(3, 4, 128, dtype=torch.bfloat16)
    cache = torch.zeros(40, 16, 4, 128, dtype=torch.bfloat16)
    backend.forward_with_kv_store(q, kv, kv, cache, cache, common.slot_mapping, plan)
    assert calls == (["paged_decode_store"] if trusted else ["store_kvcache", "paged_decode"])


# ---------------------------------------------------------------------------
# Work-list planners
# ---------------------------------------------------------------------------

def _check_decode_plan(counts, hkv, waves, per_wave, min_pages):
    items, nw, slots = make_decode_plan(np.asarray(counts), 3, 7, hkv, waves, per_wave, min_pages)
    assert items.dtype == np.int32 and items.shape[1] == ops.DECODE_ITEM_INTS
    assert 1 <= nw <= len(items) and nw <= waves
    seen = {}
    for s, pb, pe, ch, nc, base, qrow, h in items.tolist():
        i = s - 3
        assert qrow == 7 + i and 0 <= h < hkv and 0 <= pb < pe <= counts[i] and pe - pb <= ops.MAX_CHUNK_PAGES
        seen.setdefault((i, h), []).append((pb, pe, ch, nc, base))
    assert len(seen) == len(counts) * hkv
    used = set()
    for (i, h), pieces in seen.items():
        pieces.sort()
        nc = pieces[0][3]
        assert len(pieces) == nc and {p[3] for p in pieces} == {nc}
        assert pieces[0][0] == 0 and pieces[-1][1] == counts[i]
        assert all(a[1] == b[0] for a, b in zip(pieces, pieces[1:]))
        assert sorted(p[2] for p in pieces) == list(range(nc))
        if nc > 1:
            base = pieces[0][4]
            assert all(p[4] == base for p in pieces) and base + nc <= slots
            # The kernel's partial slot of chunk c: (base + c) * Hkv + h.
            ids = {(base + c) * hkv + h for c in range(nc)}
            assert not used & ids
            used |= ids
    assert len(used) <= slots * hkv
    lengths = items[:, 2] - items[:, 1]
    assert np.all(np.diff(lengths) <= 0), "pieces are listed longest first"
    return items, nw, slots


@pytest.mark.parametrize("seed", range(20))
def test_decode_plan_covers_every_page_once(seed):
    rng = np.random.default_rng(seed)
    counts = rng.integers(1, 400, size=int(rng.integers(1, 40))).tolist()
    _check_decode_plan(counts, int(rng.choice([1, 2, 8])), int(rng.integers(1, 5000)),
                       int(rng.integers(1, 9)), int(rng.integers(1, 9)))


def test_decode_plan_edges():
    items, nw, slots = _check_decode_plan([1], 1, 2048, 4, 4)
    assert len(items) == 1 and nw == 1 and slots == 0
    items, nw, _ = _check_decode_plan([300], 8, 1, 1, 4)
    assert nw == 1 and (items[:, 2] - items[:, 1]).max() <= ops.MAX_CHUNK_PAGES
    empty, nw, slots = make_decode_plan(np.zeros(0, np.int64), 0, 0, 8, 2048)
    assert empty.shape == (0, ops.DECODE_ITEM_INTS) and nw == 0 and slots == 0
    with pytest.raises(ValueError):
        make_decode_plan(np.array([0]), 0, 0, 8, 2048)


def _check_listed_plan(counts, hkv, groups, max_piece):
    counts = np.asarray(counts, dtype=np.int64)
    items, wave_extra, nw, slots = make_decode_plan_listed(counts, 3, 7, hkv, groups, max_piece)
    total = int(counts.sum())
    g = min(groups, total)
    offsets = np.concatenate(([0], np.cumsum(counts)))
    assert items.dtype == np.int32 and items.shape[1] == ops.DECODE_ITEM_INTS
    assert nw == g * hkv and wave_extra.dtype == np.int32 and wave_extra.shape == (nw + 1,)
    assert wave_extra[0] == nw and wave_extra[-1] == len(items) and np.all(np.diff(wave_extra) >= 0)
    covered = np.zeros((hkv, total), dtype=np.int64)
    slot_ids = set()
    segments = {}
    for w in range(nw):
        rows = [w] + list(range(wave_extra[w], wave_extra[w + 1]))
        spans = []
        for r in rows:
            s, pb, pe, ch, nc, base, qrow, h = (int(x) for x in items[r])
            i = s - 3
            assert qrow == 7 + i and h == w % hkv and 0 <= pb < pe <= counts[i] and pe - pb <= max_piece
            spans.append((offsets[i] + pb, offsets[i] + pe))
            covered[h, offsets[i] + pb:offsets[i] + pe] += 1
            segments.setdefault((i, h), []).append((pb, pe, ch, nc, base))
            if nc > 1:
                slot = (base + ch) * hkv + h
                assert slot not in slot_ids and base + ch < slots
                slot_ids.add(slot)
        # The wavefront's pieces tile its range [r*T//g, (r+1)*T//g) in page order.
        r = w // hkv
        assert spans[0][0] == r * total // g and spans[-1][1] == (r + 1) * total // g
        assert all(a[1] == b[0] for a, b in zip(spans, spans[1:]))
    assert np.all(covered == 1), "every (page, KV head) exactly once"
    for (i, h), pieces in segments.items():
        nc = pieces[0][3]
        assert [p[2] for p in pieces] == list(range(nc)) and {p[3] for p in pieces} == {nc}
        assert pieces[0][0] == 0 and pieces[-1][1] == counts[i]
    pages = np.diff((np.arange(g + 1) * total) // g)
    assert pages.max() - pages.min() <= 1, "equal share per wavefront"
    return items, wave_extra, nw, slots


@pytest.mark.parametrize("seed", range(20))
def test_listed_decode_plan_tiles_every_wavefront_range(seed):
    rng = np.random.default_rng(500 + seed)
    counts = rng.integers(1, 400, size=int(rng.integers(1, 40))).tolist()
    _check_listed_plan(counts, int(rng.choice([1, 2, 3, 4, 8])), int(rng.integers(1, 3000)),
                       int(rng.choice([1, 3, 17, 128])))


def test_decode_schedule_by_head_count_and_size():
    # Pages of 16 tokens x 128 dims x bf16, K and V: 8 KiB per page and KV head.
    pages_of = lambda gib, hkv: int(gib * (1 << 30)) // (8192 * hkv)
    # Eight KV heads fill a workgroup: piece lists at every size.
    assert decode_schedule(pages_of(0.5, 8), 8) == "listed"
    assert decode_schedule(pages_of(11.2, 8), 8) == "listed"
    # Other head counts: piece lists up to 2 GiB of K/V, claims above.
    assert decode_schedule(pages_of(2.0, 4), 4) == "listed"
    assert decode_schedule(pages_of(2.0, 4) + 1, 4) == "claims"
    assert decode_schedule(pages_of(3.0, 16), 16) == "claims"
    assert decode_schedule(pages_of(1.0, 1), 1) == "listed"
    # A backend's override picks either one.
    assert decode_schedule(pages_of(11.2, 8), 8, forced="claims") == "claims"
    assert decode_schedule(10, 4, forced="listed") == "listed"
    with pytest.raises(ValueError):
        decode_schedule(10, 8, forced="static")


def test_listed_decode_plan_edges():
    items, wave_extra, nw, slots = _check_listed_plan([1], 8, 256, 128)
    assert nw == 8 and len(items) == 8 and slots == 0 and wave_extra.tolist() == [8] * 9
    # More workgroups than pages: one page per range.
    items, _, nw, _ = _check_listed_plan([3, 2], 4, 1000, 128)
    assert nw == 5 * 4
    # One range over a long sequence: pieces of at most 128 pages, chunked.
    items, _, nw, slots = _check_listed_plan([300], 2, 1, 128)
    assert nw == 2 and slots == 3
    empty, wave_extra, nw, slots = make_decode_plan_listed(np.zeros(0, np.int64), 0, 0, 8, 256)
    assert empty.shape == (0, ops.DECODE_ITEM_INTS) and nw == 0 and slots == 0
    with pytest.raises(ValueError):
        make_decode_plan_listed(np.array([0]), 0, 0, 8, 256)


@pytest.mark.parametrize("seed", range(10))
def test_prefill_tile_bounds_hold_for_any_split_of_the_tokens(seed):
    # The host knows only the prefill token and sequence counts; the bounds
    # must cover every split of those tokens into sequences (the device
    # derives the real tiles, 256-row for PREFILL, 128-row for MIXED).
    rng = np.random.default_rng(100 + seed)
    n = int(rng.integers(1, 40))
    q = rng.integers(1, 3000, size=n)
    hkv = int(rng.choice([1, 2, 4, 8]))
    hq = hkv * int(rng.choice([1, 2, 3, 4, 8, 16]))
    g = hq // hkv
    for rows, bound in ((ops.PREFILL_STREAM_ROWS, ops.prefill_max_tiles),
                        (ops.PREFILL_ROWS, ops.mixed_prefill_max_tiles)):
        tile = rows // g
        assert int(np.sum(-(-q // tile))) <= bound(int(q.sum()), n, hq, hkv)


def test_mixed_beyond_one_launch_limits_plans_mixed_split():
    # More prefill sequences than one MIXED launch takes: the unified
    # backend plans MIXED_SPLIT (prefill + decode launches) and names the
    # limit, as the reference plans MIXED_SPLIT whenever it runs two
    # launches (attention_backend.py:626-663, 858-890).
    backend = HostBackend(16, 4, 128, 16, torch.bfloat16)
    assert backend.mixed_attention_available and backend.mixed_attention_unavailable_reason is None
    n = ops.MIXED_PREFILL_SEQS_MAX + 1
    common = _common((1,) * n + (1,), (5,) * n + (9,), n, trusted=True)
    plan = backend.build_plan(common)
    assert plan.route is AttentionRoute.MIXED_SPLIT
    assert plan.metadata.mixed_prefill_max_tiles == 0 and plan.metadata.prefill_max_tiles > 0
    assert plan.metadata.num_decode_merges >= 0 and plan.metadata.decode_items is not None
    assert backend.mixed_attention_available is False
    assert f"{ops.MIXED_PREFILL_SEQS_MAX} prefill sequences" in backend.mixed_attention_unavailable_reason
    small = backend.build_plan(_common((5, 1), (21, 13), 1, trusted=True))
    assert small.route is AttentionRoute.MIXED_UNIFIED and small.metadata.mixed_prefill_max_tiles > 0
    assert backend.mixed_attention_available and backend.mixed_attention_unavailable_reason is None
    # More KV heads than one MIXED launch's counters cover: split from the start.
    wide = HostBackend(128, 128, 128, 16, torch.bfloat16)
    assert ops.MIXED_MAX_KV_HEADS < 128
    assert not wide.mixed_attention_available and "KV heads" in wide.mixed_attention_unavailable_reason
    plan = wide.build_plan(_common((5, 1), (21, 13), 1, trusted=True))
    assert plan.route is AttentionRoute.MIXED_SPLIT and plan.metadata.mixed_prefill_max_tiles == 0
    # Split mode: the reference's reason string.
    split = HostSplitBackend(16, 4, 128, 16, torch.bfloat16)
    assert split.mixed_attention_unavailable_reason == "unified mixed attention is disabled in split mode"


def test_mixed_split_pair_limit_plans_mixed_split():
    # A single MIXED launch merges at most MIXED_ARRIVAL_COUNTERS split-K
    # (partial slot, KV head) pairs; a decode plan beyond that runs split.
    backend = HostBackend(64, 64, 128, 16, torch.bfloat16)
    backend.decode_waves_override = 100000  # 4-page pieces: many split segments
    common = _common((5,) + (1,) * 300, (21,) + (2048,) * 300, 1, trusted=True)
    plan = backend.build_plan(common)
    assert plan.route is AttentionRoute.MIXED_SPLIT
    assert "split-K" in backend.mixed_attention_unavailable_reason
    assert plan.metadata.num_decode_merges > 0


def _validate_dispatch_route(*, batch_type, planned_route, mixed_attention_available, expected_route="auto"):
    """The reference's dispatch-benchmark rule (bench_attention_dispatch.py:208-230):
    the planned route must equal the capability route."""
    assert batch_type == "mixed"
    capability = "mixed_unified" if mixed_attention_available else "mixed_split"
    required = capability if expected_route == "auto" else expected_route
    assert planned_route == required and planned_route == capability
    return planned_route


@pytest.mark.parametrize("case", ["within", "beyond_seqs", "split_mode", "wide"])
def test_planned_route_equals_the_capability_route(case):
    n = ops.MIXED_PREFILL_SEQS_MAX + 1
    backend = {"within": HostBackend(16, 4, 128, 16, torch.bfloat16),
               "beyond_seqs": HostBackend(16, 4, 128, 16, torch.bfloat16),
               "split_mode": HostSplitBackend(16, 4, 128, 16, torch.bfloat16),
               "wide": HostBackend(128, 128, 128, 16, torch.bfloat16)}[case]
    common = (_common((1,) * n + (1,), (5,) * n + (9,), n, trusted=True) if case == "beyond_seqs"
              else _common((5, 1), (21, 13), 1, trusted=True))
    plan = backend.build_plan(common)
    route = _validate_dispatch_route(batch_type=plan.batch_type.value, planned_route=plan.route.value,
                                     mixed_attention_available=backend.mixed_attention_available)
    assert route == ("mixed_unified" if case == "within" else "mixed_split")
    assert (backend.mixed_attention_unavailable_reason is None) == (case == "within")
    counts = dict(backend.route_counts)
    assert counts[route] == 1 and sum(counts.values()) == 1


def test_mixed_route_must_match_its_metadata():
    # A MIXED_UNIFIED plan over metadata planned for two launches (or the
    # reverse) is refused before any launch.
    backend = HostBackend(16, 4, 128, 16, torch.bfloat16)
    common = _common((5, 1), (21, 13), 1, trusted=True)
    unified = backend.build_plan(common)
    forced = AttentionPlan(unified.batch_type, AttentionRoute.MIXED_SPLIT, common, unified.metadata)
    q = torch.zeros(6, 16, 128, dtype=torch.bfloat16)
    cache = torch.zeros(3, 16, 4, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="does not match the planned metadata"):
        backend.forward(q, None, None, cache, cache, forced)


@pytest.mark.parametrize("seed", range(5))
def test_decode_merge_list_names_every_split_segment_once(seed):
    rng = np.random.default_rng(300 + seed)
    counts = rng.integers(1, 300, size=int(rng.integers(1, 30)))
    hkv = int(rng.choice([1, 4, 8]))
    items, _, slots = make_decode_plan(counts, 3, 7, hkv, int(rng.choice([16, 256, 4096])), 2.0, 1)
    merges = ops.decode_merge_list(items)
    assert merges.dtype == np.int32 and merges.shape[1] == ops.DECODE_ITEM_INTS
    split = {(int(s), int(h)) for s, n, h in items[:, [0, 4, 7]] if n > 1}
    listed = [(int(s), int(h)) for s, h in merges[:, [0, 7]]]
    assert len(listed) == len(set(listed)) and set(listed) == split
    assert np.all(merges[:, 3] == 0) and np.all(merges[:, 4] > 1)
    # Every merge's slots stay inside the plan's partial-slot count.
    assert np.all(merges[:, 5] + merges[:, 4] <= slots)


# ---------------------------------------------------------------------------
# Full-decode graph state (host side)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("seed", range(15))
def test_graph_capacities_hold_every_fitting_piece_list_plan(seed):
    from my_vllm_amd.attention_backend import graph_decode_capacities

    rng = np.random.default_rng(900 + seed)
    batch = int(rng.integers(1, 40))
    width = int(rng.integers(1, 600))
    hkv = int(rng.choice([1, 2, 4, 8]))
    groups = int(rng.choice([1, 7, 256, 1024]))
    caps = graph_decode_capacities(batch, batch * width, hkv, groups)
    counts = rng.integers(1, width + 1, size=batch)
    items, wave_extra, waves, slots = make_decode_plan_listed(counts, 0, 0, hkv, groups)
    merges = ops.decode_merge_list(items)
    assert items.shape[0] <= caps["item_capacity"]
    assert waves <= caps["wave_capacity"] <= caps["item_capacity"]
    assert merges.shape[0] <= caps["merge_capacity"]
    assert slots <= caps["part_slot_capacity"]


def test_graph_plan_buffer_layout_round_trips():
    from my_vllm_amd.attention_backend import pack_graph_decode_plan, split_graph_plan_buffer

    counts = np.array([3, 40, 1, 17])
    items, wave_extra, waves, _ = make_decode_plan_listed(counts, 0, 0, 2, 5)
    merges = ops.decode_merge_list(items)
    buf = pack_graph_decode_plan(items, wave_extra, merges, 64, 12, 9)
    c, it, we, mg = split_graph_plan_buffer(buf, 64, 12, 9)
    assert c.tolist() == [items.shape[0], waves, merges.shape[0]]
    assert np.array_equal(it[: items.shape[0]], items) and not it[items.shape[0]:].any()
    assert np.array_equal(we[: waves + 1], wave_extra)
    assert np.array_equal(mg[: merges.shape[0]], merges)
    with pytest.raises(ValueError):
        pack_graph_decode_plan(items, wave_extra, merges, items.shape[0] - 1, 12, 9)


def test_graph_hooks_validate_like_the_reference():
    backend = HostBackend(16, 8, 128, 16, torch.bfloat16)
    assert backend.supports_full_decode_graph
    with pytest.raises(ValueError):
        backend.create_full_decode_graph_state(4, 64, "cpu")
    with pytest.raises(TypeError):
        backend.create_full_decode_graph_state(True, 64, "cpu")
    with pytest.raises(ValueError):
        backend.create_full_decode_graph_state(4, 3, "cpu")
    plan = backend.build_plan(_common([1, 1], [20, 5], 0))
    assert backend.full_decode_graph_metadata_fits(object(), plan) is False
    with pytest.raises(ValueError, match="does not fit"):
        backend.plan_full_decode_graph(object(), plan)
    with pytest.raises(TypeError):
        backend.activate_full_decode_graph(object())
    backend.deactivate_full_decode_graph()


def test_pinned_staging_round_trips_int32_lists_on_the_host():
    from my_vllm_amd.attention_backend import PinnedStaging

    ring = PinnedStaging(slots=2)
    rng = np.random.default_rng(5)
    for n in (0, 1, 7, 5000, 3):
        a = rng.integers(-(2**31), 2**31 - 1, size=n, dtype=np.int64).astype(np.int32)
        t = ring.to_device(a, torch.device("cpu"))
        assert t.dtype == torch.int32 and t.shape == (n,)
        assert np.array_equal(t.numpy(), a)
