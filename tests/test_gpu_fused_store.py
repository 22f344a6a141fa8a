"""The slot_mapping KV store folded into the piece-list decode launch.

``forward_with_kv_store`` on a DECODE step must leave the caches and the
output bit-identical to ``store_kvcache`` followed by ``forward`` (the
reference's ``Attention.forward`` order, nanovllm/layers/attention.py:131-143);
the rows it stores are a bit copy, and the attention sees them because the
only reader of each row writes it first.  Steps the fused launch does not
cover (claim schedule, prefill) fall back to the separate store.
"""

import dataclasses

import pytest
import torch

from my_vllm_amd import ops
from my_vllm_amd.attention_backend import MI355XAttentionBackend
from my_vllm_amd.contract import AttentionRoute
from workloads import config_decode_small, make_paged_batch
from tests._util import assert_attention_close, set_decode_planning
from tests.test_gpu_prefill import expected, to_device

pytestmark = pytest.mark.gpu


def _both_ways(batch, device, dtype=torch.bfloat16, slots=None, trusted=True):
    hq, hkv = batch.q.shape[1], batch.k_cache.shape[2]
    common, q, kc, vc = to_device(batch, device, trusted)
    k_new, v_new = batch.k_new.to(device), batch.v_new.to(device)
    slot_mapping = common.slot_mapping if slots is None else slots.to(device)
    backend = MI355XAttentionBackend(hq, hkv, 128, 16, dtype)
    plan = backend.build_plan(common)
    kc_a, vc_a = kc.clone(), vc.clone()
    ops.store_kvcache(k_new, v_new, kc_a, vc_a, slot_mapping)
    sep = backend.forward(q, k_new, v_new, kc_a, vc_a, plan).clone()
    kc_b, vc_b = kc.clone(), vc.clone()
    fused = backend.forward_with_kv_store(q, k_new, v_new, kc_b, vc_b, slot_mapping, plan).clone()
    return plan, sep, fused, (kc_a, vc_a), (kc_b, vc_b)


def test_headline_decode_step_matches_store_then_decode(gpu):
    batch = config_decode_small(seed=1)
    plan, sep, fused, (kc_a, vc_a), (kc_b, vc_b) = _both_ways(batch, gpu)
    assert plan.route is AttentionRoute.DECODE and plan.metadata.decode_wave_extra is not None
    assert torch.equal(kc_a, kc_b) and torch.equal(vc_a, vc_b)
    assert torch.equal(sep, fused)
    seqs = [0, 1, 31, 63]
    stored = dataclasses.replace(batch, k_cache=kc_a.cpu(), v_cache=vc_a.cpu())
    exp, rows = expected(stored, seqs)
    assert_attention_close(fused.cpu()[rows], exp)


@pytest.mark.parametrize("hq,hkv", [(16, 8), (12, 3), (8, 1)])
def test_page_boundaries_int64_slots_and_skips(gpu, hq, hkv):
    # New tokens at the first, last and a middle row of their page, one-page
    # sequences, and a -1 slot that must leave the cache untouched.
    ctx = [1, 16, 17, 32, 300, 513, 2049]
    batch = make_paged_batch(83, [1] * len(ctx), ctx, 0, hq, hkv, dtype=torch.float16)
    slots = batch.common.slot_mapping.to(torch.int64).clone()
    slots[2] = -1
    plan, sep, fused, (kc_a, vc_a), (kc_b, vc_b) = _both_ways(batch, gpu, torch.float16, slots)
    assert torch.equal(kc_a, kc_b) and torch.equal(vc_a, vc_b)
    assert torch.equal(sep, fused)


def test_claim_schedule_falls_back_to_the_separate_store(gpu, monkeypatch):
    set_decode_planning(monkeypatch, schedule="claims")
    batch = make_paged_batch(89, [1] * 5, [40, 7, 1000, 16, 129], 0, 32, 8)
    plan, sep, fused, (kc_a, vc_a), (kc_b, vc_b) = _both_ways(batch, gpu)
    assert plan.metadata.decode_wave_extra is None
    assert torch.equal(kc_a, kc_b) and torch.equal(vc_a, vc_b)
    assert torch.equal(sep, fused)
    stored = dataclasses.replace(batch, k_cache=kc_a.cpu(), v_cache=vc_a.cpu())
    assert_attention_close(fused, expected(stored))


def _moved_slot_batch(where="first_page"):
    # Sequence 2's new row is sent to a slot in its first page (a page the
    # decode launch may be streaming elsewhere), or to the wrong row of its
    # last page, instead of its last position.
    batch = make_paged_batch(97, [1] * 5, [40, 7, 1000, 16, 129], 0, 16, 8)
    slots = batch.common.slot_mapping.clone()
    if where == "first_page":
        slots[2] = int(batch.common.block_tables[2, 0]) * 16 + 3
    else:
        assert (1000 - 1) % 16 > 0
        slots[2] = slots[2] - 1
    return batch, slots


@pytest.mark.parametrize("where", ["first_page", "last_page_wrong_row"])
def test_slot_outside_the_last_position_is_stored_late_and_flagged(gpu, where):
    batch, slots = _moved_slot_batch(where)
    common, q, kc, vc = to_device(batch, gpu)
    k_new, v_new = batch.k_new.to(gpu), batch.v_new.to(gpu)
    slots = slots.to(gpu)
    backend = MI355XAttentionBackend(16, 8, 128, 16, torch.bfloat16)
    plan = backend.build_plan(common)
    assert common.trusted and plan.metadata.decode_wave_extra is not None
    fused = backend.forward_with_kv_store(q, k_new, v_new, kc, vc, slots, plan).clone()
    assert backend.fused_store_error() is True
    assert backend.fused_store_error() is False  # cleared by the first read
    # The caches equal the reference's store of every row, the moved one included.
    kc_e, vc_e = batch.k_cache.to(gpu), batch.v_cache.to(gpu)
    ops.store_kvcache(k_new, v_new, kc_e, vc_e, slots)
    assert torch.equal(kc, kc_e) and torch.equal(vc, vc_e)
    # The attention ran before the moved row was written.
    kc_o, vc_o = batch.k_cache.to(gpu), batch.v_cache.to(gpu)
    keep = torch.ones(5, dtype=torch.bool, device=gpu)
    keep[2] = False
    ops.store_kvcache(k_new[keep], v_new[keep], kc_o, vc_o, slots[keep])
    assert torch.equal(fused, backend.forward(q, k_new, v_new, kc_o, vc_o, plan))
    # A second fused step on the same workspace: the late-row flags were
    # cleared, so every in-place row is written by the decode again.
    kc2, vc2 = batch.k_cache.to(gpu), batch.v_cache.to(gpu)
    good = common.slot_mapping
    again = backend.forward_with_kv_store(q, k_new, v_new, kc2, vc2, good, plan).clone()
    assert backend.fused_store_error() is False
    kc_g, vc_g = batch.k_cache.to(gpu), batch.v_cache.to(gpu)
    ops.store_kvcache(k_new, v_new, kc_g, vc_g, good)
    assert torch.equal(kc2, kc_g) and torch.equal(vc2, vc_g)
    assert torch.equal(again, backend.forward(q, k_new, v_new, kc_g, vc_g, plan))


def test_fused_store_debug_check_raises(gpu):
    batch, slots = _moved_slot_batch()
    common, q, kc, vc = to_device(batch, gpu)
    backend = MI355XAttentionBackend(16, 8, 128, 16, torch.bfloat16)
    backend.check_fused_store = True
    plan = backend.build_plan(common)
    k_new, v_new = batch.k_new.to(gpu), batch.v_new.to(gpu)
    backend.forward_with_kv_store(q, k_new, v_new, kc, vc, common.slot_mapping, plan)  # in place: no error
    with pytest.raises(RuntimeError, match="last position"):
        backend.forward_with_kv_store(q, k_new, v_new, kc, vc, slots.to(gpu), plan)


def test_untrusted_metadata_stores_first_like_the_reference(gpu):
    batch, slots = _moved_slot_batch()
    plan, sep, fused, (kc_a, vc_a), (kc_b, vc_b) = _both_ways(batch, gpu, slots=slots, trusted=False)
    assert not plan.common.trusted and plan.metadata.decode_wave_extra is not None
    assert torch.equal(kc_a, kc_b) and torch.equal(vc_a, vc_b)
    assert torch.equal(sep, fused)


def test_foreign_contract_family_takes_the_fused_path(gpu, monkeypatch):
    # The backend built on another class family (as on the reference's own
    # AttentionPlan) must still fold the store into the decode launch.
    from my_vllm_amd.attention_backend import integrate
    from tests import _foreign_contract as foreign

    class Registry(foreign.ForeignRegistry):
        backends = {}

    unified, _ = integrate(Registry, foreign.ForeignBackendBase, foreign.ForeignPlan, foreign.ForeignRoute,
                           foreign.ForeignBatchType, foreign.ForeignCommon)
    batch = config_decode_small(seed=1)
    common, q, kc, vc = to_device(batch, gpu)
    k_new, v_new = batch.k_new.to(gpu), batch.v_new.to(gpu)
    backend = unified(16, 8, 128, 16, torch.bfloat16)
    plan = backend.build_plan(foreign.to_foreign(common))
    assert type(plan) is foreign.ForeignPlan and plan.route is foreign.ForeignRoute.DECODE
    fused_calls = []
    real = ops.paged_decode_store
    monkeypatch.setattr(ops, "paged_decode_store", lambda *a, **k: (fused_calls.append(1), real(*a, **k))[1])
    kc_b, vc_b = kc.clone(), vc.clone()
    fused = backend.forward_with_kv_store(q, k_new, v_new, kc_b, vc_b, common.slot_mapping, plan).clone()
    assert fused_calls == [1]
    own = MI355XAttentionBackend(16, 8, 128, 16, torch.bfloat16)
    ops.store_kvcache(k_new, v_new, kc, vc, common.slot_mapping)
    sep = own.forward(q, k_new, v_new, kc, vc, own.build_plan(common))
    assert torch.equal(kc, kc_b) and torch.equal(vc, vc_b) and torch.equal(sep, fused)
