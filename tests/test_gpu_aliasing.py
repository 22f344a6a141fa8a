"""Same-step page aliasing: a prefix-cache follower reads pages its leader
writes in the same layer call.

The reference's end-to-end case (tests/test_e2e_flashinfer_attention.py:147-257):
the leader prefills 33 tokens (pages A, B, C) while the follower, whose first
32 tokens hit the prefix cache on the leader's pages A and B, prefills its
33rd token into its own page D.  The shared pages are NaN-filled first, so a
follower that read them before the leader's rows landed would produce NaN.
The layer call is ``Attention.forward``'s: the KV store, then attention
(here through ``forward_with_kv_store`` with the drop-in ``KVCacheStore``).

Run as PURE_PREFILL (the reference's batch) and as MIXED, with decode
sequences appended, on both MIXED routes.  The output must be finite, match
the fp32 oracle on the stored cache, and the follower's row must be bitwise
the same as with private copies of the two pages (the reference's second
run).
"""

import numpy as np
import pytest
import torch

from my_vllm_amd.attention_backend import MI355XAttentionBackend
from my_vllm_amd.contract import AttentionRoute, BatchType, CommonAttentionMetadata
from my_vllm_amd.custom_op import CustomOpConfig
from my_vllm_amd.layers import KVCacheStore
from oracle.reference import paged_attention
from tests._util import assert_attention_close

pytestmark = pytest.mark.gpu

HQ, HKV, D = 16, 8, 128


def _step(device, shared_pages, decode_ctx, seed=211):
    """One step's tensors: leader [A, B, C], follower [A', B', D] where
    (A', B') = shared_pages, then decode sequences on pages of their own."""
    gen = torch.Generator().manual_seed(seed)
    A, B, C, D_page = 0, 1, 2, 3
    private = [4, 5]
    next_page = 6
    tables = [[A, B, C], [*shared_pages, D_page]]
    for ctx in decode_ctx:
        n = (ctx + 15) // 16
        tables.append(list(range(next_page, next_page + n)))
        next_page += n
    q_lens = [33, 1] + [1] * len(decode_ctx)
    kv_lens = [33, 33] + list(decode_ctx)
    slots = [tables[0][i // 16] * 16 + i % 16 for i in range(33)] + [D_page * 16]
    slots += [tables[2 + j][(ctx - 1) // 16] * 16 + (ctx - 1) % 16 for j, ctx in enumerate(decode_ctx)]
    width = max(len(t) for t in tables)
    bt = np.full((len(tables), width), -1, dtype=np.int32)
    for s, t in enumerate(tables):
        bt[s, :len(t)] = t
    tokens = sum(q_lens)
    q = torch.randn(tokens, HQ, D, generator=gen).bfloat16()
    k_new = torch.randn(tokens, HKV, D, generator=gen).bfloat16()
    v_new = torch.randn(tokens, HKV, D, generator=gen).bfloat16()
    caches = torch.randn(2, next_page, 16, HKV, D, generator=gen).bfloat16()
    for page in (A, B, C, D_page):  # stale: written by nobody before this step
        caches[:, page] = float("nan")
    # The follower's cached prefix is the leader's first 32 rows: private
    # copies hold what the leader writes into A and B this step.
    leader_rows_k, leader_rows_v = k_new[:32].view(2, 16, HKV, D), v_new[:32].view(2, 16, HKV, D)
    caches[0, private], caches[1, private] = leader_rows_k, leader_rows_v
    counts = tuple(len(t) for t in tables)
    num_prefill = 2
    common = CommonAttentionMetadata(
        num_prefill_seqs=num_prefill, num_decode_seqs=len(decode_ctx),
        num_prefill_tokens=34, num_decode_tokens=len(decode_ctx),
        query_start_loc=torch.tensor(np.concatenate(([0], np.cumsum(q_lens))), dtype=torch.int32, device=device),
        seq_lens=torch.tensor(kv_lens, dtype=torch.int32, device=device),
        slot_mapping=torch.tensor(slots, dtype=torch.int32, device=device),
        block_tables=torch.from_numpy(bt).to(device), max_q_len=33, max_kv_len=max(kv_lens),
        block_counts=counts, num_kv_blocks=sum(counts), num_prefill_kv_blocks=sum(counts[:num_prefill]),
        trusted=True,
    )
    return common, q, k_new, v_new, caches, q_lens, kv_lens, bt


def _layer_call(device, mode, shared_pages, decode_ctx):
    common, q, k_new, v_new, caches, q_lens, kv_lens, bt = _step(device, shared_pages, decode_ctx)
    backend = MI355XAttentionBackend(HQ, HKV, D, 16, torch.bfloat16, attention_mode=mode)
    store = KVCacheStore(CustomOpConfig(platform="cuda"))
    kc, vc = caches[0].to(device), caches[1].to(device)
    plan = backend.build_plan(common)
    out = backend.forward_with_kv_store(q.to(device), k_new.to(device), v_new.to(device), kc, vc,
                                        common.slot_mapping, plan, store).cpu()
    return plan, out, kc.cpu(), vc.cpu(), q, q_lens, kv_lens, bt


@pytest.mark.parametrize("mode,decode_ctx,batch_type,route", [
    ("unified", (), BatchType.PURE_PREFILL, AttentionRoute.PREFILL),
    ("unified", (40, 300, 2049), BatchType.MIXED, AttentionRoute.MIXED_UNIFIED),
    ("split", (40, 300, 2049), BatchType.MIXED, AttentionRoute.MIXED_SPLIT),
])
def test_follower_reads_the_leaders_rows_of_this_step(gpu, mode, decode_ctx, batch_type, route):
    plan, out, kc, vc, q, q_lens, kv_lens, bt = _layer_call(gpu, mode, [0, 1], decode_ctx)
    assert plan.batch_type is batch_type and plan.route is route
    assert torch.isfinite(out).all(), "a stale (NaN) shared page was read"
    assert torch.isfinite(kc[:2]).all() and torch.isfinite(vc[:2]).all()
    expected = paged_attention(q, kc, vc, torch.from_numpy(bt), q_lens, kv_lens)
    assert_attention_close(out, expected)
    # The reference's second run: the follower on private copies of A and B.
    _, private_out, *_ = _layer_call(gpu, mode, [4, 5], decode_ctx)
    assert torch.equal(out[33], private_out[33])
    assert torch.equal(out, private_out)
