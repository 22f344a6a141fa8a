"""mva_paged_decode_noalloc (static device scratch) against mva_paged_decode
(caller workspace), both called through the C ABI.

Two calls in a row, the second on a smaller batch, must each give outputs
bitwise equal to the workspace entry point's on the same plan: first the
64-sequence Qwen3-0.6B decode batch on piece lists, then a 9-sequence batch
on the claim schedule (which needs the scratch's claim counters back at zero
after the first call), then the first batch again.  A plan whose partials
exceed the static scratch is refused before any launch.
"""

import pytest
import torch

from my_vllm_amd import _native, ops
from my_vllm_amd.attention_backend import MI355XAttentionBackend
from tests._util import set_decode_planning
from tests.test_gpu_prefill import to_device
from workloads import config_decode_small, decode_lengths, make_paged_batch

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20  # MVA_DECODE_STATIC_SCRATCH_BYTES


def _decode_args(batch, device, monkeypatch, schedule):
    set_decode_planning(monkeypatch, schedule=schedule)
    hq, hkv = batch.q.shape[1], batch.k_cache.shape[2]
    common, q, kc, vc = to_device(batch, device)
    md = MI355XAttentionBackend(hq, hkv, 128, 16, torch.bfloat16).build_plan(common).metadata
    assert (md.decode_wave_extra is not None) == (schedule == "listed")
    head = (q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(), kc.shape[0], kc.stride(0),
            kc.stride(1), md.block_tables.data_ptr(), md.block_tables.stride(0), md.seq_lens.data_ptr(),
            md.decode_items.data_ptr(), md.num_decode_items, md.num_decode_waves,
            md.decode_wave_extra.data_ptr() if md.decode_wave_extra is not None else 0,
            md.decode_waves_per_group, md.decode_merges.data_ptr() if md.num_decode_merges else 0,
            md.num_decode_merges, md.num_decode_part_slots)
    tail = (hq, hkv, 128, 16, 128 ** -0.5, _native.DTYPE_CODES[torch.bfloat16], _native.stream_handle(device))
    keep = (q, kc, vc, md)  # keep every tensor the pointers refer to alive
    return head, tail, keep, md


def _both(batch, device, monkeypatch, schedule):
    head, tail, keep, md = _decode_args(batch, device, monkeypatch, schedule)
    q = keep[0]
    ws = torch.zeros(ops.decode_workspace_bytes(md.num_decode_part_slots, tail[1], tail[0] // tail[1]),
                     dtype=torch.uint8, device=device)
    assert ws.numel() <= SCRATCH_BYTES
    out_ws = torch.full_like(q, float("nan"))
    out_static = torch.full_like(q, float("nan"))
    _native.call("mva_paged_decode", *head, out_ws.data_ptr(), out_ws.stride(0), out_ws.stride(1),
                 ws.data_ptr(), ws.numel(), *tail)
    _native.call("mva_paged_decode_noalloc", *head, out_static.data_ptr(), out_static.stride(0),
                 out_static.stride(1), *tail)
    torch.cuda.synchronize()
    return out_ws, out_static


def test_static_scratch_decode_matches_the_workspace_entry_point(gpu, monkeypatch):
    big = config_decode_small(seed=1)
    small = make_paged_batch(61, [1] * 9, decode_lengths(61, 9, 1, 700), 0, 16, 8)
    for batch, schedule in ((big, "listed"), (small, "claims"), (big, "listed")):
        out_ws, out_static = _both(batch, gpu, monkeypatch, schedule)
        assert torch.isfinite(out_ws).all()
        assert torch.equal(out_ws, out_static), schedule


def test_plans_beyond_the_static_scratch_are_refused(gpu):
    slots = SCRATCH_BYTES // (8 * 2 * 4 * 129) + 1  # partial rows past 64 MiB at Hkv=8, G=2
    assert ops.decode_workspace_bytes(slots, 8, 2) > SCRATCH_BYTES
    with pytest.raises(RuntimeError, match="static"):
        _native.call("mva_paged_decode_noalloc", *([0] * 18), slots, 0, 0, 0, 16, 8, 128, 16, 1.0, 0,
                     _native.stream_handle(gpu))
