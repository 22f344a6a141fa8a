"""Long-context decode at Qwen3-32B shape and SiLU-and-mul at intermediate
25600, at full size on one GPU.

Decode: 64 Q / 8 KV heads, head_dim 128, bf16, 16-token pages, batch 128 with
contexts uniform in [8192, 32768] (seed 4) over randomly permuted pages: one
layer's K/V, about 11.2 GB, drawn on the GPU.  With 8 KV heads the backend
plans piece lists at any size; the claim schedule is forced on the same
batch as well.  The shortest, the longest and
two random sequences are checked against the fp32 oracle on the host (their
pages gathered from the device), and every output row must be finite.

SiLU: x [8192, 51200] ~ N(0, 1) (seed 4) -> [8192, 25600]; every 16th row is
checked against the fused closed form within 1 bf16 ulp.
"""

import numpy as np
import pytest
import torch

from my_vllm_amd import ops
from my_vllm_amd.attention_backend import MI355XAttentionBackend
from my_vllm_amd.contract import AttentionRoute
from oracle.reference import paged_attention, silu_and_mul_fused
from tests._util import assert_attention_close, max_ulp_diff, set_decode_planning
from workloads import config_long_decode, silu_input

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def long_batch(gpu):
    batch = config_long_decode(seed=4, device=gpu, rng_device="cuda")
    c = batch.common
    assert c.query_start_loc.is_cuda and batch.k_cache.is_cuda
    yield batch
    del batch
    torch.cuda.empty_cache()


def _host_expected(batch, seqs):
    """Oracle output rows of `seqs`, from their pages copied to the host."""
    bt = batch.block_tables_host
    rows = []
    for s in seqs:
        count = batch.block_counts[s]
        pages = torch.from_numpy(bt[s, :count].astype(np.int64)).to(batch.k_cache.device)
        k = batch.k_cache.index_select(0, pages).cpu()
        v = batch.v_cache.index_select(0, pages).cpu()
        table = torch.arange(count, dtype=torch.int32).unsqueeze(0)
        rows.append(paged_attention(batch.q[s:s + 1].cpu(), k, v, table, [1], [batch.kv_lengths[s]]))
    return torch.cat(rows)


@pytest.mark.parametrize("schedule", ["default", "claims"])
def test_qwen3_32b_long_decode_configuration(gpu, long_batch, monkeypatch, schedule):
    batch = long_batch
    if schedule == "claims":
        set_decode_planning(monkeypatch, schedule="claims")
    backend = MI355XAttentionBackend(64, 8, 128, 16, torch.bfloat16)
    plan = backend.build_plan(batch.common)
    assert plan.route is AttentionRoute.DECODE
    if schedule == "default":
        assert plan.metadata.decode_wave_extra is not None, "8 KV heads plan piece lists at any size"
    else:
        assert plan.metadata.decode_wave_extra is None
    empty = batch.q.new_empty((0, 8, 128))
    out = backend.forward(batch.q, empty, empty, batch.k_cache, batch.v_cache, plan)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    lengths = batch.kv_lengths
    rng = np.random.default_rng(123)
    seqs = sorted({int(np.argmin(lengths)), int(np.argmax(lengths)), *map(int, rng.choice(128, 2, replace=False))})
    assert_attention_close(out[seqs].cpu(), _host_expected(batch, seqs))


def test_silu_and_mul_at_intermediate_25600(gpu):
    x = silu_input(8192, 51200, seed=4, device=gpu, rng_device="cuda")
    out = ops.silu_and_mul(x)
    assert out.shape == (8192, 25600) and out.is_contiguous()
    rows = torch.arange(0, 8192, 16, device=gpu)
    sample = x.index_select(0, rows).cpu()
    assert max_ulp_diff(out.index_select(0, rows).cpu(), silu_and_mul_fused(sample)) <= 1
    assert torch.isfinite(out).all()
