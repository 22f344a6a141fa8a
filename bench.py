"""Benchmark of the MI355X ragged-batch attention hot path (one GPU).

Headline (``value``): one step = slot_mapping KV store + PURE_DECODE paged GQA
attention at the Qwen3-0.6B shape (16 Q / 8 KV heads, head_dim 128, bf16,
16-token pages, 64 sequences with contexts uniform in [128, 2048], seed 1),
reported as algorithmic HBM GB/s of the whole step.  Inputs are resident in
HBM before timing; four copies of the KV cache are rotated so the 256 MB
Infinity Cache cannot serve a step from the previous one.

Also reported (``extra``): SiLU-and-mul GB/s (4096 x 6144 and 8192 x 51200),
PURE_PREFILL TFLOP/s (Qwen3-8B, 16 sequences with prefixes), MIXED tokens/s
(single launch vs split launches) and long-context decode GB/s (Qwen3-32B,
batch 128, contexts 8K-32K).  ``roofline`` covers the decode kernel alone,
timed with HIP events on the stream it is launched on; ``cpu_baseline`` times
the CPU oracle (the reference's fp32 paged-attention restatement) on a
bounded sample of the same workload on the host cores.

Every figure is the median of 5 timed regions (HIP events on the launch
stream).  Prefill and MIXED inputs are the CPU-seeded draws the parity tests
check; the 10.7 GB long-decode batch is drawn on the GPU, as its test does.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extra]
       python bench.py --only {decode,decode_store,long_decode,prefill,mixed,silu,store,rms,prologue,copy} [--steps K]
The ``--only`` forms run one workload's kernel K times and print one line;
they are the programs the committed rocprofv3 summaries profile (``copy`` is
a 256 MiB device copy used to calibrate the byte counters).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import torch

HBM_PEAK_GBPS = 8000.0
# Timed regions per figure; the median is reported.
REPEATS = 5
BF16_PEAK_TFLOPS = 2500.0
METRIC = "paged GQA decode HBM GB/s (% of peak); mixed-batch attention tokens/s"


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-extra", action="store_true", help="headline and roofline only")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample budget")
    ap.add_argument("--only", choices=["decode", "decode_store", "long_decode", "prefill", "mixed", "silu", "store",
                                       "rms", "prologue",
                                       "copy"],
                    help="run one workload's kernel --steps times (for profilers) and exit")
    return ap.parse_args(argv)


def to_device(batch, device):
    c = batch.common
    common = type(c)(**{**c.__dict__,
                        "query_start_loc": c.query_start_loc.to(device),
                        "seq_lens": c.seq_lens.to(device),
                        "slot_mapping": c.slot_mapping.to(device),
                        "block_tables": c.block_tables.to(device)})
    return common


def time_launches(fn, iters: int, warmup: int, repeats: int = 1) -> float:
    """ms per call of `fn`: the median over `repeats` timed regions of `iters`
    calls each, timed with HIP events on the current stream (the stream the
    kernels are launched on).  `fn(i)` gets a running call index, which the
    callers use to rotate input copies."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    per_call = []
    n = warmup
    for _ in range(repeats):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(iters):
            fn(n)
            n += 1
        end.record()
        torch.cuda.synchronize()
        per_call.append(start.elapsed_time(end) / iters)
    return statistics.median(per_call)


def time_interleaved(fns, iters: int, warmup: int, repeats: int) -> list[float]:
    """ms per call of each of `fns`, timed as time_launches does but in
    alternating regions (the order reversed every other round), so that the
    clock's swings under back-to-back MFMA work fall on all of them alike."""
    for fn in fns:
        for i in range(warmup):
            fn(i)
    torch.cuda.synchronize()
    per_call = [[] for _ in fns]
    for r in range(repeats):
        order = range(len(fns)) if r % 2 == 0 else reversed(range(len(fns)))
        for k in order:
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            for i in range(iters):
                fns[k](i)
            end.record()
            torch.cuda.synchronize()
            per_call[k].append(start.elapsed_time(end) / iters)
    return [statistics.median(x) for x in per_call]


def decode_bytes(batch, num_q_heads, num_kv_heads, elem=2) -> int:
    """Algorithmic bytes of one decode launch: unique K/V rows read, q read,
    o written, page ids and seq_lens read."""
    kv = sum(batch.kv_lengths) * num_kv_heads * 128 * elem * 2
    qo = 2 * len(batch.kv_lengths) * num_q_heads * 128 * elem
    meta = sum(batch.block_counts) * 4 + len(batch.kv_lengths) * 4
    return kv + qo + meta


def store_bytes(num_tokens, num_kv_heads, elem=2) -> int:
    """KV store: read K and V rows, write them to the cache, read slots."""
    return num_tokens * (4 * num_kv_heads * 128 * elem + 4)


def causal_pairs(q_lens, kv_lens) -> int:
    return sum(q * (kv - q) + q * (q + 1) // 2 for q, kv in zip(q_lens, kv_lens))


def headline(args, device):
    from my_vllm_amd import ops
    from my_vllm_amd.layers import KVCacheStore
    from my_vllm_amd.attention_backend import MI355XAttentionBackend
    from my_vllm_amd.custom_op import CustomOpConfig
    from workloads import config_decode_small

    batch = config_decode_small(seed=1)
    hq, hkv = 16, 8
    common = to_device(batch, device)
    q = batch.q.to(device)
    k_new, v_new = batch.k_new.to(device), batch.v_new.to(device)
    copies = 4
    caches = [(batch.k_cache.to(device), batch.v_cache.to(device)) for _ in range(copies)]
    backend = MI355XAttentionBackend(hq, hkv, 128, 16, torch.bfloat16)
    store = KVCacheStore(CustomOpConfig(platform="cuda"))
    plan = backend.build_plan(common)
    empty = q.new_empty((0, hkv, 128))

    def step(i):
        # Attention.forward's store + attention, as the layer calls it: the
        # backend folds the store into the piece-list decode launch.
        kc, vc = caches[i % copies]
        backend.forward_with_kv_store(q, k_new, v_new, kc, vc, common.slot_mapping, plan, store)

    torch.cuda.synchronize()
    ms_step = time_launches(step, args.steps, args.warmup, repeats=REPEATS)
    step_bytes = decode_bytes(batch, hq, hkv) + store_bytes(len(batch.kv_lengths), hkv)

    # Roofline of the decode kernel alone: direct launches (no store), same
    # rotation, timed on the launch stream.
    md = plan.metadata
    out = torch.empty_like(q)
    ws = backend._get_workspace(
        ops.decode_workspace_bytes(md.num_decode_part_slots, hkv, hq // hkv), device)

    def decode_only(i):
        kc, vc = caches[i % copies]
        ops.paged_decode(q, kc, vc, md.block_tables, md.seq_lens, md.decode_items, md.num_decode_items,
                         md.num_decode_waves, md.decode_merges, md.num_decode_merges,
                         md.num_decode_part_slots, out, ws, backend.softmax_scale,
                         md.decode_wave_extra, md.decode_waves_per_group)

    ms_decode = time_launches(decode_only, max(args.steps, 500), args.warmup, repeats=REPEATS)
    dec_bytes = decode_bytes(batch, hq, hkv)
    achieved = dec_bytes / ms_decode / 1e6
    return {
        "ms_per_step": ms_step,
        "value": step_bytes / ms_step / 1e6,
        "decode_ms": ms_decode,
        "decode_bytes": dec_bytes,
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": measured_traffic(),
            "kernel": "paged_decode_kernel<bf16> + decode_merge_kernel<bf16> (one mva_paged_decode call)",
            "bytes_per_launch": dec_bytes,
            "avg_launch_ms": round(ms_decode, 5),
        },
        "batch": batch,
        "waves": md.num_decode_waves,
        "items": md.num_decode_items,
        "schedule": "piece lists" if md.decode_wave_extra is not None else "claims",
    }


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_rate(fn, nbytes: int, seconds: float) -> tuple[float, int]:
    """GB/s of `fn` (moving `nbytes` per call) over about `seconds` of calls."""
    fn()  # warm up
    reps = 0
    t0 = time.perf_counter()
    while True:
        fn()
        reps += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = (time.perf_counter() - t0) / reps
    return nbytes / dt / 1e9, reps


def cpu_baseline(batch, seconds: float):
    """The reference's native paths as restated by the CPU oracle, timed on
    this host's cores: fp32 paged attention (the reference's test oracle; its
    only CPU attention) on the first 16 sequences of the headline batch
    (`value`, GB/s of K/V), plus the SiLU-and-mul eager path at the
    Qwen3-0.6B MLP shape and the index_copy_ KV store of 16384 tokens."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle.reference import kv_store_index_copy, paged_attention, silu_and_mul_eager
    from workloads import silu_input

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    n = 16
    q_rows = sum(batch.query_lengths[:n])
    args = (batch.q[:q_rows], batch.k_cache, batch.v_cache, batch.common.block_tables[:n],
            batch.query_lengths[:n], batch.kv_lengths[:n])
    kv_bytes = sum(batch.kv_lengths[:n]) * 8 * 128 * 2 * 2
    attn_gbps, attn_reps = _cpu_rate(lambda: paged_attention(*args), kv_bytes, seconds)

    x = silu_input(4096, 6144, seed=0)
    silu_gbps, silu_reps = _cpu_rate(lambda: silu_and_mul_eager(x), 75497472, seconds / 2)

    tokens, hkv = 16384, 8
    gen = torch.Generator().manual_seed(5)
    key = torch.randn(tokens, hkv, 128, generator=gen).bfloat16()
    value = torch.randn(tokens, hkv, 128, generator=gen).bfloat16()
    pages = tokens // 16 + 64
    k_cache = torch.zeros(pages, 16, hkv, 128, dtype=torch.bfloat16)
    v_cache = torch.zeros_like(k_cache)
    slots = torch.randperm(pages * 16, generator=gen)[:tokens].to(torch.int32)
    store_gbps, store_reps = _cpu_rate(lambda: kv_store_index_copy(key, value, k_cache, v_cache, slots),
                                       store_bytes(tokens, hkv), seconds / 2)
    return {
        "value": round(attn_gbps, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "cpu_model": cpu_model(),
        "sample": f"oracle.reference.paged_attention (fp32 einsum, the reference's test oracle) on sequences "
                  f"0-15 of the headline batch ({sum(batch.kv_lengths[:n])} keys), {attn_reps} reps in "
                  f"{seconds:.0f}s on {cores} threads",
        "legs": {
            "silu_and_mul_eager_4096x6144_GBps": round(silu_gbps, 3),
            "silu_and_mul_eager_reps": silu_reps,
            "kv_store_index_copy_16384tok_GBps": round(store_gbps, 3),
            "kv_store_index_copy_reps": store_reps,
        },
    }


def extra_measurements(device, steps: int):
    from my_vllm_amd import ops
    from my_vllm_amd.attention_backend import MI355XAttentionBackend
    from workloads import config_decode_small, config_long_decode, config_mixed, config_prefill, silu_input

    res = {}
    # SiLU-and-mul, Qwen3-0.6B MLP: 8 rotating inputs (600 MB > Infinity Cache).
    x = silu_input(4096, 6144, seed=0).to(device)
    xs = [x.clone() for _ in range(8)]
    ms = time_launches(lambda i: ops.silu_and_mul(xs[i % 8]), 400, 20)
    res["silu_4096x6144_GBps"] = round(75497472 / ms / 1e6, 1)
    del xs, x
    # SiLU-and-mul at intermediate 25600, 8192 tokens.
    x5 = silu_input(8192, 51200, seed=4, device=device, rng_device="cuda")
    ms = time_launches(lambda i: ops.silu_and_mul(x5), 50, 5)
    res["silu_8192x51200_GBps"] = round(8192 * 51200 * 2 * 1.5 / ms / 1e6, 1)
    del x5

    # RMSNorm and fused residual-add RMSNorm, 4096 tokens x 4096 (Qwen3-8B
    # hidden), 8 rotating inputs (the residual pair: 512 MB > Infinity Cache).
    from workloads import silu_input as _randn_rows

    xs = [_randn_rows(4096, 4096, seed=10 + i, device=device, rng_device="cuda") for i in range(8)]
    rs = [_randn_rows(4096, 4096, seed=20 + i, device=device, rng_device="cuda") for i in range(8)]
    w = torch.ones(4096, dtype=torch.bfloat16, device=device)
    row_bytes = 4096 * 4096 * 2
    ms = time_launches(lambda i: ops.rms_norm(xs[i % 8], w, 1e-6), 200, 20)
    res["rms_norm_4096x4096_GBps"] = round(2 * row_bytes / ms / 1e6, 1)
    ms = time_launches(lambda i: ops.fused_add_rms_norm(xs[i % 8], rs[i % 8], w, 1e-6), 200, 20)
    res["fused_add_rms_norm_4096x4096_GBps"] = round(4 * row_bytes / ms / 1e6, 1)
    del xs, rs

    res.update(prologue_fused_vs_separate(device))

    def attn_case(batch, hq, hkv, mode="unified", iters=20):
        backend = MI355XAttentionBackend(hq, hkv, 128, 16, torch.bfloat16, attention_mode=mode)
        common = to_device(batch, device)
        q = batch.q.to(device)
        kc, vc = batch.k_cache.to(device), batch.v_cache.to(device)
        plan = backend.build_plan(common)
        empty = q.new_empty((0, hkv, 128))
        # Median of 5 timed regions, as for the headline: one region of 20
        # MFMA-bound launches swings with the clock by 10% or more.
        return time_launches(lambda i: backend.forward(q, empty, empty, kc, vc, plan), iters, 3, repeats=5)

    # PURE_PREFILL with prefix, Qwen3-8B.
    # The same CPU-seeded draw the parity tests check.
    # The backend plans the tiles on a step's first layer and streams that
    # plan on the others, so this is the per-layer time; prefill_with_plan_*
    # is one launch that plans for itself (a one-layer step).
    batch = config_prefill(seed=2, device=device)
    flops = 4 * 128 * 32 * causal_pairs(batch.query_lengths, batch.kv_lengths)
    backend = MI355XAttentionBackend(32, 8, 128, 16, torch.bfloat16)
    common = to_device(batch, device)
    plan = backend.build_plan(common)
    md = plan.metadata
    q, kc, vc = batch.q.to(device), batch.k_cache.to(device), batch.v_cache.to(device)
    empty = q.new_empty((0, 8, 128))
    out = torch.empty_like(q)
    ws = torch.empty(ops.prefill_workspace_bytes(md.prefill_max_tiles), dtype=torch.uint8, device=device)
    n_seqs = len(batch.query_lengths)
    # Median of 9 regions of 20 launches each, the two in alternating regions.
    ms, ms_plan = time_interleaved([
        lambda i: backend.forward(q, empty, empty, kc, vc, plan),
        lambda i: ops.paged_prefill(q, kc, vc, md.block_tables, md.seq_lens, md.query_start_loc, n_seqs,
                                    md.prefill_max_tiles, ws, out, backend.softmax_scale, validate=False),
    ], 20, 3, 9)
    res["prefill_TFLOPs"] = round(flops / ms / 1e9, 1)
    res["prefill_ms"] = round(ms, 4)
    res["prefill_with_plan_TFLOPs"] = round(flops / ms_plan / 1e9, 1)
    res["prefill_with_plan_ms"] = round(ms_plan, 4)
    del batch, q, kc, vc, out, ws, backend, plan

    # MIXED, Qwen3-8B, token budget 8192.
    batch = config_mixed(seed=3, device=device)
    t = sum(batch.query_lengths)
    ms_u = attn_case(batch, 32, 8, "unified")
    ms_s = attn_case(batch, 32, 8, "split")
    dec_bytes = sum(batch.kv_lengths[4:]) * 8 * 128 * 2 * 2
    pf_flops = 4 * 128 * 32 * causal_pairs(batch.query_lengths[:4], batch.kv_lengths[:4])
    bound_ms = max(dec_bytes / HBM_PEAK_GBPS / 1e6, pf_flops / BF16_PEAK_TFLOPS / 1e9)
    res["mixed_tokens"] = t
    res["mixed_unified_tokens_per_s"] = round(t / ms_u * 1e3, 1)
    res["mixed_split_tokens_per_s"] = round(t / ms_s * 1e3, 1)
    res["mixed_unified_ms"] = round(ms_u, 4)
    res["mixed_split_ms"] = round(ms_s, 4)
    res["mixed_unified_roofline_frac"] = round(bound_ms / ms_u, 4)
    res.update(host_planning(device, [("mixed_budget8192", batch, 32, 8)]))
    del batch

    # Context for the MFMA-bound figures: the vendor library's dense bf16 GEMM
    # on N(0,1) operands.  The chip holds lower clocks under dense MFMA work
    # on real data than the 2.5 PFLOP/s peak assumes.  Run after the attention
    # cases: its heat would lower their clocks.
    ga = _randn_rows(8192, 8192, seed=30, device=device, rng_device="cuda")
    gb = _randn_rows(8192, 8192, seed=31, device=device, rng_device="cuda")
    ms = time_launches(lambda i: torch.matmul(ga, gb), 30, 5)
    res["gemm_8192_bf16_TFLOPs"] = round(2 * 8192**3 / ms / 1e9, 1)
    del ga, gb

    res.update(graph_vs_eager(device))
    res.update(host_planning(device, [("decode_64seq", config_decode_small(seed=1), 16, 8)]))

    # Long-context decode, Qwen3-32B (one layer's KV, ~10.7 GB).
    batch = config_long_decode(seed=4, device=device, rng_device="cuda")
    ms = attn_case(batch, 64, 8, iters=10)
    gbps = decode_bytes(batch, 64, 8) / ms / 1e6
    res["long_decode_GBps"] = round(gbps, 1)
    res["long_decode_frac"] = round(gbps / HBM_PEAK_GBPS, 4)
    del batch
    torch.cuda.empty_cache()
    return res


def prologue_bytes(tokens: int, hq: int, hkv: int) -> int:
    """Algorithmic HBM bytes of one fused prologue launch: read each q, k and v
    row once; write q and k back in place and k and v into the cache (bf16,
    128 per row)."""
    rows_read = hq + 2 * hkv
    rows_written = (hq + hkv) + 2 * hkv
    return tokens * (rows_read + rows_written) * 128 * 2


def prologue_fused_vs_separate(device, tokens: int = 4096, hq: int = 32, hkv: int = 8):
    """Attention prologue at the Qwen3-8B shape for a 4096-token chunk: q/k
    RMSNorm + RoPE + KV store as one launch vs the four separate ops."""
    from my_vllm_amd import ops
    from my_vllm_amd.custom_op import CustomOpConfig
    from my_vllm_amd.layers import RotaryEmbedding
    from workloads import silu_input as _randn_rows

    width = (hq + 2 * hkv) * 128
    qkv = _randn_rows(tokens, width, seed=30, device=device, rng_device="cuda")
    q = qkv[:, : hq * 128].view(tokens, hq, 128)
    k = qkv[:, hq * 128:(hq + hkv) * 128].view(tokens, hkv, 128)
    v = qkv[:, (hq + hkv) * 128:].view(tokens, hkv, 128)
    pos = torch.arange(tokens, device=device, dtype=torch.int64)
    table = RotaryEmbedding(128, 128, 40960, 1e6, CustomOpConfig(platform="cuda")).cos_sin_cache.to(device)
    w = torch.ones(128, dtype=torch.bfloat16, device=device)
    pages = tokens // 16
    kc = torch.zeros(pages, 16, hkv, 128, dtype=torch.bfloat16, device=device)
    vc = torch.zeros_like(kc)
    slots = torch.arange(tokens, dtype=torch.int32, device=device)

    def fused(_):
        ops.qk_norm_rope_store(pos, q, k, table, w, w, 1e-6, v, kc, vc, slots)

    def separate(_):
        qn = ops.rms_norm(q, w, 1e-6)
        kn = ops.rms_norm(k, w, 1e-6)
        qr, kr = ops.rotary_embedding(pos, qn, kn, table)
        ops.store_kvcache(kr, v, kc, vc, slots)

    fused_ms = time_launches(fused, 200, 20)
    sep_ms = time_launches(separate, 200, 20)
    moved = prologue_bytes(tokens, hq, hkv)
    return {"prologue_4096tok_fused_us": round(fused_ms * 1e3, 2),
            "prologue_4096tok_separate_us": round(sep_ms * 1e3, 2),
            "prologue_4096tok_fused_GBps": round(moved / fused_ms / 1e6, 1)}


def host_planning(device, cases, reps: int = 200):
    """Host time of one step's planning (``build_plan``: metadata checks, the
    decode planner, the pinned staging copy) per ``(name, batch, hq, hkv)``
    case, trusted metadata as the engine passes it; the copies are left in
    flight, as in a serving loop."""
    from my_vllm_amd.attention_backend import MI355XAttentionBackend

    res = {}
    for name, batch, hq, hkv in cases:
        backend = MI355XAttentionBackend(hq, hkv, 128, 16, torch.bfloat16)
        common = to_device(batch, device)
        for _ in range(10):
            backend.build_plan(common)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            backend.build_plan(common)
        res[f"build_plan_{name}_host_us"] = round((time.perf_counter() - t0) / reps * 1e6, 1)
        torch.cuda.synchronize()
    return res


def graph_vs_eager(device, batch_size: int = 8, ctx: int = 512, steps: int = 200):
    """Launch-bound decode step (KV store + attention) for a small batch at the
    Qwen3-0.6B shape: eager launches vs one replay of a captured HIP graph of
    the same two launches, per step (plan built once, as in steady decode)."""
    from my_vllm_amd.layers import KVCacheStore
    from my_vllm_amd.attention_backend import MI355XAttentionBackend
    from my_vllm_amd.custom_op import CustomOpConfig
    from workloads import make_paged_batch

    hq, hkv = 16, 8
    batch = make_paged_batch(7, [1] * batch_size, [ctx] * batch_size, 0, hq, hkv)
    common = to_device(batch, device)
    q = batch.q.to(device)
    k_new, v_new = batch.k_new.to(device), batch.v_new.to(device)
    kc, vc = batch.k_cache.to(device), batch.v_cache.to(device)
    backend = MI355XAttentionBackend(hq, hkv, 128, 16, torch.bfloat16)
    store = KVCacheStore(CustomOpConfig(platform="cuda"))
    plan = backend.build_plan(common)
    empty = q.new_empty((0, hkv, 128))

    def step(_):
        store(k_new, v_new, kc, vc, common.slot_mapping)
        backend.forward(q, empty, empty, kc, vc, plan)

    eager_ms = time_launches(step, steps, 10)
    state = backend.create_full_decode_graph_state(batch_size, sum(batch.block_counts), device)
    backend.plan_full_decode_graph(state, plan)
    backend.activate_full_decode_graph(state)
    try:
        step(0)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step(0)
        torch.cuda.synchronize()
    finally:
        backend.deactivate_full_decode_graph()
    graph_ms = time_launches(lambda i: graph.replay(), steps, 10)
    return {"decode_step_8seq_eager_us": round(eager_ms * 1e3, 2), "decode_step_8seq_graph_us": round(graph_ms * 1e3, 2)}


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "paged_decode_64seq_ctx128-2048_traffic.txt")


def measured_traffic():
    """HBM bytes per decode launch from the committed counter passes, or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch="):
                    return int(line.split("=", 1)[1])
    except OSError:
        return None
    return None


def run_only(args, device):
    """One workload's kernel, --steps launches, for rocprofv3 passes."""
    from my_vllm_amd import ops
    from my_vllm_amd.attention_backend import MI355XAttentionBackend
    from workloads import (config_decode_small, config_long_decode, config_mixed, config_prefill,
                                       silu_input)

    n = args.steps
    if args.only == "copy":
        a = torch.empty(256 << 20, dtype=torch.uint8, device=device)
        b = torch.empty_like(a)
        for _ in range(n):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"only": "copy", "bytes_read_per_launch": 256 << 20, "bytes_written_per_launch": 256 << 20,
                          "launches": n}))
        return 0
    if args.only == "silu":
        # 8 rotated inputs (600 MB, past the 256 MB Infinity Cache).
        x = silu_input(4096, 6144, seed=0).to(device)
        xs = [x.clone() for _ in range(8)]
        for i in range(n):
            ops.silu_and_mul(xs[i % 8])
        torch.cuda.synchronize()
        print(json.dumps({"only": "silu", "bytes_per_launch": 75497472, "launches": n, "rotated_inputs": 8}))
        return 0
    if args.only == "rms":
        # Fused residual-add RMSNorm, 4096 x 4096 (Qwen3-8B hidden), 8 rotated
        # input / residual pairs (512 MB, past the 256 MB Infinity Cache).
        xs = [silu_input(4096, 4096, seed=10 + i, device=device, rng_device="cuda") for i in range(8)]
        rs = [silu_input(4096, 4096, seed=20 + i, device=device, rng_device="cuda") for i in range(8)]
        w = torch.ones(4096, dtype=torch.bfloat16, device=device)
        for i in range(n):
            ops.fused_add_rms_norm(xs[i % 8], rs[i % 8], w, 1e-6)
        torch.cuda.synchronize()
        print(json.dumps({"only": "rms", "bytes_per_launch": 4 * 4096 * 4096 * 2, "launches": n,
                          "rotated_inputs": 8}))
        return 0
    if args.only == "prologue":
        # Fused q/k-RMSNorm + RoPE + KV store, 4096 tokens at Qwen3-8B heads
        # (32 Q / 8 KV), 6 rotated qkv buffers (300 MB, past the Infinity Cache).
        from my_vllm_amd.custom_op import CustomOpConfig
        from my_vllm_amd.layers import RotaryEmbedding

        tokens, hq, hkv = 4096, 32, 8
        width = (hq + 2 * hkv) * 128
        qkvs = [silu_input(tokens, width, seed=30 + i, device=device, rng_device="cuda") for i in range(6)]
        pos = torch.arange(tokens, device=device, dtype=torch.int64)
        table = RotaryEmbedding(128, 128, 40960, 1e6, CustomOpConfig(platform="cuda")).cos_sin_cache.to(device)
        w = torch.ones(128, dtype=torch.bfloat16, device=device)
        kc = torch.zeros(tokens // 16, 16, hkv, 128, dtype=torch.bfloat16, device=device)
        vc = torch.zeros_like(kc)
        slots = torch.arange(tokens, dtype=torch.int32, device=device)
        for i in range(n):
            qkv = qkvs[i % 6]
            q = qkv[:, : hq * 128].view(tokens, hq, 128)
            k = qkv[:, hq * 128:(hq + hkv) * 128].view(tokens, hkv, 128)
            v = qkv[:, (hq + hkv) * 128:].view(tokens, hkv, 128)
            ops.qk_norm_rope_store(pos, q, k, table, w, w, 1e-6, v, kc, vc, slots)
        torch.cuda.synchronize()
        print(json.dumps({"only": "prologue", "bytes_per_launch": prologue_bytes(tokens, hq, hkv),
                          "launches": n, "rotated_inputs": 6}))
        return 0
    if args.only == "store":
        # 16384 new tokens (a 16K-token prefill chunk) at 8 KV heads, scattered
        # to random slots of a 1.1 GB cache pair; 4 rotated inputs.
        tokens, hkv = 16384, 8
        gen = torch.Generator(device=device).manual_seed(5)
        keys = [torch.randn(tokens, hkv, 128, generator=gen, device=device).bfloat16() for _ in range(4)]
        vals = [torch.randn(tokens, hkv, 128, generator=gen, device=device).bfloat16() for _ in range(4)]
        pages = 32768
        k_cache = torch.zeros(pages, 16, hkv, 128, dtype=torch.bfloat16, device=device)
        v_cache = torch.zeros_like(k_cache)
        slots = [torch.randperm(pages * 16, generator=gen, device=device)[:tokens].to(torch.int32)
                 for _ in range(4)]
        for i in range(n):
            ops.store_kvcache(keys[i % 4], vals[i % 4], k_cache, v_cache, slots[i % 4])
        torch.cuda.synchronize()
        print(json.dumps({"only": "store", "bytes_per_launch": store_bytes(tokens, hkv), "launches": n,
                          "rotated_inputs": 4}))
        return 0
    if args.only == "decode_store":
        # The headline step's kernel: the KV store folded into the decode launch.
        from my_vllm_amd.layers import KVCacheStore
        from my_vllm_amd.custom_op import CustomOpConfig

        batch, hq, hkv = config_decode_small(seed=1), 16, 8
        common = to_device(batch, device)
        q = batch.q.to(device)
        k_new, v_new = batch.k_new.to(device), batch.v_new.to(device)
        caches = [(batch.k_cache.to(device), batch.v_cache.to(device)) for _ in range(4)]
        backend = MI355XAttentionBackend(hq, hkv, 128, 16, torch.bfloat16)
        store = KVCacheStore(CustomOpConfig(platform="cuda"))
        plan = backend.build_plan(common)
        for i in range(n):
            kc, vc = caches[i % 4]
            backend.forward_with_kv_store(q, k_new, v_new, kc, vc, common.slot_mapping, plan, store)
        torch.cuda.synchronize()
        print(json.dumps({"only": "decode_store", "bytes_per_launch": decode_bytes(batch, hq, hkv)
                          + store_bytes(len(batch.kv_lengths), hkv), "launches": n}))
        return 0
    if args.only in ("decode", "long_decode"):
        if args.only == "decode":
            batch, hq, hkv, copies = config_decode_small(seed=1), 16, 8, 4
        else:
            batch, hq, hkv, copies = config_long_decode(seed=4, device=device, rng_device="cuda"), 64, 8, 1
        common = to_device(batch, device)
        q = batch.q.to(device)
        caches = [(batch.k_cache.to(device), batch.v_cache.to(device)) for _ in range(copies)]
        backend = MI355XAttentionBackend(hq, hkv, 128, 16, torch.bfloat16)
        md = backend.build_plan(common).metadata
        out = torch.empty_like(q)
        ws = backend._get_workspace(
            ops.decode_workspace_bytes(md.num_decode_part_slots, hkv, hq // hkv), device)
        for i in range(n):
            kc, vc = caches[i % copies]
            ops.paged_decode(q, kc, vc, md.block_tables, md.seq_lens, md.decode_items, md.num_decode_items,
                             md.num_decode_waves, md.decode_merges, md.num_decode_merges,
                             md.num_decode_part_slots, out, ws, backend.softmax_scale,
                             md.decode_wave_extra, md.decode_waves_per_group)
        torch.cuda.synchronize()
        print(json.dumps({"only": args.only, "bytes_per_launch": decode_bytes(batch, hq, hkv), "launches": n,
                          "waves": md.num_decode_waves, "pieces": md.num_decode_items}))
        return 0
    batch = (config_prefill if args.only == "prefill" else config_mixed)(seed=2 if args.only == "prefill" else 3,
                                                                        device=device)
    backend = MI355XAttentionBackend(32, 8, 128, 16, torch.bfloat16)
    common = to_device(batch, device)
    q = batch.q.to(device)
    kc, vc = batch.k_cache.to(device), batch.v_cache.to(device)
    plan = backend.build_plan(common)
    empty = q.new_empty((0, 8, 128))
    for _ in range(n):
        backend.forward(q, empty, empty, kc, vc, plan)
    torch.cuda.synchronize()
    print(json.dumps({"only": args.only, "tokens": sum(batch.query_lengths), "launches": n,
                      "route": plan.route.value}))
    return 0


def main(argv=None):
    args = parse_args(argv)
    if args.gpus != 1:
        print(
            f"bench.py measures one MI355X only; --gpus {args.gpus} is not supported "
            "(attention shards by KV head with no exchange; see the design notes)",
            file=sys.stderr,
        )
        return 2
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    from my_vllm_amd import _native

    _native.load_library()  # fails loudly when the gfx950 library is missing
    if args.only:
        return run_only(args, device)
    head = headline(args, device)
    extra = {} if args.no_extra else extra_measurements(device, args.steps)
    cpu = cpu_baseline(head["batch"], args.cpu_seconds)
    value = head["value"]
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: N(0,1) values, seeded lengths and page permutations",
        "config": {
            "workload": "slot_mapping KV store + PURE_DECODE paged GQA attention, 16 Q / 8 KV heads, "
                        "head_dim 128, bf16, page 16, 64 seqs, ctx U[128,2048] (seed 1), "
                        "4 rotated KV-cache copies",
            "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBPS, 2),
            "decode_waves": head["waves"],
            "decode_pieces": head["items"],
            "decode_schedule": head["schedule"],
        },
        "timing": f"median of {REPEATS} timed regions of {args.steps} steps each (HIP events), "
                  "4 KV-cache copies rotated",
        "roofline": head["roofline"],
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
