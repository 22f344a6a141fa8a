"""CPU: the oracle's floating-point functions pinned by mathematics.

SiLU is checked against the closed form evaluated element by element with
``math.exp`` and against torch's ``F.silu``; attention against pure-Python
brute force on tiny inputs, against ``F.scaled_dot_product_attention`` on the
cacheless causal case, and against invariants (one-key context, equal scores,
split-K log-sum-exp merge).  Each check is chosen so that a plausible
mistake fails it; the planted-mistake tests show that on the CPU.
"""

import json
import math
from pathlib import Path

import pytest
import torch
import torch.nn.functional as F

from oracle import reference as ref
from tests._util import max_ulp_diff

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


# ---------------------------------------------------------------------------
# SiLU-and-mul
# ---------------------------------------------------------------------------

def _closed_form(x: torch.Tensor) -> torch.Tensor:
    """g * sigmoid(g) * u per element in Python floats, rounded once."""
    width = x.shape[-1] // 2
    flat = x.float().reshape(-1, x.shape[-1]).tolist()
    out = [[g / (1.0 + math.exp(-g)) * u for g, u in zip(row[:width], row[width:])] for row in flat]
    return torch.tensor(out, dtype=torch.float64).reshape(*x.shape[:-1], width).to(x.dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", KATS["silu"]["shapes"])
def test_silu_fused_matches_closed_form(dtype, shape):
    gen = torch.Generator().manual_seed(7)
    x = (torch.randn(shape, generator=gen) * 3).to(dtype)
    fused = ref.silu_and_mul_fused(x)
    assert fused.shape == (*shape[:-1], shape[-1] // 2) and fused.dtype == dtype
    # fp32 arithmetic vs double: at most one unit of the last place apart.
    assert max_ulp_diff(fused, _closed_form(x)) <= 1


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_silu_eager_is_torch_library_silu(dtype):
    x = torch.randn(31, 64, generator=torch.Generator().manual_seed(3)).to(dtype)
    a, b = x.chunk(2, -1)
    assert torch.equal(ref.silu_and_mul_eager(x), F.silu(a) * b)
    # Two roundings (eager) vs one (fused) differ by at most one ulp.
    assert max_ulp_diff(ref.silu_and_mul_eager(x), ref.silu_and_mul_fused(x)) <= 1


def test_silu_special_values():
    x = torch.tensor([[0.0, -30.0, 30.0, 2.0, 5.0, 3.0]], dtype=torch.float32)
    out = ref.silu_and_mul_fused(x)
    # silu(0) = 0; silu(-30) ~ -2.8e-12; silu(30) ~ 30
    assert out[0, 0].item() == 0.0
    assert abs(out[0, 1].item()) < 1e-10
    assert out[0, 2].item() == pytest.approx(90.0, rel=1e-6)


def test_planted_silu_mistake_is_caught():
    # A dropped sigmoid (g * u) must fail the closed-form check.
    x = torch.randn(4, 16, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    a, b = x.float().chunk(2, -1)
    wrong = (a * b).to(torch.bfloat16)
    assert max_ulp_diff(wrong, _closed_form(x)) > 1


# ---------------------------------------------------------------------------
# Paged attention
# ---------------------------------------------------------------------------

def _brute_force_paged(q, k_cache, v_cache, block_tables, q_lens, kv_lens):
    """Scalar loops: token (page, slot) lookup, causal bound, GQA head map."""
    page = k_cache.shape[1]
    hq, hkv, dim = q.shape[1], k_cache.shape[2], q.shape[2]
    group = hq // hkv
    scale = 1.0 / math.sqrt(dim)
    out = torch.zeros(q.shape, dtype=torch.float64)
    row = 0
    for s, (ql, kl) in enumerate(zip(q_lens, kv_lens)):
        for i in range(ql):
            last = kl - ql + i  # absolute position of query i
            for h in range(hq):
                kvh = h // group
                scores = []
                for j in range(last + 1):
                    pg = int(block_tables[s][j // page])
                    kv = k_cache[pg, j % page, kvh]
                    scores.append(sum(float(q[row, h, d]) * float(kv[d]) for d in range(dim)) * scale)
                top = max(scores)
                w = [math.exp(x - top) for x in scores]
                total = sum(w)
                for j in range(last + 1):
                    pg = int(block_tables[s][j // page])
                    for d in range(dim):
                        out[row, h, d] += w[j] / total * float(v_cache[pg, j % page, kvh, d])
            row += 1
    return out


def _tiny_case(seed, q_lens, kv_lens, hq, hkv, dim=8, page=4):
    gen = torch.Generator().manual_seed(seed)
    pages = sum((n + page - 1) // page for n in kv_lens) + 2
    perm = torch.randperm(pages, generator=gen).tolist()
    width = max((n + page - 1) // page for n in kv_lens)
    bt, used = [], 0
    for n in kv_lens:
        c = (n + page - 1) // page
        bt.append(perm[used : used + c] + [-1] * (width - c))
        used += c
    q = torch.randn(sum(q_lens), hq, dim, generator=gen)
    k_cache = torch.randn(pages, page, hkv, dim, generator=gen)
    v_cache = torch.randn(pages, page, hkv, dim, generator=gen)
    return q, k_cache, v_cache, torch.tensor(bt), q_lens, kv_lens


@pytest.mark.parametrize(
    "q_lens,kv_lens,hq,hkv",
    [([1, 1], [5, 9], 4, 2), ([3, 1], [7, 4], 4, 4), ([2, 3, 1], [2, 11, 6], 6, 2), ([4], [4], 2, 1)],
)
def test_paged_attention_matches_brute_force(q_lens, kv_lens, hq, hkv):
    q, kc, vc, bt, ql, kl = _tiny_case(11, q_lens, kv_lens, hq, hkv)
    got = ref.paged_attention(q, kc, vc, bt, ql, kl)
    torch.testing.assert_close(got.double(), _brute_force_paged(q, kc, vc, bt, ql, kl), atol=1e-5, rtol=1e-5)


def test_planted_causal_offset_mistake_is_caught():
    # Queries aligned to the start of the context (a dropped kv - q offset)
    # must fail the brute-force comparison.
    q, kc, vc, bt, ql, kl = _tiny_case(5, [3], [7], 2, 1)
    good = _brute_force_paged(q, kc, vc, bt, ql, kl)
    wrong = _brute_force_paged(q, kc, vc, bt, ql, [3])  # offset 0: sees keys j <= i only
    assert not torch.allclose(good, wrong, atol=1e-3)
    torch.testing.assert_close(ref.paged_attention(q, kc, vc, bt, ql, kl).double(), good, atol=1e-5, rtol=1e-5)


def test_planted_gqa_mapping_mistake_is_caught():
    # Query head h reads KV head h // G; a tiled map (h % Hkv) must differ.
    q, kc, vc, bt, ql, kl = _tiny_case(9, [1], [6], 4, 2)
    got = ref.paged_attention(q, kc, vc, bt, ql, kl)
    permuted = q.clone()
    permuted[:, [1, 2]] = q[:, [2, 1]]  # swap heads across groups
    tiled = ref.paged_attention(permuted, kc, vc, bt, ql, kl)[:, [0, 2, 1, 3]]
    assert not torch.allclose(got, tiled, atol=1e-3)


def test_one_key_context_returns_value_exactly():
    q, kc, vc, bt, ql, kl = _tiny_case(2, [1, 1], [1, 1], 4, 2)
    got = ref.paged_attention(q, kc, vc, bt, ql, kl)
    for s in range(2):
        expected = vc[int(bt[s][0]), 0].repeat_interleave(2, dim=0)
        torch.testing.assert_close(got[s], expected, atol=0, rtol=0)


def test_equal_scores_give_mean_of_values():
    q, kc, vc, bt, ql, kl = _tiny_case(4, [1], [10], 2, 1)
    q.zero_()
    got = ref.paged_attention(q, kc, vc, bt, ql, kl)
    keys = torch.cat([vc[int(p)] for p in bt[0][:3]])[:10]
    torch.testing.assert_close(got[0], keys.mean(0).repeat_interleave(2, dim=0), atol=1e-6, rtol=1e-6)


def test_ragged_attention_matches_sdpa():
    gen = torch.Generator().manual_seed(13)
    lengths = [3, 1, 6]
    q = torch.randn(10, 4, 16, generator=gen)
    k = torch.randn(10, 2, 16, generator=gen)
    v = torch.randn(10, 2, 16, generator=gen)
    got = ref.ragged_attention(q, k, v, lengths)
    start = 0
    for n in lengths:
        qs = q[start : start + n].transpose(0, 1)
        ks = k[start : start + n].repeat_interleave(2, dim=1).transpose(0, 1)
        vs = v[start : start + n].repeat_interleave(2, dim=1).transpose(0, 1)
        expected = F.scaled_dot_product_attention(qs, ks, vs, is_causal=True).transpose(0, 1)
        torch.testing.assert_close(got[start : start + n], expected, atol=1e-5, rtol=1e-5)
        start += n


def test_paged_equals_ragged_when_context_is_the_query():
    # A prefill with no cached prefix is the cacheless causal case.
    q, kc, vc, bt, ql, kl = _tiny_case(21, [5, 3], [5, 3], 4, 2)
    k = torch.cat([torch.cat([kc[int(p)] for p in bt[s][: (n + 3) // 4]])[:n] for s, n in enumerate(kl)])
    v = torch.cat([torch.cat([vc[int(p)] for p in bt[s][: (n + 3) // 4]])[:n] for s, n in enumerate(kl)])
    torch.testing.assert_close(ref.paged_attention(q, kc, vc, bt, ql, kl), ref.ragged_attention(q, k, v, kl),
                               atol=1e-6, rtol=1e-6)


@pytest.mark.parametrize("cuts", [[0, 37, 64], [0, 1, 2, 64], [0, 16, 32, 48, 64]])
def test_split_k_lse_merge_equals_unsplit(cuts):
    gen = torch.Generator().manual_seed(17)
    qv = torch.randn(32, generator=gen)
    keys = torch.randn(64, 32, generator=gen) * 2
    values = torch.randn(64, 32, generator=gen)
    scale = 32 ** -0.5
    full, full_lse = ref.attention_partial(qv, keys, values, scale)
    parts = [ref.attention_partial(qv, keys[a:b], values[a:b], scale) for a, b in zip(cuts, cuts[1:])]
    merged = ref.lse_merge([o for o, _ in parts], [l for _, l in parts])
    torch.testing.assert_close(merged, full, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(torch.logsumexp(torch.stack([l for _, l in parts]), 0), full_lse)


# ---------------------------------------------------------------------------
# RMSNorm oracle (nanovllm/layers/layernorm.py:31-52)
# ---------------------------------------------------------------------------

def _ulp(a, b):
    from tests._util import max_ulp_diff

    return max_ulp_diff(a, b)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rms_norm_oracle_matches_torch_library_rms_norm(dtype):
    from oracle.reference import rms_norm

    g = torch.Generator().manual_seed(5)
    x = torch.randn(64, 1024, generator=g).to(dtype)
    ones = torch.ones(1024, dtype=dtype)
    lib = F.rms_norm(x.float(), (1024,), ones.float(), 1e-6).to(dtype)
    assert _ulp(rms_norm(x, ones, 1e-6), lib) <= 1
    w = (1 + 0.1 * torch.randn(1024, generator=g)).to(dtype)
    lib = F.rms_norm(x.float(), (1024,), w.float(), 1e-6).to(dtype)
    assert _ulp(rms_norm(x, w, 1e-6), lib) <= 2  # the oracle rounds twice, the library once


def test_rms_norm_constant_rows_give_the_weight():
    from oracle.reference import rms_norm

    w = torch.randn(256, generator=torch.Generator().manual_seed(6)).bfloat16()
    for c in (0.25, 1.0, -3.0, 100.0):
        x = torch.full((3, 256), c).bfloat16()
        expected = (w if c > 0 else -w).expand(3, -1)
        assert torch.equal(rms_norm(x, w, 1e-6), expected)


def test_fused_add_rms_norm_uses_fp32_sum_statistics():
    from oracle.reference import fused_add_rms_norm, rms_norm

    # x + residual = [257, 129] in fp32; bf16 rounds 257 to 256.  Normalising
    # the fp32 sum (the reference) and normalising the rounded residual (a
    # plausible mistake) differ in the second element.
    x = torch.tensor([[256.0, 129.0]]).bfloat16()
    residual = torch.tensor([[1.0, 0.0]]).bfloat16()
    w = torch.ones(2).bfloat16()
    out, res = fused_add_rms_norm(x, residual, w, 0.0)
    assert res.tolist() == [[256.0, 129.0]]
    s = [257.0, 129.0]
    inv = 1.0 / ((s[0] ** 2 + s[1] ** 2) / 2) ** 0.5
    assert out.tolist() == torch.tensor([[s[0] * inv, s[1] * inv]]).bfloat16().tolist()
    planted = rms_norm(res, w, 0.0)
    assert not torch.equal(out, planted)


def test_rms_scaled_is_the_unit_weight_rms_norm():
    from oracle.reference import rms_norm, rms_scaled

    x = torch.randn(8, 96, generator=torch.Generator().manual_seed(7)).bfloat16()
    assert torch.equal(rms_scaled(x.float(), 1e-6, torch.bfloat16), rms_norm(x, torch.ones(96).bfloat16(), 1e-6))


# ---------------------------------------------------------------------------
# Rotary embedding oracle (nanovllm/layers/rotary_embedding.py)
# ---------------------------------------------------------------------------

def test_rope_position_zero_is_identity():
    from oracle.reference import rope, rope_cos_sin_cache

    x = torch.randn(3, 4, 128, generator=torch.Generator().manual_seed(8)).bfloat16()
    table = rope_cos_sin_cache(128, 64, 1e6)
    assert torch.equal(rope(x, torch.zeros(3, dtype=torch.long), table), x)


def test_rope_is_complex_rotation_of_neox_pairs():
    from oracle.reference import rope, rope_cos_sin_cache

    g = torch.Generator().manual_seed(9)
    x = torch.randn(5, 2, 128, generator=g).bfloat16()
    pos = torch.tensor([0, 1, 17, 1000, 4095])
    table = rope_cos_sin_cache(128, 4096, 1e6)
    got = rope(x, pos, table).double()
    theta = 1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float64) / 128))
    z = torch.complex(x[..., :64].double(), x[..., 64:].double()) * torch.exp(1j * pos[:, None, None].double() * theta)
    ref = torch.cat((z.real, z.imag), dim=-1)
    assert (got - ref).abs().max().item() < 2 ** -6  # bf16 rounding of values up to ~4
    # Each (j, j + 64) pair keeps its length.
    pair = lambda t: t[..., :64] ** 2 + t[..., 64:] ** 2  # noqa: E731
    torch.testing.assert_close(pair(got), pair(x.double()), atol=0.05, rtol=0.02)
    # A planted interleaved (GPT-J) pairing is caught.
    xi = x.float().reshape(5, 2, 64, 2)
    cos, sin = table[pos].chunk(2, dim=-1)
    planted = torch.stack((xi[..., 0] * cos - xi[..., 1] * sin, xi[..., 1] * cos + xi[..., 0] * sin), -1)
    assert (planted.reshape(5, 2, 128).double() - ref).abs().max().item() > 0.1
