"""Comparison helpers shared by the tests."""

from __future__ import annotations

import torch

# Attention tolerance: within 2e-2 absolute / 1e-2 relative of an
# fp32-accumulated reference (bf16/fp16 outputs).
ATTN_ATOL = 2e-2
ATTN_RTOL = 1e-2


def ordered_bits(t: torch.Tensor) -> torch.Tensor:
    """Map bf16/fp16 values to integers whose difference counts ulps."""
    bits = t.contiguous().view(torch.int16).to(torch.int32)
    return torch.where(bits < 0, -(bits & 0x7FFF), bits)


def max_ulp_diff(a: torch.Tensor, b: torch.Tensor) -> int:
    assert a.dtype == b.dtype and a.shape == b.shape
    if a.numel() == 0:
        return 0
    return int((ordered_bits(a.cpu()) - ordered_bits(b.cpu())).abs().max().item())


def assert_attention_close(actual: torch.Tensor, expected_fp32: torch.Tensor) -> None:
    actual = actual.float().cpu()
    expected = expected_fp32.float().cpu()
    assert actual.shape == expected.shape
    assert torch.isfinite(actual).all(), "non-finite attention output"
    torch.testing.assert_close(actual, expected, atol=ATTN_ATOL, rtol=ATTN_RTOL)


def set_decode_planning(monkeypatch, waves=None, schedule=None) -> None:
    """Override the decode wavefront count and schedule of every MI355X
    backend for one test (the backends' planning-override attributes)."""
    from my_vllm_amd.attention_backend import MI355XAttentionBackendMixin

    monkeypatch.setattr(MI355XAttentionBackendMixin, "decode_waves_override",
                        None if waves is None else int(waves))
    monkeypatch.setattr(MI355XAttentionBackendMixin, "decode_schedule_override", schedule)
