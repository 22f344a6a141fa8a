"""Which of the reference's operator providers this package serves, and how a
requested provider name resolves.

The reference's ordinary operators pick a provider once, at construction,
from ``CustomOpConfig.overrides[op_name]`` (nanovllm/layers/activation.py:11-20,
attention.py:55-64, layernorm.py:82-154, rotary_embedding.py:58-110).  On
MI355X every accelerated choice runs the same gfx950 kernel of this package,
so the table below lists, per operator, every name that selects it: ``hip``
(this package's own name) and the reference's names for its GPU providers,
so that override maps written for the reference
(``example_optimized.py:10-16``) keep working unchanged.  ``auto`` selects
the kernel on a GPU platform.

The reference's torch implementations (``native`` / ``native_torch``) are not
shipped here: they belong to the reference's own operator classes, and the
tests restate them as the oracle.  Requesting them from this package's
operators raises a RuntimeError, as does any request off a GPU platform;
there is no silent CPU fallback.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _native
from .custom_op import NATIVE_IMPLEMENTATIONS, CustomOp

HIP = "hip"
KERNEL_DTYPES = (torch.float16, torch.bfloat16)


@dataclass(frozen=True)
class KernelProvider:
    """The gfx950 kernel behind one of the reference's operator names."""

    op_name: str
    entry_points: tuple[str, ...]  # C-ABI functions the operator calls
    aliases: frozenset[str]  # the reference's provider names this kernel stands in for

    @property
    def names(self) -> frozenset[str]:
        """Every accepted value of ``overrides[op_name]``."""
        return frozenset({"auto", HIP}) | self.aliases | NATIVE_IMPLEMENTATIONS


_TABLE = {
    spec.op_name: spec
    for spec in (
        KernelProvider("silu_and_mul", ("mva_silu_and_mul",),
                       frozenset({"custom_cuda", "adaptive_cuda", "flashinfer"})),
        KernelProvider("kv_cache_store", ("mva_kv_store",), frozenset({"native_triton"})),
        KernelProvider("rms_norm", ("mva_rms_norm",), frozenset({"flashinfer"})),
        KernelProvider("fused_add_rms_norm", ("mva_fused_add_rms_norm",), frozenset({"flashinfer"})),
        KernelProvider("rotary_embedding", ("mva_qk_norm_rope_store",), frozenset({"flashinfer"})),
    )
}


def provider(op_name: str) -> KernelProvider:
    return _TABLE[op_name]


def operator_names() -> tuple[str, ...]:
    return tuple(_TABLE)


def resolve(op: CustomOp, op_name: str | None = None) -> str:
    """Check the provider requested for ``op_name`` (default ``op.op_name``)
    and load the kernel library; returns the bound provider name, "hip".

    ValueError for a name the operator does not know (the reference's
    message); RuntimeError for a request this package cannot serve on this
    platform or dtype, or when the gfx950 library is missing.
    """
    name = op_name or op.op_name
    spec = _TABLE[name]
    config = op.custom_op_config
    choice = config.implementation_for(name)
    if choice not in spec.names:
        raise ValueError(
            f"unsupported {name!r} implementation {choice!r}; available: {', '.join(sorted(spec.names))}"
        )
    if choice in NATIVE_IMPLEMENTATIONS:
        raise RuntimeError(
            f"{choice!r} for {name!r} is the reference's torch implementation; my_vllm_amd provides the "
            f"gfx950 kernel only ('auto', 'hip' or {', '.join(repr(a) for a in sorted(spec.aliases))})"
        )
    if op.platform != "cuda":
        raise RuntimeError(f"{choice!r} for {name!r} requires CUDA")
    if config.dtype is not None and config.dtype not in KERNEL_DTYPES:
        raise RuntimeError(f"{choice!r} for {name!r} does not support dtype {config.dtype}")
    lib = _native.load_library()  # RuntimeError when the gfx950 library is missing
    for entry in spec.entry_points:
        getattr(lib, entry)
    return HIP
