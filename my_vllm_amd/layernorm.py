"""RMSNorm / fused residual-add RMSNorm CustomOp with a gfx950 provider.

Mirrors nanovllm/layers/layernorm.py:7-154: two operators, ``rms_norm`` and
``fused_add_rms_norm``, each bound to a provider once at construction from
``CustomOpConfig`` overrides, plus ``forward_inplace`` for callers whose
inputs are dead after the call.  Providers:

* ``hip`` (alias ``flashinfer``, the reference's name for its accelerated
  provider, so existing override maps keep working): the gfx950 kernels via
  the C ABI (``mva_rms_norm``, ``mva_fused_add_rms_norm``);
* ``native`` / ``native_torch``: the reference's torch formulation;
* ``auto``: ``hip`` on a GPU platform, ``native_torch`` otherwise.

On a GPU platform ``auto`` never falls back to torch: when the native library
is missing, construction raises.
"""

from __future__ import annotations

import torch
from torch import nn

from . import _native, ops
from .custom_op import CustomOp, CustomOpConfig


class RMSNorm(CustomOp):
    """RMSNorm and fused residual-add RMSNorm ordinary operator."""

    op_name = "rms_norm"
    _SUPPORTED = frozenset({"auto", "native", "native_torch", "hip", "flashinfer"})

    def __init__(self, hidden_size: int, eps: float = 1e-6, custom_op_config: CustomOpConfig | None = None) -> None:
        super().__init__(custom_op_config)
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.rms_provider_name, self.rms_impl, _ = self._select_impl("rms_norm")
        (
            self.add_rms_provider_name,
            self.add_rms_impl,
            self.add_rms_inplace_impl,
        ) = self._select_impl("fused_add_rms_norm")

    def _native_rms(self, x: torch.Tensor) -> torch.Tensor:
        orig_dtype = x.dtype
        x = x.float()
        var = x.pow(2).mean(dim=-1, keepdim=True)
        x.mul_(torch.rsqrt(var + self.eps))
        return x.to(orig_dtype).mul_(self.weight)

    def _native_add_rms(self, x: torch.Tensor, residual: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        orig_dtype = x.dtype
        x = x.float().add_(residual.float())
        residual = x.to(orig_dtype)
        var = x.pow(2).mean(dim=-1, keepdim=True)
        x.mul_(torch.rsqrt(var + self.eps))
        return x.to(orig_dtype).mul_(self.weight), residual

    def forward_native(self, x: torch.Tensor, residual: torch.Tensor | None = None):
        if residual is None:
            return self._native_rms(x)
        return self._native_add_rms(x, residual)

    def forward_cuda(self, x: torch.Tensor, residual: torch.Tensor | None = None):
        if residual is None:
            return self.rms_impl(x)
        return self.add_rms_impl(x, residual)

    def forward_inplace(self, x: torch.Tensor, residual: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Use the selected fast path when both incoming tensor values are dead."""
        return self.add_rms_inplace_impl(x, residual)

    def _select_impl(self, operator: str):
        implementation = self.custom_op_config.implementation_for(operator)
        if implementation not in self._SUPPORTED:
            available = ", ".join(sorted(self._SUPPORTED))
            raise ValueError(f"unsupported {operator!r} implementation {implementation!r}; available: {available}")
        if self.platform != "cuda" and implementation not in ("auto", "native", "native_torch"):
            raise RuntimeError(f"{implementation!r} for {operator!r} requires CUDA")
        native = self._native_rms if operator == "rms_norm" else self._native_add_rms
        if implementation in ("native", "native_torch") or self.platform != "cuda":
            return "native_torch", native, native
        dtype = self.custom_op_config.dtype
        if dtype not in (torch.float16, torch.bfloat16, None):
            if implementation == "auto":
                return "native_torch", native, native
            raise RuntimeError(f"'hip' for {operator!r} does not support dtype {dtype}")
        _native.load_library()  # raises if the gfx950 library is missing
        if operator == "rms_norm":
            def forward(x: torch.Tensor) -> torch.Tensor:
                return ops.rms_norm(x, self.weight, self.eps)

            return "hip", forward, forward

        def forward_add(x: torch.Tensor, residual: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
            return ops.fused_add_rms_norm(x, residual, self.weight, self.eps)

        def forward_add_inplace(x: torch.Tensor, residual: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
            return ops.fused_add_rms_norm(x, residual, self.weight, self.eps, inplace=True)

        return "hip", forward_add, forward_add_inplace
