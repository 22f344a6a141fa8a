"""SiLU-and-mul CustomOp with the gfx950 kernel as its MI355X provider.

Mirrors nanovllm/layers/activation.py:7-84: the provider is chosen once at
construction from ``CustomOpConfig`` overrides.  Providers:

* ``hip`` (alias ``custom_cuda``, the reference's name for its in-tree
  compiled kernel): the vectorised gfx950 kernel via the C ABI;
* ``native`` / ``native_torch``: ``x.chunk(2, -1); F.silu(a) * b`` in torch;
* ``auto``: ``hip`` on a GPU platform, ``native_torch`` otherwise.

On a GPU platform ``auto`` never falls back to torch: when the native library
is missing, construction raises.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _native, ops
from .custom_op import CustomOp, CustomOpConfig


class SiluAndMul(CustomOp):
    """SwiGLU activation with construction-time platform dispatch."""

    op_name = "silu_and_mul"
    _CUDA_IMPLEMENTATIONS = frozenset({"auto", "native", "native_torch", "hip", "custom_cuda"})

    def __init__(self, custom_op_config: CustomOpConfig | None = None) -> None:
        super().__init__(custom_op_config)
        implementation = self.require_cuda_implementation(self._CUDA_IMPLEMENTATIONS)
        self.provider_name, self.forward_impl = self._select_cuda_impl(implementation)

    def forward_native(self, x: torch.Tensor) -> torch.Tensor:
        x, y = x.chunk(2, -1)
        return F.silu(x) * y

    def forward_cuda(self, x: torch.Tensor) -> torch.Tensor:
        return self.forward_impl(x)

    def _select_cuda_impl(self, implementation: str):
        if implementation in ("native", "native_torch") or self.platform != "cuda":
            return "native_torch", self.forward_native
        dtype = self.custom_op_config.dtype
        if dtype not in (torch.float16, torch.bfloat16, None):
            if implementation == "auto":
                return "native_torch", self.forward_native
            raise RuntimeError(f"{implementation!r} for 'silu_and_mul' does not support dtype {dtype}")
        _native.load_library()  # raises if the gfx950 library is missing
        return ("custom_cuda" if implementation == "custom_cuda" else "hip"), ops.silu_and_mul
