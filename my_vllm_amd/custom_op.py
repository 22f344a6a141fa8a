"""Construction-time dispatch for ordinary operators.

Interface of the reference's nanovllm/layers/custom_op.py:16-120, which the
model's layers are written against:

* ``CustomOpConfig(platform, dtype, overrides)``: frozen; the platform and
  every override value are lower-cased, the override map is read-only and
  detached from the caller's dict; ``implementation_for(op)`` defaults to
  ``"auto"``; the config is hashable (it keys shared-module caches);
* ``CustomOp``: an ``nn.Module`` whose ``forward`` is bound once, at
  construction, to ``forward_<platform>`` (``dispatch_forward``), falling back
  to ``forward_native``; on ROCm PyTorch the platform is ``"cuda"``.

This package's operators (``layers.py``) implement only ``forward_cuda`` and
take their kernels from the provider table in ``providers.py``.
"""

from __future__ import annotations

from collections.abc import Mapping
from dataclasses import dataclass, field
from types import MappingProxyType
from typing import Any, Callable

import torch
from torch import nn

PLATFORMS = ("auto", "cuda", "cpu", "xpu")
NATIVE_IMPLEMENTATIONS = frozenset({"native", "native_torch"})


def _lowered_copy(overrides: Mapping[str, str]) -> Mapping[str, str]:
    return MappingProxyType({str(op): str(choice).lower() for op, choice in overrides.items()})


@dataclass(frozen=True)
class CustomOpConfig:
    """Which device family an operator binds to, and which provider each
    operator name asks for (``overrides``: op name -> provider name, "auto"
    when absent).  Immutable and hashable once built."""

    platform: str = "auto"
    dtype: torch.dtype | None = None
    overrides: Mapping[str, str] = field(default_factory=dict)

    def __post_init__(self) -> None:
        platform = self.platform.lower()
        if platform not in PLATFORMS:
            raise ValueError("platform must be 'auto', 'cuda', 'cpu', or 'xpu'")
        object.__setattr__(self, "platform", platform)
        object.__setattr__(self, "overrides", _lowered_copy(self.overrides))

    def implementation_for(self, operator: str) -> str:
        return self.overrides.get(operator, "auto")

    def __hash__(self) -> int:
        return hash((self.platform, self.dtype, frozenset(self.overrides.items())))


def default_platform() -> str:
    """The device type new tensors land on, or "cpu" for any other device type."""
    kind = torch.get_default_device().type
    return kind if kind in PLATFORMS[1:] else "cpu"


class CustomOp(nn.Module):
    """An operator module whose ``forward`` is chosen once, when it is built:
    ``forward_<platform>`` if the subclass defines it, else ``forward_native``.
    Subclasses pick their kernel from ``requested_implementation``."""

    op_name = "custom_op"

    def __init__(self, custom_op_config: CustomOpConfig | None = None) -> None:
        super().__init__()
        config = custom_op_config if custom_op_config is not None else CustomOpConfig()
        self.custom_op_config = config
        self.platform = default_platform() if config.platform == "auto" else config.platform
        self._forward_method = self.dispatch_forward()

    @property
    def requested_implementation(self) -> str:
        return self.custom_op_config.implementation_for(self.op_name)

    def dispatch_forward(self) -> Callable[..., Any]:
        return getattr(self, "forward_" + self.platform, self.forward_native)

    def forward(self, *args: Any, **kwargs: Any) -> Any:
        return self._forward_method(*args, **kwargs)

    def forward_native(self, *args: Any, **kwargs: Any) -> Any:
        raise NotImplementedError

    def forward_cuda(self, *args: Any, **kwargs: Any) -> Any:
        return self.forward_native(*args, **kwargs)

    def forward_cpu(self, *args: Any, **kwargs: Any) -> Any:
        return self.forward_native(*args, **kwargs)

    def forward_xpu(self, *args: Any, **kwargs: Any) -> Any:
        return self.forward_native(*args, **kwargs)
