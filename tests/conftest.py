import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built native library")


def pytest_sessionstart(session):
    """Build the C-ABI library when a checkout has none yet (it is not committed)."""
    from my_vllm_amd import _native

    if not _native.LIB_PATH.exists():
        from my_vllm_amd import build

        build.build()


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; fails (does not skip) when the GPU or the native library is missing."""
    import torch

    from my_vllm_amd import _native

    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    _native.load_library()
    arch = torch.cuda.get_device_properties(0).gcnArchName
    assert arch.startswith("gfx950"), f"expected gfx950, found {arch}"
    return torch.device("cuda", 0)
