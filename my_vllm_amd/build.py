"""Build the gfx950 C-ABI library ``my_vllm_amd/lib/libmy_vllm_amd.so``.

Every ``csrc/*.hip`` translation unit is compiled with ``hipcc`` for gfx950
only and linked into one shared library that exports the ``extern "C"`` entry
points declared in ``include/my_vllm_amd.h``.  The library is built in-tree so
that it travels with the source tree; no JIT cache is involved.

Run ``python -m my_vllm_amd.build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC_DIR = PACKAGE_DIR / "csrc"
LIB_DIR = PACKAGE_DIR / "lib"
LIB_PATH = LIB_DIR / "libmy_vllm_amd.so"
BUILD_DIR = PACKAGE_DIR / "_build"

OFFLOAD_ARCH = "gfx950"
# Packed fp32 VALU forms are disabled for every kernel of this library.  The
# atomic optimizer is off: it turns a single-lane atomic into a wave-wide
# reduction whose result is broadcast right after the atomic, which makes the
# decode kernel's piece claims wait for every load in flight.
HIP_FLAGS = (
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-mllvm",
    "-amdgpu-atomic-optimizer-strategy=None",
)


def _hipcc() -> str:
    candidates = (
        os.environ.get("HIPCC"),
        "/opt/rocm/bin/hipcc",
        shutil.which("hipcc"),
    )
    for candidate in candidates:
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found; the gfx950 library cannot be built")


def _compile(hipcc: str, source: Path, obj: Path) -> None:
    cmd = [hipcc, *HIP_FLAGS, f"-I{CSRC_DIR}", "-c", str(source), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(
            f"hipcc failed for {source.name}:\n{proc.stdout}\n{proc.stderr}"
        )


def build(verbose: bool = False) -> Path:
    """Compile all kernels for gfx950 and link the shared library; return its path."""
    hipcc = _hipcc()
    sources = sorted(CSRC_DIR.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC_DIR}")
    BUILD_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    objects = [BUILD_DIR / (src.stem + ".o") for src in sources]
    jobs = max(1, min(len(sources), int(os.environ.get("MAX_JOBS", "8"))))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        list(pool.map(lambda pair: _compile(hipcc, *pair), zip(sources, objects)))
    fd, tmp = tempfile.mkstemp(prefix=".libmy_vllm_amd.", suffix=".so.tmp", dir=LIB_DIR)
    os.close(fd)
    cmd = [hipcc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", "-o", tmp, *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        os.unlink(tmp)
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
