"""CPU: the C-ABI library loads and exports every entry point include/*.h declares.

Only host-side entry points are called here (queries and argument
validation that fails before any launch); nothing touches a GPU.
"""

import ctypes
import re
from pathlib import Path

import pytest
import torch

from my_vllm_amd import _native

ROOT = Path(__file__).resolve().parents[1]


def _declared_functions() -> list[str]:
    names = []
    for header in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names += re.findall(r"\b(mva_\w+)\s*\(", text)
    return names


def test_header_declares_the_bound_signatures():
    declared = _declared_functions()
    assert declared, "no entry points found in include/*.h"
    assert len(set(declared)) == len(declared)
    assert set(declared) == set(_native.EXPORTED_SYMBOLS)


def test_library_loads_and_exports_every_declared_symbol():
    lib = _native.load_library()
    for name in _declared_functions():
        assert hasattr(lib, name), f"{name} missing from {_native.LIB_PATH.name}"
    assert lib.mva_abi_version() == _native.ABI_VERSION


def test_library_binds_to_the_process_hip_runtime():
    # torch is imported first; the library must reuse its libamdhip64 rather
    # than load a second HIP runtime.
    _native.load_library()
    maps = Path("/proc/self/maps").read_text().splitlines()
    runtimes = {line.split()[-1] for line in maps if "libamdhip64" in line}
    assert len(runtimes) <= 1, runtimes


def test_host_queries():
    assert _native.query("mva_prefill_tile_tokens", 16, 8) == 64
    assert _native.query("mva_prefill_tile_tokens", 32, 8) == 32
    assert _native.query("mva_prefill_tile_tokens", 64, 8) == 16
    assert _native.query("mva_prefill_tile_tokens", 12, 5) == -1
    small = _native.query("mva_decode_workspace_bytes", 0, 8, 2)
    big = _native.query("mva_decode_workspace_bytes", 100, 8, 2)
    assert small > 0 and big > small and big % 256 == 0
    assert _native.query("mva_decode_workspace_bytes", -1, 8, 2) == -1


def test_invalid_arguments_fail_before_launch_with_a_message():
    lib = _native.load_library()
    with pytest.raises(RuntimeError, match="mva_silu_and_mul failed"):
        _native.call("mva_silu_and_mul", 0, 0, 4, 8, 7, 0)  # dtype code 7 is invalid
    assert lib.mva_last_error().decode()
    # head_dim 64 is rejected by the decode entry point before anything runs.
    with pytest.raises(RuntimeError, match="mva_paged_decode failed"):
        _native.call("mva_paged_decode", 0, 0, 0, 0, 0, 1, 0, 0, 0, 0, 0, 0, 1, 1, 0, 1, 0, 0, 0, 0, 0, 0, 0, 0,
                     16, 8, 64, 16, 1.0, 0, 0)
    # A MIXED launch orders at most 1024 prefill sequences in LDS.
    with pytest.raises(RuntimeError, match="at most 1024 prefill sequences"):
        _native.call("mva_paged_mixed", 0, 0, 0, 0, 0, 1, 0, 0, 0, 0, 0, 0, 1025, 2000, 0, 0, 0, 0,
                     0, 0, 0, 0, 0, 16, 8, 128, 16, 1.0, 0, 0)
    # The prefill plan and run entry points check heads and the workspace
    # before they touch the device; an empty batch is a no-op.
    with pytest.raises(RuntimeError, match="positive multiple of num_kv_heads"):
        _native.call("mva_paged_prefill_plan", 0, 0, 1, 0, 0, 1, 1, 0, 0, 12, 8, 0)
    with pytest.raises(RuntimeError, match="prefill workspace too small"):
        _native.call("mva_paged_prefill_plan", 0, 0, 1, 0, 0, 1, 1, 0, 0, 32, 8, 0)
    _native.call("mva_paged_prefill_plan", 0, 0, 1, 0, 0, 0, 1, 0, 0, 32, 8, 0)
    with pytest.raises(RuntimeError, match="prefill workspace too small"):
        _native.call("mva_paged_prefill_run", 0, 0, 0, 0, 0, 1, 0, 0, 0, 0, 0, 0, 1, 1, 0, 0, 0, 0, 0,
                     32, 8, 128, 16, 1.0, 0, 0)


def test_dtype_codes_match_the_header():
    header = (ROOT / "include" / "my_vllm_amd.h").read_text()
    assert f"#define MVA_DTYPE_BF16 {_native.DTYPE_CODES[torch.bfloat16]}" in header
    assert f"#define MVA_DTYPE_F16 {_native.DTYPE_CODES[torch.float16]}" in header


def test_store_error_offset_matches_the_header_and_the_workspace_layout():
    from my_vllm_amd import ops

    header = (ROOT / "include" / "my_vllm_amd.h").read_text()
    assert f"#define MVA_DECODE_STORE_ERROR_OFFSET {ops.DECODE_STORE_ERROR_OFFSET}" in header
    # The word sits inside the scheduler area every decode workspace has.
    assert ops.DECODE_STORE_ERROR_OFFSET + 4 <= _native.query("mva_decode_workspace_bytes", 0, 8, 1)
    assert f"#define MVA_PREFILL_DROPPED_TILES_OFFSET {ops.PREFILL_DROPPED_TILES_OFFSET}" in header
    assert ops.PREFILL_DROPPED_TILES_OFFSET + 4 <= _native.query("mva_prefill_workspace_bytes", 0)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setattr(_native, "LIB_PATH", tmp_path / "absent.so")
    with pytest.raises(RuntimeError, match="missing"):
        _native.load_library()
    assert _native.native_available() is False


def test_abi_revision_mismatch_raises(monkeypatch):
    # A library built from other sources than this package's signatures
    # describe must not load.
    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setattr(_native, "_load_error", _native._load_error)
    monkeypatch.setattr(_native, "ABI_VERSION", _native.ABI_VERSION + 1)
    with pytest.raises(RuntimeError, match="ABI revision"):
        _native.load_library()


def test_stale_library_without_a_new_entry_point_asks_for_a_rebuild(monkeypatch):
    # A library built before an entry point was added must fail with the
    # same "rebuild" RuntimeError (not an AttributeError), and
    # native_available() must report False rather than raise.
    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setattr(_native, "_load_error", _native._load_error)
    signatures = dict(_native._SIGNATURES)
    signatures["mva_entry_point_from_the_future"] = (ctypes.c_int, [])
    monkeypatch.setattr(_native, "_SIGNATURES", signatures)
    with pytest.raises(RuntimeError, match="rebuild"):
        _native.load_library()
    assert _native.native_available() is False
