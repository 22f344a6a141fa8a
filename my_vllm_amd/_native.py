"""ctypes binding of ``lib/libmy_vllm_amd.so`` (C ABI in ``include/my_vllm_amd.h``).

The library is loaded lazily, after ``torch`` (whose bundled HIP runtime the
library then binds to: both carry the soname ``libamdhip64.so.7``).  There is no
fallback: when the library is missing every call raises ``RuntimeError`` naming
the build command, so a GPU run can never silently use another implementation.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libmy_vllm_amd.so"

DTYPE_CODES = {torch.bfloat16: 0, torch.float16: 1}
# Weight element codes of the RMSNorm entry points (MVA_DTYPE_F32 = 2).
WEIGHT_DTYPE_CODES = {**DTYPE_CODES, torch.float32: 2}

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float

# name -> (restype, argtypes); mirrors include/my_vllm_amd.h.
_SIGNATURES = {
    "mva_last_error": (ctypes.c_char_p, []),
    "mva_abi_version": (_i32, []),
    "mva_silu_and_mul": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _i32, _c_void_p]),
    "mva_kv_store": (
        _i32,
        [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _c_void_p, _i64, _c_void_p, _i32, _i64, _i64, _i32, _c_void_p],
    ),
    "mva_rms_norm": (
        _i32,
        [_c_void_p, _i64, _i64, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _i32, _c_void_p],
    ),
    "mva_fused_add_rms_norm": (
        _i32,
        [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _c_void_p, _i64, _c_void_p, _i64, _i64, _i64, _f32, _i32, _i32,
         _c_void_p],
    ),
    "mva_qk_norm_rope_store": (
        _i32,
        [
            _c_void_p, _c_void_p, _i64, _i64, _i32,  # q_in, q_out, q strides, num_q_heads
            _c_void_p, _c_void_p, _i64, _i64,  # k_in, k_out, k strides
            _c_void_p, _i64, _i64, _i32,  # v, v strides, num_kv_heads
            _c_void_p, _c_void_p, _i64, _i32,  # positions, cos_sin_cache, max_position, rotary_dim
            _c_void_p, _c_void_p, _i32, _f32,  # q/k norm weights, weight dtype, eps
            _c_void_p, _c_void_p, _i64, _c_void_p, _i32,  # k_cache, v_cache, num_slots, slot_mapping, int64 slots
            _i64, _i32, _i32, _c_void_p,  # num_tokens, head_dim, dtype, stream
        ],
    ),
    "mva_decode_workspace_bytes": (_i64, [_i64, _i32, _i32]),
    "mva_paged_decode": (
        _i32,
        [
            _c_void_p, _i64, _i64,  # q, q_token_stride, q_head_stride
            _c_void_p, _c_void_p, _i64, _i64, _i64,  # k_cache, v_cache, num_pages, page_stride, token_stride
            _c_void_p, _i64, _c_void_p,  # block_tables, block_table_stride, seq_lens
            _c_void_p, _i64, _i64,  # items, num_items, num_waves
            _c_void_p, _i32,  # wave_extra, waves_per_group
            _c_void_p, _i64, _i64,  # merges, num_merges, num_part_slots
            _c_void_p, _i64, _i64,  # out, out_token_stride, out_head_stride
            _c_void_p, _i64,  # workspace, workspace_bytes
            _i32, _i32, _i32, _i32, _f32, _i32, _c_void_p,  # heads, head_dim, page, scale, dtype, stream
        ],
    ),
    "mva_paged_decode_store": (
        _i32,
        [
            _c_void_p, _i64, _i64,  # q, q_token_stride, q_head_stride
            _c_void_p, _c_void_p, _i64, _i64, _i64,  # k_cache, v_cache, num_pages, page_stride, token_stride
            _c_void_p, _i64, _c_void_p,  # block_tables, block_table_stride, seq_lens
            _c_void_p, _i64, _i64,  # items, num_items, num_waves
            _c_void_p, _i32,  # wave_extra, waves_per_group
            _c_void_p, _i64, _i64,  # merges, num_merges, num_part_slots
            _c_void_p, _i64, _i64,  # out, out_token_stride, out_head_stride
            _c_void_p, _i64,  # workspace, workspace_bytes
            _c_void_p, _i64, _i64,  # k_new, k_token_stride, k_head_stride
            _c_void_p, _i64, _i64,  # v_new, v_token_stride, v_head_stride
            _c_void_p, _i32, _i64,  # slot_mapping, slot_is_int64, num_new_tokens
            _i32, _i32, _i32, _i32, _f32, _i32, _c_void_p,  # heads, head_dim, page, scale, dtype, stream
        ],
    ),
    "mva_paged_decode_graph": (
        _i32,
        [
            _c_void_p, _i64, _i64,  # q, q_token_stride, q_head_stride
            _c_void_p, _c_void_p, _i64, _i64, _i64,  # k_cache, v_cache, num_pages, page_stride, token_stride
            _c_void_p, _i64, _c_void_p,  # block_tables, block_table_stride, seq_lens
            _c_void_p,  # counts
            _c_void_p, _i64, _c_void_p, _i64, _i32,  # items, item_capacity, wave_extra, wave_capacity, waves_per_group
            _c_void_p, _i64, _i64,  # merges, merge_capacity, num_part_slots
            _c_void_p, _i64, _i64,  # out, out_token_stride, out_head_stride
            _c_void_p, _i64,  # workspace, workspace_bytes
            _i32, _i32, _i32, _i32, _f32, _i32, _c_void_p,
        ],
    ),
    "mva_paged_decode_noalloc": (
        _i32,
        [
            _c_void_p, _i64, _i64,  # q, q_token_stride, q_head_stride
            _c_void_p, _c_void_p, _i64, _i64, _i64,  # k_cache, v_cache, num_pages, page_stride, token_stride
            _c_void_p, _i64, _c_void_p,  # block_tables, block_table_stride, seq_lens
            _c_void_p, _i64, _i64,  # items, num_items, num_waves
            _c_void_p, _i32,  # wave_extra, waves_per_group
            _c_void_p, _i64, _i64,  # merges, num_merges, num_part_slots
            _c_void_p, _i64, _i64,  # out, out_token_stride, out_head_stride
            _i32, _i32, _i32, _i32, _f32, _i32, _c_void_p,  # heads, head_dim, page, scale, dtype, stream
        ],
    ),
    "mva_decode_plan_listed_rows": (_i64, [_i64, _i64, _i32, _i32, _i32]),
    "mva_decode_plan_listed": (
        _i32,
        [
            _c_void_p, _i64, _i64, _i64,  # block_counts, num_seqs, first_seq, first_q_row
            _i32, _i32, _i32,  # num_kv_heads, num_groups, max_piece_pages
            _c_void_p, _i64, _c_void_p, _i64,  # items, item_rows, wave_extra, wave_extra_len
            _c_void_p, _i64, _c_void_p,  # merges, merge_rows, out_counts
        ],
    ),
    "mva_decode_plan_claims_rows": (_i64, [_i64, _i64, _i32, _i32]),
    "mva_decode_plan_claims": (
        _i32,
        [
            _c_void_p, _i64, _i64, _i64,  # block_counts, num_seqs, first_seq, first_q_row
            _i32, _i64, ctypes.c_double, _i32, _i32,  # num_kv_heads, num_waves, pieces/wave, piece bounds
            _c_void_p, _i64, _c_void_p, _i64, _c_void_p,  # items, item_rows, merges, merge_rows, out_counts
        ],
    ),
    "mva_prefill_tile_tokens": (_i32, [_i32, _i32]),
    "mva_prefill_workspace_bytes": (_i64, [_i64]),
    "mva_paged_prefill": (
        _i32,
        [
            _c_void_p, _i64, _i64,  # q, q_token_stride, q_head_stride
            _c_void_p, _c_void_p, _i64, _i64, _i64,  # k_cache, v_cache, num_pages, page_stride, token_stride
            _c_void_p, _i64, _c_void_p, _c_void_p,  # block_tables, stride, seq_lens, query_start_loc
            _i64, _i64, _c_void_p, _i64,  # num_seqs, max_tiles, workspace, workspace_bytes
            _c_void_p, _i64, _i64,  # out, out_token_stride, out_head_stride
            _i32, _i32, _i32, _i32, _f32, _i32, _c_void_p,
        ],
    ),
    "mva_paged_prefill_plan": (
        _i32,
        [
            _c_void_p, _i64, _i64,  # block_tables, stride, num_pages
            _c_void_p, _c_void_p, _i64, _i64,  # seq_lens, query_start_loc, num_seqs, max_tiles
            _c_void_p, _i64, _i32, _i32, _c_void_p,  # workspace, workspace_bytes, heads, stream
        ],
    ),
    "mva_paged_prefill_run": (
        _i32,
        [
            _c_void_p, _i64, _i64,
            _c_void_p, _c_void_p, _i64, _i64, _i64,
            _c_void_p, _i64, _c_void_p, _c_void_p,
            _i64, _i64, _c_void_p, _i64,
            _c_void_p, _i64, _i64,
            _i32, _i32, _i32, _i32, _f32, _i32, _c_void_p,
        ],
    ),
    "mva_paged_mixed": (
        _i32,
        [
            _c_void_p, _i64, _i64,
            _c_void_p, _c_void_p, _i64, _i64, _i64,
            _c_void_p, _i64, _c_void_p, _c_void_p,
            _i64, _i64, _c_void_p, _i64, _i64,  # prefill seqs, max prefill tiles, decode items, waves
            _i64,  # num_part_slots
            _c_void_p, _i64, _i64,
            _c_void_p, _i64,
            _i32, _i32, _i32, _i32, _f32, _i32, _c_void_p,
        ],
    ),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)
# The C ABI revision these signatures describe (mva_abi_version()).
ABI_VERSION = 11

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_load_error: Exception | None = None


def load_library() -> ctypes.CDLL:
    """Load and type the shared library (once); raise RuntimeError if absent."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            _load_error = FileNotFoundError(str(LIB_PATH))
            raise RuntimeError(
                f"my_vllm_amd native library is missing ({LIB_PATH}); "
                "build it with `python -m my_vllm_amd.build`"
            )
        try:
            lib = ctypes.CDLL(str(LIB_PATH))
        except OSError as error:
            _load_error = error
            raise RuntimeError(f"cannot load {LIB_PATH}: {error}") from error
        rebuild = "rebuild it with `python -m my_vllm_amd.build`"
        # The revision first: a stale library may lack entry points added
        # since, and that must read as "rebuild", not as a missing attribute.
        try:
            version_fn = lib.mva_abi_version
        except AttributeError:
            _load_error = RuntimeError("no mva_abi_version")
            raise RuntimeError(f"{LIB_PATH} exports no mva_abi_version; {rebuild}") from None
        version_fn.restype, version_fn.argtypes = ctypes.c_int, []
        revision = version_fn()
        if revision != ABI_VERSION:
            _load_error = RuntimeError(f"ABI revision {revision}")
            raise RuntimeError(
                f"{LIB_PATH} has C ABI revision {revision}, this package expects {ABI_VERSION}; {rebuild}"
            )
        missing = [name for name in _SIGNATURES if not hasattr(lib, name)]
        if missing:
            _load_error = RuntimeError(f"missing exports {missing}")
            raise RuntimeError(f"{LIB_PATH} lacks the entry points {', '.join(missing)}; {rebuild}")
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


def native_available() -> bool:
    try:
        load_library()
    except RuntimeError:
        return False
    return True


def call(name: str, *args) -> None:
    """Call a status-returning entry point; map a nonzero status to RuntimeError."""
    lib = load_library()
    status = getattr(lib, name)(*args)
    if status != 0:
        message = lib.mva_last_error().decode("utf-8", "replace")
        raise RuntimeError(f"{name} failed ({status}): {message}")


def query(name: str, *args):
    """Call an entry point that returns a value rather than a status."""
    return getattr(load_library(), name)(*args)


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device`."""
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise RuntimeError(f"unsupported dtype {dtype}; expected bfloat16 or float16") from None
