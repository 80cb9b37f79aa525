"""ctypes binding of libdsa_amd.so (the C ABI declared in include/dsa_abi.h).

The library must have been built (``python -m dsa_amd.build`` or
``__graft_entry__.build()``).  There is no fallback: if it is missing or does
not export the ABI, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os

# DSA_AMD_LIB names another build of the same ABI (e.g. libdsa_amd_san.so,
# the sanitizer build the CPU ABI tests run against).
LIB_PATH = os.environ.get("DSA_AMD_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                         "libdsa_amd.so")

DSA_OK = 0
DSA_EINVAL = 1
DSA_EUNSUPPORTED = 2
DSA_ELAUNCH = 3
DSA_EWORKSPACE = 4
ABI_VERSION = 5
NOALLOC_SCRATCH_BYTES = 32 << 20   # DSA_NOALLOC_SCRATCH_BYTES

EXPORTED_SYMBOLS = (
    "dsa_attn_fwd",
    "dsa_attn_fwd_noalloc",
    "dsa_attn_fwd_partial",
    "dsa_attn_merge",
    "dsa_attn_num_splits",
    "dsa_attn_partial_bytes",
    "dsa_attn_workspace_bytes",
    "dsa_attn_counter_bytes",
    "dsa_attn_call_counter_bytes",
    "dsa_indexer_topk",
    "dsa_indexer_k_append",
    "dsa_indexer_workspace_bytes",
    "dsa_indexer_workspace_bytes_prepared",
    "dsa_indexer_k_planes_bytes",
    "dsa_indexer_prepare_k",
    "dsa_last_error",
    "dsa_abi_version",
)

_i64 = ctypes.c_int64
_vp = ctypes.c_void_p


class AttnArgs(ctypes.Structure):
    """Mirror of ``dsa_attn_args``."""

    _fields_ = [
        ("q_nope", _vp), ("q_nope_stride_t", _i64), ("q_nope_stride_h", _i64),
        ("q_pe", _vp), ("q_pe_stride_t", _i64), ("q_pe_stride_h", _i64),
        ("ckv", _vp), ("ckv_stride_page", _i64), ("ckv_stride_tok", _i64),
        ("kpe", _vp), ("kpe_stride_page", _i64), ("kpe_stride_tok", _i64),
        ("sparse_indices", _vp), ("idx_stride_t", _i64),
        ("output", _vp), ("out_stride_t", _i64), ("out_stride_h", _i64),
        ("lse", _vp), ("lse_stride_t", _i64), ("lse_stride_h", _i64),
        ("num_tokens", _i64), ("num_heads", _i64), ("topk", _i64),
        ("page_size", _i64), ("num_pages", _i64),
        ("head_dim_ckv", _i64), ("head_dim_kpe", _i64),
        ("sm_scale", ctypes.c_float),
        ("num_splits", ctypes.c_int32),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("split_counters", _vp), ("split_counters_bytes", ctypes.c_size_t),
    ]


class MergeArgs(ctypes.Structure):
    """Mirror of ``dsa_attn_merge_args``."""

    _fields_ = [
        ("part_acc", _vp), ("part_ml", _vp),
        ("num_tokens", _i64), ("num_splits", _i64), ("num_heads", _i64),
        ("output", _vp), ("out_stride_t", _i64), ("out_stride_h", _i64),
        ("lse", _vp), ("lse_stride_t", _i64), ("lse_stride_h", _i64),
    ]


class IndexerArgs(ctypes.Structure):
    """Mirror of ``dsa_indexer_args``."""

    _fields_ = [
        ("q_idx", _vp), ("k_idx", _vp), ("k_scale", _vp), ("weights", _vp),
        ("causal_limit", _vp),
        ("num_tokens", _i64), ("num_heads", _i64), ("head_dim", _i64),
        ("num_positions", _i64), ("topk", _i64),
        ("block_table", _vp), ("block_table_stride", _i64), ("page_size", _i64),
        ("out", _vp), ("scores_out", _vp),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("k_cache", _vp), ("k_pages", _vp), ("k_page_size", _i64),
        ("block_table_width", _i64), ("k_num_pages", _i64),
        ("k_planes", _vp), ("k_planes_capacity", _i64),
    ]


class KPrepareArgs(ctypes.Structure):
    """Mirror of ``dsa_indexer_k_prepare_args``."""

    _fields_ = [
        ("k_idx", _vp), ("k_scale", _vp), ("k_cache", _vp), ("k_pages", _vp),
        ("k_page_size", _i64), ("k_num_pages", _i64), ("num_positions", _i64),
        ("first_position", _i64), ("count", _i64),
        ("k_planes", _vp), ("k_planes_capacity", _i64),
    ]


class KAppendArgs(ctypes.Structure):
    """Mirror of ``dsa_k_append_args``."""

    _fields_ = [
        ("k", _vp), ("k_stride", _i64), ("slots", _vp), ("num_tokens", _i64),
        ("k_cache", _vp), ("num_pages", _i64), ("page_size", _i64),
    ]


class DSAError(RuntimeError):
    """A non-zero status returned through the C ABI."""

    def __init__(self, fn: str, status: int, msg: str):
        super().__init__(f"{fn} failed (status {status}): {msg}")
        self.status = status


_lib = None


def load() -> ctypes.CDLL:
    """Load libdsa_amd.so once.  torch must already be imported so the library
    binds to the HIP runtime torch uses (both carry soname libamdhip64.so.7)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build the HIP library first "
            "(python -m dsa_amd.build, or __graft_entry__.build()).")
    lib = ctypes.CDLL(LIB_PATH)
    for name in EXPORTED_SYMBOLS:
        if not hasattr(lib, name):
            raise RuntimeError(f"{LIB_PATH} does not export {name}")
    lib.dsa_attn_fwd.argtypes = [ctypes.POINTER(AttnArgs), _vp]
    lib.dsa_attn_fwd.restype = ctypes.c_int
    lib.dsa_attn_fwd_noalloc.argtypes = [ctypes.POINTER(AttnArgs), _vp]
    lib.dsa_attn_fwd_noalloc.restype = ctypes.c_int
    lib.dsa_attn_fwd_partial.argtypes = [ctypes.POINTER(AttnArgs), _vp]
    lib.dsa_attn_fwd_partial.restype = ctypes.c_int
    lib.dsa_attn_merge.argtypes = [ctypes.POINTER(MergeArgs), _vp]
    lib.dsa_attn_merge.restype = ctypes.c_int
    lib.dsa_attn_partial_bytes.argtypes = [_i64, _i64, _i64, ctypes.c_int32]
    lib.dsa_attn_partial_bytes.restype = ctypes.c_size_t
    lib.dsa_attn_num_splits.argtypes = [_i64, _i64, _i64, ctypes.c_int32]
    lib.dsa_attn_num_splits.restype = ctypes.c_int32
    lib.dsa_attn_workspace_bytes.argtypes = [_i64, _i64, _i64, ctypes.c_int32]
    lib.dsa_attn_workspace_bytes.restype = ctypes.c_size_t
    lib.dsa_attn_counter_bytes.argtypes = [_i64, _i64]
    lib.dsa_attn_counter_bytes.restype = ctypes.c_size_t
    lib.dsa_attn_call_counter_bytes.argtypes = [_i64, _i64, _i64, ctypes.c_int32]
    lib.dsa_attn_call_counter_bytes.restype = ctypes.c_size_t
    lib.dsa_indexer_topk.argtypes = [ctypes.POINTER(IndexerArgs), _vp]
    lib.dsa_indexer_topk.restype = ctypes.c_int
    lib.dsa_indexer_k_append.argtypes = [ctypes.POINTER(KAppendArgs), _vp]
    lib.dsa_indexer_k_append.restype = ctypes.c_int
    lib.dsa_indexer_workspace_bytes.argtypes = [_i64, _i64, _i64, _i64]
    lib.dsa_indexer_workspace_bytes.restype = ctypes.c_size_t
    lib.dsa_indexer_workspace_bytes_prepared.argtypes = [_i64, _i64, _i64, _i64]
    lib.dsa_indexer_workspace_bytes_prepared.restype = ctypes.c_size_t
    lib.dsa_indexer_k_planes_bytes.argtypes = [_i64]
    lib.dsa_indexer_k_planes_bytes.restype = ctypes.c_size_t
    lib.dsa_indexer_prepare_k.argtypes = [ctypes.POINTER(KPrepareArgs), _vp]
    lib.dsa_indexer_prepare_k.restype = ctypes.c_int
    lib.dsa_last_error.argtypes = []
    lib.dsa_last_error.restype = ctypes.c_char_p
    lib.dsa_abi_version.argtypes = []
    lib.dsa_abi_version.restype = ctypes.c_int
    if lib.dsa_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH}: ABI version {lib.dsa_abi_version()} != {ABI_VERSION}")
    _lib = lib
    return lib


def check(fn: str, status: int) -> None:
    if status != DSA_OK:
        msg = load().dsa_last_error().decode(errors="replace")
        if status in (DSA_EINVAL, DSA_EUNSUPPORTED, DSA_EWORKSPACE):
            raise ValueError(f"{fn} failed (status {status}): {msg}")
        raise DSAError(fn, status, msg)
