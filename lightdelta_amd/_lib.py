"""ctypes binding of liblightdelta_hip.so (the C ABI declared in include/lightdelta_hip.h).

torch is imported first on purpose: torch ships its own libamdhip64.so.7, and loading it
before the library makes the library's `libamdhip64.so.7` dependency resolve to that same
copy, so torch's streams and allocations are valid in the library (one HIP runtime per
process).  There is no fallback: a missing or unloadable library raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  -- must precede the CDLL load (see module docstring)

LIBRARY_PATH = Path(__file__).resolve().with_name("liblightdelta_hip.so")
ABI_VERSION = 12
DTYPE_F32 = 0
DTYPE_BF16 = 1
CACHE_KEEP = 0
CACHE_STREAM = 1
HEAD_DIM = 128
MAX_TOKENS = 4

_c_i32 = ctypes.c_int32
_c_i64 = ctypes.c_int64
_vp = ctypes.c_void_p


class DecodeArgs(ctypes.Structure):
    """Mirror of ld_gdn_decode_args (include/lightdelta_hip.h)."""

    _fields_ = [
        ("qkv", _vp),
        ("qkv_row_stride", _c_i64),
        ("a", _vp),
        ("a_row_stride", _c_i64),
        ("b", _vp),
        ("b_row_stride", _c_i64),
        ("a_log", _vp),
        ("dt_bias", _vp),
        ("dt_bias_dtype", _c_i32),
        ("norm_weight_dtype", _c_i32),
        ("indices", _vp),
        ("cu", _vp),
        ("accepted", _vp),
        ("state", _vp),
        ("state_slot_stride", _c_i64),
        ("gate", _vp),
        ("gate_row_stride", _c_i64),
        ("norm_weight", _vp),
        ("out", _vp),
        ("num_requests", _c_i32),
        ("width", _c_i32),
        ("num_k_heads", _c_i32),
        ("num_v_heads", _c_i32),
        ("scale", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("cache_policy", _c_i32),
    ]


class ConvArgs(ctypes.Structure):
    """Mirror of ld_conv_args (include/lightdelta_hip.h)."""

    _fields_ = [
        ("x", _vp),
        ("x_row_stride", _c_i64),
        ("state", _vp),
        ("state_slots", _c_i64),
        ("state_slot_stride", _c_i64),
        ("state_dim_stride", _c_i64),
        ("state_len_stride", _c_i64),
        ("state_len", _c_i32),
        ("width", _c_i32),
        ("weight", _vp),
        ("weight_dtype", _c_i32),
        ("bias_dtype", _c_i32),
        ("bias", _vp),
    ]


class PrefillArgs(ctypes.Structure):
    """Mirror of ld_gdn_prefill_args (include/lightdelta_hip.h)."""

    _fields_ = [
        ("qkv", _vp),
        ("qkv_row_stride", _c_i64),
        ("a", _vp),
        ("a_row_stride", _c_i64),
        ("b", _vp),
        ("b_row_stride", _c_i64),
        ("a_log", _vp),
        ("dt_bias", _vp),
        ("dt_bias_dtype", _c_i32),
        ("norm_weight_dtype", _c_i32),
        ("slots", _vp),
        ("has_initial", _vp),
        ("cu_seqlens", _vp),
        ("state", _vp),
        ("state_slot_stride", _c_i64),
        ("gate", _vp),
        ("gate_row_stride", _c_i64),
        ("norm_weight", _vp),
        ("out", _vp),
        ("num_tokens", _c_i64),
        ("num_sequences", _c_i32),
        ("num_k_heads", _c_i32),
        ("num_v_heads", _c_i32),
        ("scale", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("algorithm", _c_i32),
        ("workspace", _vp),
        ("workspace_bytes", _c_i64),
    ]


PREFILL_AUTO, PREFILL_TOKEN_SERIAL, PREFILL_CHUNKED, PREFILL_CHUNKED_32 = 0, 1, 2, 3
PREFILL_STATIC_SCRATCH_BYTES = 64 << 20


# Exported entry points and their C signatures (argtypes, restype).
SIGNATURES = {
    "ld_gdn_decode": ([ctypes.POINTER(DecodeArgs), _vp], ctypes.c_int),
    "ld_gdn_prefill": ([ctypes.POINTER(PrefillArgs), _vp], ctypes.c_int),
    "ld_gdn_prefill_static": ([ctypes.POINTER(PrefillArgs), _vp], ctypes.c_int),
    "ld_gdn_prefill_workspace_bytes": ([_c_i64, _c_i32, _c_i32], _c_i64),
    "ld_gdn_prefill_auto_chunked": ([_c_i64, _c_i32, _c_i32], _c_i32),
    "ld_gdn_decode_conv": (
        [ctypes.POINTER(DecodeArgs), ctypes.POINTER(ConvArgs), _vp],
        ctypes.c_int,
    ),
    "ld_state_gather": (
        [_vp, _c_i64, _vp, _c_i64, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp],
        ctypes.c_int,
    ),
    "ld_state_scatter": (
        [_vp, _c_i64, _vp, _c_i64, _vp, _c_i64, _c_i64, _c_i64, _vp],
        ctypes.c_int,
    ),
    "ld_state_copy": ([_vp, _c_i64, _vp, _vp, _c_i64, _c_i64, _vp], ctypes.c_int),
    "ld_state_copy_checked": ([_vp, _c_i64, _vp, _vp, _c_i64, _c_i64, _vp, _vp], ctypes.c_int),
    "ld_state_zero": ([_vp, _c_i64, _vp, _c_i64, _c_i64, _vp], ctypes.c_int),
    "ld_packed_plan": ([_vp, _vp, _vp, _c_i32, _c_i32, _vp, _vp, _vp, _vp, _vp], ctypes.c_int),
    "ld_last_error": ([], ctypes.c_char_p),
    "ld_abi_version": ([], ctypes.c_int),
}

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises RuntimeError if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIBRARY_PATH.exists():
                raise RuntimeError(
                    f"{LIBRARY_PATH.name} is not built; run `python -m lightdelta_amd.build` "
                    "(hipcc, gfx950) before using the lightdelta ops"
                )
            lib = ctypes.CDLL(str(LIBRARY_PATH))
            for name, (argtypes, restype) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = restype
            version = lib.ld_abi_version()
            if version != ABI_VERSION:
                raise RuntimeError(f"{LIBRARY_PATH.name} ABI {version}, expected {ABI_VERSION}")
            _lib = lib
    return _lib


def check(code: int) -> None:
    """Raise RuntimeError with the library's message for a non-zero return code."""
    if code != 0:
        message = load().ld_last_error().decode(errors="replace")
        raise RuntimeError(message or f"lightdelta HIP call failed with code {code}")
