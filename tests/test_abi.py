"""The C-ABI library loads and exports every entry point include/lightdelta_hip.h declares
(no GPU calls), and its argument checks fail with the documented codes without launching."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from lightdelta_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "lightdelta_hip.h"


def declared_functions() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(ld_\w+)\s*\(", text, flags=re.M))


def test_header_declares_the_entry_points():
    assert declared_functions() == {
        "ld_gdn_decode", "ld_gdn_decode_conv", "ld_gdn_prefill", "ld_gdn_prefill_static",
        "ld_gdn_prefill_workspace_bytes", "ld_gdn_prefill_auto_chunked", "ld_state_gather",
        "ld_state_scatter",
        "ld_state_copy", "ld_state_copy_checked", "ld_state_zero", "ld_packed_plan",
        "ld_last_error", "ld_abi_version",
    }


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert set(_lib.SIGNATURES) == declared_functions()
    assert lib.ld_abi_version() == _lib.ABI_VERSION


@pytest.mark.parametrize("struct,mirror", [("ld_gdn_decode_args", _lib.DecodeArgs),
                                           ("ld_conv_args", _lib.ConvArgs),
                                           ("ld_gdn_prefill_args", _lib.PrefillArgs)])
def test_args_layout_matches_header(struct, mirror):
    """ctypes mirrors of the argument structs: same field names in the same order."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    body = re.search(r"typedef struct " + struct + r" \{(.*?)\}", text, flags=re.S).group(1)
    fields = re.findall(r"(\w+);", body)
    assert fields == [name for name, _ in mirror._fields_]


@pytest.mark.parametrize("width,heads,eps,message", [
    (0, (16, 32), 1e-6, "1 through 4 tokens"),
    (5, (16, 32), 1e-6, "1 through 4 tokens"),
    (1, (16, 24), 1e-6, "multiple of num_k_heads"),
    (1, (16, 32), 0.0, "epsilon must be positive"),
])
def test_decode_rejects_bad_arguments_without_launching(width, heads, eps, message):
    lib = _lib.load()
    args = _lib.DecodeArgs()
    args.num_requests = 1
    args.width = width
    args.num_k_heads, args.num_v_heads = heads
    args.eps = eps
    args.scale = 128 ** -0.5
    code = lib.ld_gdn_decode(ctypes.byref(args), None)
    assert code == 1
    assert message in lib.ld_last_error().decode()


def test_empty_work_is_a_no_op():
    lib = _lib.load()
    args = _lib.DecodeArgs()
    args.num_requests = 0
    args.width = 1
    args.num_k_heads, args.num_v_heads = 16, 32
    args.eps = 1e-6
    assert lib.ld_gdn_decode(ctypes.byref(args), None) == 0
    assert lib.ld_state_copy(None, 0, None, None, 0, 2048, None) == 0
    assert lib.ld_state_copy_checked(None, 0, None, None, 0, 2048, None, None) == 0
    assert lib.ld_state_zero(None, 0, None, 0, 2048, None) == 0
    assert lib.ld_state_gather(None, 0, None, 1, None, None, 0, 2048, 0, None) == 0


def test_decode_conv_rejects_bad_widths_and_conv_shapes():
    lib = _lib.load()
    args = _lib.DecodeArgs()
    args.num_requests = 1
    args.num_k_heads, args.num_v_heads = 16, 32
    args.eps = 1e-6
    conv = _lib.ConvArgs()
    conv.width, conv.state_len, conv.weight_dtype = 4, 3, _lib.DTYPE_BF16
    args.width = 5
    assert lib.ld_gdn_decode_conv(ctypes.byref(args), ctypes.byref(conv), None) == 1
    assert "1 through 4 tokens" in lib.ld_last_error().decode()
    args.width = 1
    conv.width = 3
    assert lib.ld_gdn_decode_conv(ctypes.byref(args), ctypes.byref(conv), None) == 1
    assert "conv width must be 4" in lib.ld_last_error().decode()
    conv.width, conv.state_len = 4, 9
    assert lib.ld_gdn_decode_conv(ctypes.byref(args), ctypes.byref(conv), None) == 1
    assert "3 through 8" in lib.ld_last_error().decode()
    conv.state_len, conv.state_slots = 3, (1 << 20)
    assert lib.ld_gdn_decode_conv(ctypes.byref(args), ctypes.byref(conv), None) == 1
    assert "too large" in lib.ld_last_error().decode()


def test_copy_rejects_misaligned_rows():
    lib = _lib.load()
    code = lib.ld_state_gather(16, 24, 32, 1, None, 48, 24, 24, 1, None)
    assert code == 1 and "16-byte aligned" in lib.ld_last_error().decode()
    code = lib.ld_state_zero(16, 2048, 32, 1, 24, None)
    assert code == 1 and "16-byte aligned" in lib.ld_last_error().decode()


def test_checked_copy_needs_a_status_array_and_nonempty_slots():
    lib = _lib.load()
    assert lib.ld_state_copy_checked(16, 2048, 32, 48, 1, 2048, None, None) == 1
    assert b"rejected is NULL" in lib.ld_last_error()
    assert lib.ld_state_copy_checked(16, 2048, 32, 48, 1, 0, 64, None) == 1
    assert b"slot_bytes must be positive" in lib.ld_last_error()


def test_packed_plan_rejects_bad_arguments_without_launching():
    lib = _lib.load()
    assert lib.ld_packed_plan(None, None, None, 0, 1, None, None, None, None, None) == 0
    for batch, width in ((-1, 1), (4, 0), (4, 5)):
        assert lib.ld_packed_plan(None, None, None, batch, width, None, None, None, None,
                                  None) == 1
        assert b"width 1..4" in lib.ld_last_error()
    assert lib.ld_packed_plan(16, None, 16, 4, 1, 16, 16, 16, 16, None) == 1
    assert b"NULL pointer" in lib.ld_last_error()


def test_prefill_rejects_bad_arguments_without_launching():
    lib = _lib.load()
    args = _lib.PrefillArgs()
    args.num_sequences = 1
    args.num_k_heads, args.num_v_heads = 16, 24
    args.eps = 1e-6
    assert lib.ld_gdn_prefill(ctypes.byref(args), None) == 1
    assert "multiple of num_k_heads" in lib.ld_last_error().decode()
    args.num_v_heads = 32
    assert lib.ld_gdn_prefill(ctypes.byref(args), None) == 1
    assert "NULL tensor pointer" in lib.ld_last_error().decode()
    args.num_sequences = 0
    assert lib.ld_gdn_prefill(ctypes.byref(args), None) == 0


def test_prefill_workspace_query_and_chunked_without_workspace():
    lib = _lib.load()
    # one record of 28928 floats per (chunk, v-head), chunks <= tokens / 64 + sequences, then
    # the per-sequence chunk index (sequences + 1 int32, rounded up to 256 bytes)
    record = 28928 * 4
    assert lib.ld_gdn_prefill_workspace_bytes(4096, 1, 32) == (4096 // 64 + 1) * 32 * record + 256
    assert lib.ld_gdn_prefill_workspace_bytes(100, 70, 8) == (100 // 64 + 70) * 8 * record + 512
    assert lib.ld_gdn_prefill_workspace_bytes(-1, 1, 32) == 0
    args = _lib.PrefillArgs()
    args.num_sequences, args.num_tokens = 1, 64
    args.num_k_heads, args.num_v_heads = 16, 32
    args.eps = 1e-6
    args.algorithm = 7
    assert lib.ld_gdn_prefill(ctypes.byref(args), None) == 1
    assert "unknown prefill algorithm" in lib.ld_last_error().decode()


@pytest.mark.parametrize("tokens,sequences,heads,expected", [
    (4096, 1, 32, 64),        # one long prompt: 64-token chunks halve its chain of chunks
    (512, 1, 32, 64),
    (4096, 1, 63, 64),        # 63 (sequence, head) pairs
    (4096, 1, 64, 32),        # 64 pairs
    (2 * 2048, 2, 32, 32),
    (511, 1, 32, 32),         # a mean under 512 tokens
    (32 * 1024, 32, 32, 32),  # long prompts that fill the GPU anyway
    (16 * 128, 16, 32, 32),
    (512 * 64, 512, 32, 32),
    (1024 * 32, 1024, 32, 32),  # short prompts: one full 32-token chunk each
    (1024 * 36, 1024, 32, 32),  # a second chunk that holds few tokens
    (1024 * 20, 1024, 32, 32),
    (1024 * 17, 1024, 32, 32),  # the shortest that go chunked
    (1024 * 17 - 1, 1024, 32, 0),
    (1024 * 16, 1024, 32, 0),
    (2 * 16, 2, 32, 0),
    (0, 1, 32, 0),
    (100, 0, 32, 0),
])
def test_prefill_auto_rule(tokens, sequences, heads, expected):
    assert _lib.load().ld_gdn_prefill_auto_chunked(tokens, sequences, heads) == expected


def test_static_prefill_rejects_without_launching():
    """ld_gdn_prefill_static: a caller workspace, and a chunked prefill larger than the
    static scratch, are refused before anything touches a device."""
    lib = _lib.load()
    args = _lib.PrefillArgs()
    args.num_sequences, args.num_k_heads, args.num_v_heads = 32, 16, 32
    args.num_tokens, args.eps, args.scale = 32 * 1024, 1e-6, 128**-0.5
    args.algorithm = _lib.PREFILL_CHUNKED
    args.workspace, args.workspace_bytes = 256, 1 << 20
    assert lib.ld_gdn_prefill_static(args, None) == 1
    assert b"workspace must be NULL" in lib.ld_last_error()
    args.workspace, args.workspace_bytes = None, 0
    need = lib.ld_gdn_prefill_workspace_bytes(32 * 1024, 32, 32)
    assert need > _lib.PREFILL_STATIC_SCRATCH_BYTES
    assert lib.ld_gdn_prefill_static(args, None) == 1
    assert b"static scratch" in lib.ld_last_error()
