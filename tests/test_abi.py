"""CPU: the C-ABI library loads, exports every declared symbol, and rejects bad
arguments before any launch (no kernel runs here)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from sihc_hip import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "sihc_hip.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(sihc_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_functions()
    assert len(names) >= 14, names
    for name in names:
        assert hasattr(lib, name), f"{name} declared in sihc_hip.h but not exported"
    # ... and the ctypes prototypes cover exactly the header.
    assert set(names) == set(_lib.PROTOTYPES), set(names) ^ set(_lib.PROTOTYPES)
    assert lib.sihc_abi_version() == _lib.ABI_VERSION


def test_workspace_sizes_are_pure_functions_of_sizes():
    lib = _lib.lib()
    # 65,536 tokens (batch 256 of a 16x16 grid), 24 events, 4 slots, 1152 channels.
    ws = lib.sihc_weight_grad_workspace_size(24, 256, 16, 2, 1152)
    assert ws == 128 * 24 * 4 * 1152 * 4
    assert lib.sihc_weight_grad_workspace_size(0, 256, 16, 2, 1152) == 0
    # few event lanes: more chunks (about 16 waves per CU), at least 32 tokens each
    assert lib.sihc_triangular_gamma_grad_workspace_size(3, 147, 67) == 4 * 3 * 67 * 4
    assert lib.sihc_triangular_gamma_grad_workspace_size(1, 65536, 1152) == 1366 * 1 * 1152 * 4
    # the query also covers the fused triangular backward: one chunk per 64 tokens, at
    # most 1024 (more than the 152 chunks the 11-update gamma gradient takes)
    assert lib.sihc_triangular_gamma_grad_workspace_size(11, 65536, 1152) == 1024 * 11 * 1152 * 4
    # per-event backward: 4-slot cells one chunk per 64 tokens up to 1024, 16-slot cells one
    # per 256 tokens up to 512
    assert lib.sihc_event_backward_workspace_size(256, 16, 2, 1152) == 1024 * 2 * 4 * 1152 * 4
    assert lib.sihc_event_backward_workspace_size(3, 16, 2, 136) == 12 * 2 * 4 * 136 * 4
    assert lib.sihc_event_backward_workspace_size(256, 16, 4, 1152) == 256 * 2 * 16 * 1152 * 4


FAKE = 0x1000  # never dereferenced: every call below fails argument validation first


@pytest.mark.parametrize("events", [0, 33])
def test_event_count_is_validated_before_launch(events):
    lib = _lib.lib()
    outs = _lib.ptr_array([FAKE] * max(events, 1))
    rc = lib.sihc_read(FAKE, FAKE, outs, events, 2, 16, 2, 64, None, _lib.DTYPE_BF16, None)
    assert rc == 1
    assert b"events must be in 1..32" in lib.sihc_last_error()


def test_bad_cell_dtype_and_null_pointers_are_rejected():
    lib = _lib.lib()
    outs = _lib.ptr_array([FAKE])
    assert lib.sihc_read(FAKE, FAKE, outs, 1, 2, 16, 3, 64, None, _lib.DTYPE_BF16, None) == 1
    assert b"cell must be 2 or 4" in lib.sihc_last_error()
    assert lib.sihc_read(FAKE, FAKE, outs, 1, 2, 16, 2, 64, None, 7, None) == 1
    assert b"bad dtype" in lib.sihc_last_error()
    assert lib.sihc_read(None, FAKE, outs, 1, 2, 16, 2, 64, None, _lib.DTYPE_BF16, None) == 1
    assert b"null" in lib.sihc_last_error()
    nulls = _lib.ptr_array([FAKE, None])
    assert lib.sihc_write(FAKE, nulls, FAKE, FAKE, 2, 2, 16, 2, 64, 1, None, 1, 1, None) == 1
    assert b"null tensor pointer 1" in lib.sihc_last_error()
    assert lib.sihc_write(FAKE, outs, FAKE, FAKE, 1, 2, 16, 2, 64, 1, None,
                          _lib.DTYPE_BF16, _lib.DTYPE_F32, None) == 1
    assert lib.sihc_event_forward(FAKE, FAKE, FAKE, FAKE, FAKE, None, 2, 16, 2, 64, None, 1, None) == 1
    assert b"alpha_next and z_out" in lib.sihc_last_error()


def test_too_small_workspace_is_rejected():
    lib = _lib.lib()
    ups = _lib.ptr_array([FAKE])
    rc = lib.sihc_weight_grad(FAKE, ups, FAKE, 1, 256, 16, 2, 1152, None, 1, 1, FAKE, 16, None)
    assert rc == 1 and b"workspace of" in lib.sihc_last_error()
    rc = lib.sihc_event_backward(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                                 256, 16, 2, 1152, None, 1, 1, FAKE, 16, None)
    assert rc == 1 and b"workspace of" in lib.sihc_last_error()
    rc = lib.sihc_triangular_backward(FAKE, ups, FAKE, ups, FAKE, 1, 65536, 1152, 1, 1, 0, FAKE, 16, None)
    assert rc == 1 and b"workspace of" in lib.sihc_last_error()


def test_triangular_backward_arguments_are_validated():
    lib = _lib.lib()
    ups = _lib.ptr_array([FAKE, FAKE])
    nulls = _lib.ptr_array([FAKE, None])
    ws = 1 << 30
    assert lib.sihc_triangular_backward(FAKE, ups, FAKE, nulls, FAKE, 2, 512, 64, 1, 1, 0, FAKE, ws, None) == 1
    assert b"null tensor pointer 1" in lib.sihc_last_error()
    assert lib.sihc_triangular_backward(FAKE, ups, FAKE, ups, None, 2, 512, 64, 1, 1, 0, FAKE, ws, None) == 1
    assert b"null output" in lib.sihc_last_error()
    assert lib.sihc_triangular_backward(FAKE, ups, FAKE, ups, FAKE, 2, 512, 64, 1, 5, 0, FAKE, ws, None) == 1
    assert b"bad dtype" in lib.sihc_last_error()
    assert lib.sihc_triangular_backward(FAKE, ups, FAKE, ups, FAKE, 33, 512, 64, 1, 1, 0, FAKE, ws, None) == 1
    assert b"1..32" in lib.sihc_last_error()


def test_event_backward_weight_dtype_must_match_carrier():
    # beta / alpha_next are read as the carrier dtype: fp32 weights with a bf16 carrier
    # would be reinterpreted, so the mismatch is an argument error
    lib = _lib.lib()
    rc = lib.sihc_event_backward(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                                 2, 16, 2, 64, None, _lib.DTYPE_BF16, _lib.DTYPE_F32, FAKE, 1 << 30, None)
    assert rc == 1 and b"weights must share the carrier dtype" in lib.sihc_last_error()


def test_scatter_add_cells_arguments_are_validated():
    lib = _lib.lib()
    assert lib.sihc_scatter_add_cells(FAKE, FAKE, None, 2, 16, 2, 64, _lib.DTYPE_BF16, None) == 1
    assert b"null pointer" in lib.sihc_last_error()
    assert lib.sihc_scatter_add_cells(FAKE, FAKE, FAKE, 2, 16, 2, 64, 9, None) == 1
    assert b"bad dtype" in lib.sihc_last_error()
    assert lib.sihc_scatter_add_cells(FAKE, FAKE, FAKE, 2, 16, 3, 64, _lib.DTYPE_BF16, None) == 1
    assert b"cell must be 2 or 4" in lib.sihc_last_error()
    # empty batch: nothing to do, no pointer is touched
    assert lib.sihc_scatter_add_cells(None, None, None, 0, 16, 2, 64, _lib.DTYPE_BF16, None) == 0


def test_deferred_finalize_arguments_are_validated():
    lib = _lib.lib()
    info = (ctypes.c_int * 2)(7, 3)
    one = _lib.ptr_array([FAKE])
    nul = _lib.ptr_array([None])
    rc = lib.sihc_event_backward_partial(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                                         2, 16, 2, 64, None, 1, 1, FAKE, 1 << 30, None, None)
    assert rc == 1 and b"null info" in lib.sihc_last_error()
    big = _lib.size_array([1 << 30])
    assert lib.sihc_event_finalize(1, one, big, info, nul, one, 2, 64, 1, None) == 1
    assert b"null gradient of event 0" in lib.sihc_last_error()
    bad = (ctypes.c_int * 2)(7, 4)
    assert lib.sihc_event_finalize(1, one, big, bad, one, one, 2, 64, 1, None) == 1
    assert b"bad info" in lib.sihc_last_error()
    assert lib.sihc_event_finalize(1, one, big, info, one, one, 3, 64, 1, None) == 1
    # 7 partial rows of 2 x 4 slots x 64 channels need 14,336 bytes
    small = _lib.size_array([7 * 2 * 4 * 64 * 4 - 4])
    assert lib.sihc_event_finalize(1, one, small, info, one, one, 2, 64, 1, None) == 1
    assert b"partial rows need 14336" in lib.sihc_last_error()
    assert lib.sihc_event_finalize(1, one, None, info, one, one, 2, 64, 1, None) == 1
    assert b"null array" in lib.sihc_last_error()
    assert lib.sihc_event_finalize(0, None, None, None, None, None, 2, 64, 1, None) == 0  # nothing to do
    empty = (ctypes.c_int * 2)(0, 0)  # a zero-token event: no partial rows, nothing read
    assert lib.sihc_event_finalize(1, nul, _lib.size_array([0]), empty, nul, nul, 2, 64, 1, None) == 0


def test_stream_calibration_arguments_are_validated():
    lib = _lib.lib()
    arr = _lib.ptr_array([FAKE, FAKE])
    assert lib.sihc_stream(arr, 3, arr, 1, 1 << 20, 0, None) == 1
    assert b"unsupported mix" in lib.sihc_last_error()
    assert lib.sihc_stream(arr, 1, arr, 1, 1000, 0, None) == 1
    assert b"multiple of 4096" in lib.sihc_last_error()
    assert lib.sihc_stream(_lib.ptr_array([FAKE + 8]), 1, arr, 1, 1 << 20, 0, None) == 1
    assert b"misaligned" in lib.sihc_last_error()
    assert lib.sihc_stream(arr, 1, arr, 1, 1 << 20, 3, None) == 1
    assert b"shape must be" in lib.sihc_last_error()
    assert lib.sihc_stream(arr, 2, arr, 1, 1 << 20, 1, None) == 1
    assert b"shape 1 takes" in lib.sihc_last_error()
    assert lib.sihc_stream(arr, 2, arr, 2, 1 << 20, 2, None) == 1
    assert b"shape 2 takes" in lib.sihc_last_error()


def test_stream_mix_arguments_are_validated():
    lib = _lib.lib()
    arr = _lib.ptr_array([FAKE] * 33)
    assert lib.sihc_stream_mix(arr, 33, 0, arr, 1, 0, 1, 1 << 20, None, None) == 1
    assert b"sources and" in lib.sihc_last_error()
    assert lib.sihc_stream_mix(arr, 0, 0, arr, 0, 0, 1, 1 << 20, None, None) == 1
    assert b"not both 0" in lib.sihc_last_error()
    assert lib.sihc_stream_mix(arr, 2, 3, arr, 1, 0, 4, 1 << 20, None, None) == 1
    assert b"carrier-shaped counts" in lib.sihc_last_error()
    assert lib.sihc_stream_mix(arr, 2, 1, arr, 1, 2, 4, 1 << 20, None, None) == 1
    assert b"carrier-shaped counts" in lib.sihc_last_error()
    assert lib.sihc_stream_mix(arr, 2, 1, arr, 1, 0, 8, 1 << 20, None, None) == 1
    assert b"slots must be" in lib.sihc_last_error()
    assert lib.sihc_stream_mix(arr, 2, 1, arr, 1, 0, 4, 1000, None, None) == 1
    assert b"multiple of 4096" in lib.sihc_last_error()
    assert lib.sihc_stream_mix(_lib.ptr_array([FAKE, FAKE + 8]), 2, 1, arr, 1, 0, 4, 1 << 20, None, None) == 1
    assert b"misaligned" in lib.sihc_last_error()
    assert lib.sihc_stream_mix(arr, 2, 1, arr, 0, 0, 4, 1 << 20, None, None) == 1
    assert b"needs a 16-byte aligned sink" in lib.sihc_last_error()
    assert lib.sihc_stream_mix(arr, 2, 1, arr, 0, 0, 4, 0, None, None) == 0  # nothing to move


def test_oversized_tensor_is_rejected():
    lib = _lib.lib()
    outs = _lib.ptr_array([FAKE])
    assert lib.sihc_read(FAKE, FAKE, outs, 1, 1 << 40, 16, 2, 64, None, 1, None) == 1
    assert b"too large" in lib.sihc_last_error()


def test_fma_rate_arguments_are_validated():
    lib = _lib.lib()
    assert lib.sihc_fma_rate(FAKE, 5, 0, 1, 1, None) == 1
    assert b"chains must be 4, 8 or 16" in lib.sihc_last_error()
    assert lib.sihc_fma_rate(FAKE, 4, 4, 1, 1, None) == 1
    assert b"form must be 0..3" in lib.sihc_last_error()
    assert lib.sihc_fma_rate(FAKE, 4, 0, 0, 1, None) == 1
    assert b"must be positive" in lib.sihc_last_error()
    assert lib.sihc_fma_rate(None, 4, 0, 1, 1, None) == 1
    assert b"null or misaligned" in lib.sihc_last_error()


def test_token_counts_stop_short_of_int32():
    # chunk ends (chunks x tokens per chunk < tokens + chunks) and a thread's next token
    # are int32 in the kernels: token and row counts must stay below 2^31 - 2^16
    lib = _lib.lib()
    limit = (1 << 31) - (1 << 16)
    ups = _lib.ptr_array([FAKE])
    assert limit % 256 == 0  # limit // 256 batches of a 16 x 16 grid: exactly the limit
    assert lib.sihc_read(FAKE, FAKE, ups, 1, limit // 256, 16, 2, 64, None, 1, None) == 1
    assert b"too large" in lib.sihc_last_error()
    assert lib.sihc_triangular(FAKE, ups, FAKE, FAKE, 1, limit, 64, 1, 0, None) == 1
    assert b"bad sizes" in lib.sihc_last_error()
    assert lib.sihc_triangular_gamma_grad(FAKE, ups, FAKE, 1, limit, 64, 1, 0, FAKE, 1 << 30, None) == 1
    assert b"bad sizes" in lib.sihc_last_error()
    assert lib.sihc_triangular_backward(FAKE, ups, FAKE, ups, FAKE, 1, limit, 64, 1, 0, 0, FAKE, 1 << 30,
                                        None) == 1
    assert b"bad sizes" in lib.sihc_last_error()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libsihc_hip.so")
    with pytest.raises(RuntimeError, match="missing"):
        _lib.lib()
