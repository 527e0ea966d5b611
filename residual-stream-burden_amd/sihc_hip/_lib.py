"""ctypes binding of libsihc_hip.so, the C ABI declared in include/sihc_hip.h.

The library is required: there is no CPU or PyTorch fallback for any op, and a
missing or stale build raises at first use.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libsihc_hip.so")
ABI_VERSION = 5
MAX_EVENTS = 32
DTYPE_F32 = 0
DTYPE_BF16 = 1

_vp = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t
_vpp = ctypes.POINTER(ctypes.c_void_p)

# name -> (restype, argtypes); mirrors include/sihc_hip.h one for one.
PROTOTYPES: dict[str, tuple] = {
    "sihc_last_error": (ctypes.c_char_p, []),
    "sihc_abi_version": (_i32, []),
    "sihc_read": (_i32, [_vp, _vp, _vpp, _i32, _i64, _i32, _i32, _i32, _vp, _i32, _vp]),
    "sihc_write": (_i32, [_vp, _vpp, _vp, _vp, _i32, _i64, _i32, _i32, _i32, _i32, _vp, _i32, _i32, _vp]),
    "sihc_weight_grad_workspace_size": (_sz, [_i32, _i64, _i32, _i32, _i32]),
    "sihc_weight_grad": (_i32, [_vp, _vpp, _vp, _i32, _i64, _i32, _i32, _i32, _vp, _i32, _i32, _vp, _sz, _vp]),
    "sihc_triangular": (_i32, [_vp, _vpp, _vp, _vp, _i32, _i64, _i32, _i32, _i32, _vp]),
    "sihc_triangular_gamma_grad_workspace_size": (_sz, [_i32, _i64, _i32]),
    "sihc_triangular_gamma_grad": (_i32, [_vp, _vpp, _vp, _i32, _i64, _i32, _i32, _i32, _vp, _sz, _vp]),
    "sihc_triangular_backward": (_i32, [_vp, _vpp, _vp, _vpp, _vp, _i32, _i64, _i32, _i32, _i32, _i32,
                                        _vp, _sz, _vp]),
    "sihc_event_forward": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _vp, _i32, _vp]),
    "sihc_event_backward_workspace_size": (_sz, [_i64, _i32, _i32, _i32]),
    "sihc_event_backward": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                   _i64, _i32, _i32, _i32, _vp, _i32, _i32, _vp, _sz, _vp]),
    "sihc_event_backward_partial": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                           _i64, _i32, _i32, _i32, _vp, _i32, _i32, _vp, _sz,
                                           ctypes.POINTER(ctypes.c_int), _vp]),
    "sihc_event_backward_chain": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                         _i64, _i32, _i32, _i32, _vp, _i32, _i32, _vp, _sz,
                                         ctypes.POINTER(ctypes.c_int), _vp, _sz, ctypes.POINTER(ctypes.c_int),
                                         _vp, _vp, _vp]),
    "sihc_event_finalize": (_i32, [_i32, _vpp, ctypes.POINTER(_sz), ctypes.POINTER(ctypes.c_int), _vpp, _vpp,
                                   _i32, _i32, _i32, _vp]),
    "sihc_event_backward_noalloc": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                           _i64, _i32, _i32, _i32, _vp, _i32, _i32, _vp]),
    "sihc_gather_cells": (_i32, [_vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _vp]),
    "sihc_scatter_cells": (_i32, [_vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _vp]),
    "sihc_scatter_add_cells": (_i32, [_vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _vp]),
    "sihc_stream": (_i32, [_vpp, _i32, _vpp, _i32, _sz, _i32, _vp]),
    "sihc_stream_mix": (_i32, [_vpp, _i32, _i32, _vpp, _i32, _i32, _i32, _sz, _vp, _vp]),
    "sihc_copy": (_i32, [_vp, _vp, _sz, _vp]),
    "sihc_fma_rate": (_i32, [_vp, _i32, _i32, _i32, _i32, _vp]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class SihcError(RuntimeError):
    """A C-ABI call returned an error code."""


def lib() -> ctypes.CDLL:
    """Load the library once and declare every prototype. Raises if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with "
                    "`python residual-stream-burden_amd/build.py` (hipcc, gfx950)")
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in PROTOTYPES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            version = handle.sihc_abi_version()
            if version != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH} has ABI {version}, expected {ABI_VERSION}: rebuild it")
            _lib = handle
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        msg = lib().sihc_last_error().decode(errors="replace")
        raise SihcError(msg or f"sihc call failed with code {rc}")


def size_array(sizes) -> ctypes.Array:
    sizes = list(sizes)
    return (ctypes.c_size_t * max(1, len(sizes)))(*sizes)


def ptr_array(ptrs) -> ctypes.Array:
    ptrs = list(ptrs)
    return (ctypes.c_void_p * max(1, len(ptrs)))(*ptrs)
