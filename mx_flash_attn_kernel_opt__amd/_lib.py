"""ctypes binding of libmxattn.so (declarations in include/mx_paged_decode.h).

The argument types mirror the reference's own binding of its kernel library
(verify_real.py:12-14: ``[c_void_p]*6 + [c_int64]*9``, ``restype=None`` for ``run_kernel``).
Loading fails loudly when the library has not been built: there is no fallback path.
"""

from __future__ import annotations

import ctypes
import os
import threading

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libmxattn.so")

# Status codes (include/mx_paged_decode.h)
MX_STATUS_OK = 0
MX_STATUS_NULL_POINTER = -1
MX_STATUS_INVALID_SHAPE = -2
MX_STATUS_UNSUPPORTED = -3
MX_STATUS_WORKSPACE_TOO_SMALL = -4
MX_STATUS_HIP_ERROR = -5
MX_STATUS_ALLOC_FAILED = -6
MX_STATUS_INVALID_ARGUMENT = -7

MX_DEVICE_BAD_PAGE_ID = 1
MX_DEVICE_SEQ_TOO_LONG = 2
MX_DEVICE_WORKSPACE_STATE = 4
# mx_read_device_status's workspace sentinel for the no-alloc array ((void*)(intptr_t)-1).
MX_NOALLOC_WORKSPACE = ctypes.c_void_p(-1).value

MX_SCHEDULE_SPLIT_GRID = 0
MX_SCHEDULE_BALANCED = 1
MX_SCHEDULE_SPLIT_GRID_PAIRED = 2
MX_SCHEDULE_BALANCED_PAIRED = 3

MX_PHASE_ALL = 0
MX_PHASE_MAIN_ONLY = 1
MX_PHASE_COMBINE_ONLY = 2

STATUS_NAMES = {
    MX_STATUS_OK: "OK",
    MX_STATUS_NULL_POINTER: "NULL_POINTER",
    MX_STATUS_INVALID_SHAPE: "INVALID_SHAPE",
    MX_STATUS_UNSUPPORTED: "UNSUPPORTED",
    MX_STATUS_WORKSPACE_TOO_SMALL: "WORKSPACE_TOO_SMALL",
    MX_STATUS_HIP_ERROR: "HIP_ERROR",
    MX_STATUS_ALLOC_FAILED: "ALLOC_FAILED",
    MX_STATUS_INVALID_ARGUMENT: "INVALID_ARGUMENT",
}

# (name, restype, argtypes) for every function of include/mx_paged_decode.h
_VP, _I64, _I32, _F32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_float
_P64 = ctypes.POINTER(ctypes.c_int64)
_P32 = ctypes.POINTER(ctypes.c_int32)
SIGNATURES = {
    "run_kernel": (None, [_VP] * 6 + [_I64] * 9),
    "mx_paged_gqa_decode": (
        ctypes.c_int,
        [_VP] * 6 + [_I64] * 9 + [_I32, _F32, _I64, _VP, _I64, _I32, _VP],
    ),
    "mx_paged_gqa_decode_noalloc": (
        ctypes.c_int,
        [_VP] * 6 + [_I64] * 9 + [_I32, _F32, _I64, _VP],
    ),
    "mx_paged_gqa_decode_fp8kv": (
        ctypes.c_int,
        [_VP] * 6 + [_I64] * 9 + [_I32, _F32, _F32, _F32, _I64, _VP, _I64, _I32, _VP],
    ),
    "mx_paged_gqa_decode_partial": (
        ctypes.c_int,
        [_VP] * 7 + [_I64] * 9 + [_I32, _F32, _I64, _VP, _I64, _VP],
    ),
    "mx_lse_merge": (ctypes.c_int, [_VP, _VP, _I64, _I64, _I64, _VP, _VP]),
    "mx_paged_gqa_decode_plan": (ctypes.c_int, [_I64] * 10 + [_P64] * 5),
    "mx_paged_gqa_decode_plan_fp8kv": (ctypes.c_int, [_I64] * 10 + [_P64] * 5),
    "mx_paged_gqa_decode_workspace_size": (ctypes.c_int64, [_I64] * 9),
    "mx_paged_kv_append": (ctypes.c_int, [_VP] * 6 + [_I64] * 7 + [_VP, _VP]),
    "mx_paged_gqa_decode_append": (
        ctypes.c_int,
        [_VP] * 8 + [_I64] * 10 + [_I32, _F32, _I64, _VP, _I64, _VP],
    ),
    "mx_paged_kv_append_fp8kv": (ctypes.c_int, [_VP] * 6 + [_I64] * 7 + [_F32, _F32, _VP, _VP]),
    "mx_paged_gqa_decode_append_fp8kv": (
        ctypes.c_int,
        [_VP] * 8 + [_I64] * 10 + [_I32, _F32, _F32, _F32, _I64, _VP, _I64, _VP],
    ),
    "mx_read_device_status": (ctypes.c_int, [_VP, _I32, _VP, _P32]),
    "mx_last_status": (ctypes.c_int, []),
    "mx_last_error": (ctypes.c_char_p, []),
    "mx_version": (ctypes.c_char_p, []),
}


class MXAttnError(RuntimeError):
    """A libmxattn call returned a negative status."""

    def __init__(self, status: int, message: str):
        self.status = status
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")


_lock = threading.Lock()
_lib = None


def library_path() -> str:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Load libmxattn.so once; raise if it has not been built."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -m "
                    "mx_flash_attn_kernel_opt__amd.build` (or __graft_entry__.build())"
                )
            lib = ctypes.CDLL(LIB_PATH)
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = lib
        return _lib


def check(status: int) -> None:
    if status != MX_STATUS_OK:
        msg = load().mx_last_error()
        raise MXAttnError(status, msg.decode() if msg else "")
