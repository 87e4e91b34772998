"""ctypes binding of the loom-hip C ABI (``include/loom_hip.h``).

The library is loaded from the in-tree build ``attnarc_amd/_build/
libloom_hip.so``. There is no fallback: if the library is missing or fails to
load, every call raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

from . import build as _build

# LOOM_HIP_LIBRARY selects another build of the same ABI (A/B runs, the
# profiling build); it is read when the library is first loaded.
LIB_PATH = os.environ.get("LOOM_HIP_LIBRARY", _build.LIB_PATH)


def library_path() -> str:
    return os.environ.get("LOOM_HIP_LIBRARY", _build.LIB_PATH)

SUCCESS = 0
INVALID_ARGUMENT = 1
UNSUPPORTED = 2
LAUNCH_ERROR = 3
UNAVAILABLE = 4

KV_CACHE_NATIVE = 0
KV_CACHE_FP8_E4M3 = 1

F32, F16, BF16 = 0, 1, 2
ROPE_PAGED_KV_WRITE = 5
PAGED_DECODE_ATTENTION = 9
KERNEL_DECODE, KERNEL_MERGE, KERNEL_ROPE = 0, 1, 2
# F32 elements of the per-device array behind the no-allocation entry point
# (LOOM_HIP_STATIC_WORKSPACE_ELEMENTS in include/loom_hip.h).
STATIC_WORKSPACE_ELEMENTS = 16 * 1024 * 1024

# Bridge status codes (include/loom_hip_bridge.h); they differ from the
# unchecked library's codes above, as loom_cuda_bridge.h's do from loom_cuda.h's.
BRIDGE_SUCCESS, BRIDGE_INVALID_ARGUMENT, BRIDGE_LAUNCH_ERROR, BRIDGE_UNAVAILABLE = 0, 1, 2, 3

P = ctypes.c_void_p
U32 = ctypes.c_uint32
U64 = ctypes.c_uint64
F = ctypes.c_float

# (name, argtypes, restype) for every symbol declared in include/loom_hip.h,
# include/loom_hip_bridge.h and include/loom_hip_views.h.
_BASE = [P, P, P, P, P, P] + [U32] * 7 + [U64, U64, U32, U32, F, P]
_SPLIT = [P, P, P, P, P, P, P, U64] + [U32] * 7 + [U64, U64, U32, U32, F, P]
_EXT = [P, P, P, P, P, P, P, P, P, P, U64] + [U32] * 9 + [U64] * 6 + [U32, U32, U32, F, P]
_NO_ALLOC = [U32] + [P] * 9 + [U32] * 9 + [U64] * 6 + [U32, U32, U32, F, P]
_ROPE = [P] * 10 + [U32] * 12 + [U64] * 12 + [U32, P]
# Checked bridge (include/loom_hip_bridge.h).
_BRIDGE_ROPE = [U32, U32] + [P, U64] * 10 + [U32] * 10 + [U64] * 12 + [U32, P]
_BRIDGE_DECODE = [U32] + [P, U64] * 7 + [U32] * 7 + [U64, U64, U32, U32, F, P]

class TensorView(ctypes.Structure):
    """``loom_hip_tensor_view`` (include/loom_hip_views.h)."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("device_index", ctypes.c_int32),
        ("dtype", ctypes.c_uint32),
        ("rank", ctypes.c_uint32),
        ("sizes", ctypes.c_int64 * 5),
        ("strides", ctypes.c_int64 * 5),
    ]


VIEW_F32, VIEW_F16, VIEW_BF16, VIEW_U8, VIEW_FP8_E4M3FN, VIEW_I32, VIEW_I64, VIEW_OTHER = 0, 1, 2, 3, 4, 5, 6, 255
VIEWS_OK, VIEWS_CONTRACT, VIEWS_BRIDGE = 0, 1, 2
_VIEWS = ctypes.POINTER(TensorView)
D = ctypes.c_double
I64 = ctypes.c_int64

SIGNATURES = {
    "loom_hip_status_string": ([ctypes.c_int], ctypes.c_char_p),
    "loom_hip_paged_decode_attention_f32": (_BASE, ctypes.c_int),
    "loom_hip_paged_decode_attention_f16": (_BASE, ctypes.c_int),
    "loom_hip_paged_decode_attention_bf16": (_BASE, ctypes.c_int),
    "loom_hip_paged_decode_attention_split_k_workspace_elements": ([U32] * 6, U64),
    "loom_hip_paged_decode_attention_split_k_f32": (_SPLIT, ctypes.c_int),
    "loom_hip_paged_decode_attention_split_k_f16": (_SPLIT, ctypes.c_int),
    "loom_hip_paged_decode_attention_split_k_bf16": (_SPLIT, ctypes.c_int),
    "loom_hip_paged_decode_attention_extended_workspace_elements": ([U32] * 5, U64),
    "loom_hip_paged_decode_attention_extended_f32": (_EXT, ctypes.c_int),
    "loom_hip_paged_decode_attention_extended_f16": (_EXT, ctypes.c_int),
    "loom_hip_paged_decode_attention_extended_bf16": (_EXT, ctypes.c_int),
    "loom_hip_paged_decode_attention_extended_no_alloc": (_NO_ALLOC, ctypes.c_int),
    "loom_hip_paged_decode_attention_supports": (
        [U32] * 11 + [F, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_char_p)],
        ctypes.c_int,
    ),
    "loom_hip_rope_paged_kv_write_f32": (_ROPE, ctypes.c_int),
    "loom_hip_rope_paged_kv_write_f16": (_ROPE, ctypes.c_int),
    "loom_hip_rope_paged_kv_write_bf16": (_ROPE, ctypes.c_int),
    "loom_hip_backend_name": ([], ctypes.c_char_p),
    "loom_hip_bridge_abi_version": ([], U32),
    "loom_hip_bridge_last_error_message": ([], ctypes.c_char_p),
    "loom_hip_bridge_launch_count": ([U32, ctypes.POINTER(U64)], ctypes.c_int),
    "loom_hip_bridge_reset_launch_count": ([U32], ctypes.c_int),
    "loom_hip_bridge_rope_paged_kv_write": (_BRIDGE_ROPE, ctypes.c_int),
    "loom_hip_bridge_paged_decode_workspace_elements": ([U32] * 10 + [F, ctypes.POINTER(U64)], ctypes.c_int),
    "loom_hip_bridge_paged_decode_attention": (_BRIDGE_DECODE, ctypes.c_int),
    "loom_hip_views_last_error_message": ([], ctypes.c_char_p),
    "loom_hip_views_paged_decode_check": ([_VIEWS, U32, I64, D], ctypes.c_int),
    "loom_hip_views_paged_decode_workspace_elements": ([_VIEWS, I64, D, ctypes.POINTER(U64)], ctypes.c_int),
    "loom_hip_views_paged_decode_attention": ([_VIEWS, I64, D, P, U64, P], ctypes.c_int),
    "loom_hip_views_rope_paged_kv_check": ([_VIEWS], ctypes.c_int),
    "loom_hip_views_rope_paged_kv_write": ([_VIEWS, U32, P], ctypes.c_int),
    "loom_hip_abi_version": ([], U32),
    "loom_hip_last_error_message": ([], ctypes.c_char_p),
    "loom_hip_last_kernel_family": ([], ctypes.c_char_p),
    "loom_hip_last_internal_partition_tokens": ([], ctypes.c_uint32),
    "loom_hip_last_kernel_name": ([], ctypes.c_char_p),
    "loom_hip_paged_decode_attention_plan": ([U32] * 8 + [ctypes.c_void_p, ctypes.POINTER(U32), ctypes.POINTER(U32)],
                                             ctypes.c_int),
    "loom_hip_launch_count": ([U32, ctypes.POINTER(U64)], ctypes.c_int),
    "loom_hip_reset_launch_count": ([U32], ctypes.c_int),
    "loom_hip_kernel_timing_enable": ([U32], ctypes.c_int),
    "loom_hip_kernel_timing_read": ([U32, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(U64)], ctypes.c_int),
}

_lib = None
_lock = threading.Lock()


class LoomHipError(RuntimeError):
    """A non-success status from the loom-hip C ABI."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


def lib() -> ctypes.CDLL:
    """Load the in-tree HIP library (raises if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            global LIB_PATH
            LIB_PATH = library_path()
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"loom-hip native library not found at {LIB_PATH}; "
                    "run `python -m attnarc_amd.build` (or __graft_entry__.build())"
                )
            handle = ctypes.CDLL(LIB_PATH)
            for name, (argtypes, restype) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.argtypes = argtypes
                fn.restype = restype
            _lib = handle
    return _lib


def status_string(status: int) -> str:
    return lib().loom_hip_status_string(status).decode()


def last_error() -> str:
    return lib().loom_hip_last_error_message().decode()


def check(status: int, what: str) -> None:
    if status != SUCCESS:
        raise LoomHipError(
            status, f"{what} failed: {status_string(status)}: {last_error()}"
        )
