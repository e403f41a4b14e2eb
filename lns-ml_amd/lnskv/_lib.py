"""ctypes binding of liblnskv.so (the C ABI declared in include/lnskv.h).

The shared library is built in-tree (lns-ml_amd/liblnskv.so).  Loading fails
loudly when it is missing: there is no CPU fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "liblnskv.so")

PAGE_SIZE = 16
NO_PAGE = 0xFFFFFFFF

DTYPE_F32, DTYPE_F16, DTYPE_Q8A = 0, 1, 2
DTYPE_NAMES = {DTYPE_F32: "f32", DTYPE_F16: "f16", DTYPE_Q8A: "q8a"}
DTYPE_BYTES = {DTYPE_F32: 4, DTYPE_F16: 2, DTYPE_Q8A: 1}

OK = 0
ERR_INVALID = -1
ERR_NOMEM = -2
ERR_POOL_EXHAUSTED = -3
ERR_HIP = -4
ERR_UNSUPPORTED = -5
ERR_WORKSPACE = -6

# changed block-table entries that one lnskv_block_tables_sync writes by value
TABLE_PATCH_MAX = 64

# leading bytes of a decode workspace that must be zero before its first use
# (the workgroup schedule's counters; every call leaves them zero)
WORKSPACE_HEADER_BYTES = 4096


class LnskvError(RuntimeError):
    """A non-zero lnskv_status with the library's message (the reference's
    Result<(), String> error, lns-inference/src/engine.rs:2969-2971)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"lnskv status {status}: {message}")
        self.status = status
        self.message = message


class Pages(C.Structure):
    """lnskv_pages: one layer's paged K/V pools (device pointers + geometry)."""

    _fields_ = [
        ("k_pages", C.c_void_p),
        ("v_pages", C.c_void_p),
        ("k_scales", C.c_void_p),
        ("v_scales", C.c_void_p),
        ("num_pages", C.c_uint32),
        ("n_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("dtype", C.c_int32),
    ]


class Rope(C.Structure):
    """lnskv_rope: device inverse frequencies + rotary width."""

    _fields_ = [("inv_freqs_dev", C.c_void_p), ("rotary_dim", C.c_int32)]


_P = C.POINTER(Pages)
_R = C.POINTER(Rope)
_vp, _i32, _u32, _sz, _f32 = C.c_void_p, C.c_int32, C.c_uint32, C.c_size_t, C.c_float

# name -> (restype, argtypes); every symbol include/lnskv.h declares.
SIGNATURES = {
    "lnskv_last_error": (C.c_char_p, []),
    "lnskv_version": (C.c_char_p, []),
    "lnskv_page_bytes": (_sz, [_P]),
    "lnskv_pages_alloc": (C.c_int, [_P]),
    "lnskv_pages_free": (C.c_int, [_P]),
    "lnskv_clear": (C.c_int, [_P, _vp]),
    "lnskv_append": (C.c_int, [_P, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _i32, _vp]),
    "lnskv_decode_workspace_size": (C.c_int, [_P, _i32, _i32, _i32, _i32, C.POINTER(_sz)]),
    "lnskv_decode": (C.c_int, [_P, _vp, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _i32, _f32, _i32, _vp, _sz, _vp]),
    "lnskv_append_decode": (
        C.c_int, [_P, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _i32, _f32, _i32, _vp, _sz, _vp]),
    "lnskv_append_decode_noalloc": (
        C.c_int, [_P, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _i32, _f32, _i32, _vp]),
    "lnskv_attention_paged": (C.c_int, [_vp, _vp, _vp, _P, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _vp]),
    "lnskv_dispatch_attention_paged": (
        C.c_int, [_vp, _vp, _vp, _P, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _vp]),
    "lnskv_page_copy": (C.c_int, [_P, _vp, _vp, _i32, _vp]),
    "lnskv_gather": (C.c_int, [_P, _vp, _i32, _i32, _vp, _vp, _vp, _vp, _vp]),
    "lnskv_sync": (C.c_int, [_vp]),
    "lnskv_workspace_reserve": (C.c_int, [_sz, _sz, _sz]),
    "lnskv_workspace_release": (C.c_int, []),
    "lnskv_page_pool_create": (C.c_int, [_u32, C.POINTER(_vp)]),
    "lnskv_page_pool_destroy": (None, [_vp]),
    "lnskv_page_pool_alloc": (C.c_int, [_vp, C.POINTER(_u32)]),
    "lnskv_page_pool_free": (C.c_int, [_vp, _u32]),
    "lnskv_page_pool_retain": (C.c_int, [_vp, _u32]),
    "lnskv_page_pool_reset": (None, [_vp]),
    "lnskv_page_pool_num_free": (_u32, [_vp]),
    "lnskv_page_pool_capacity": (_u32, [_vp]),
    "lnskv_page_pool_refcount": (_u32, [_vp, _u32]),
    "lnskv_block_tables_create": (C.c_int, [_i32, _i32, C.POINTER(_vp)]),
    "lnskv_block_tables_destroy": (None, [_vp]),
    "lnskv_block_tables_host": (C.POINTER(_u32), [_vp]),
    "lnskv_block_tables_stride": (_i32, [_vp]),
    "lnskv_block_tables_len": (_i32, [_vp, _i32]),
    "lnskv_block_tables_reset": (None, [_vp]),
    "lnskv_ensure_kv_page": (C.c_int, [_vp, _vp, _i32, _i32, _i32]),
    "lnskv_evict_kv_pages": (C.c_int, [_vp, _vp, _i32, _i32, _i32]),
    "lnskv_kv_p_start": (_i32, [_i32, _i32]),
    "lnskv_step_pages": (C.c_int, [_vp, _vp, _i32, _i32, _i32, _i32]),
    "lnskv_window_pages": (_i32, [_i32]),
    "lnskv_free_sequence": (C.c_int, [_vp, _vp, _i32]),
    "lnskv_fork_sequence": (
        C.c_int, [_vp, _vp, _i32, _i32, _i32, C.POINTER(_u32), C.POINTER(_u32), C.POINTER(_i32)]),
    "lnskv_block_tables_upload": (C.c_int, [_vp, _vp, _vp]),
    "lnskv_block_tables_sync": (C.c_int, [_vp, _vp, _vp]),
    "lnskv_block_tables_changed": (C.c_int64, [_vp]),
    "lnskv_block_table_patch": (C.c_int, [_vp, _i32, _vp, _vp, _vp]),
    "lnskv_rope_dim": (_i32, [_i32, _f32]),
    "lnskv_rope_inv_freqs": (C.c_int, [_i32, _f32, _i32, _vp, _vp]),
    "lnskv_rope_append_workspace_size": (C.c_int, [_P, _R, _i32, C.POINTER(_sz)]),
    "lnskv_rope_append": (C.c_int, [_P, _R, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _i32, _vp, _sz, _vp]),
    "lnskv_rope_decode_workspace_size": (C.c_int, [_P, _R, _i32, _i32, _i32, _i32, C.POINTER(_sz)]),
    "lnskv_rope_append_decode": (
        C.c_int, [_P, _R, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _i32, _f32, _i32, _vp, _sz, _vp]),
    "lnskv_prefill_attention": (C.c_int, [_P, _vp, _vp, _vp, _i32, _i32, _vp, _i32, _i32, _vp, _i32, _i32, _f32,
                                          _vp]),
    "lnskv_split_gated_query": (C.c_int, [_vp, _vp, _vp, _i32, _i32, _i32, _vp]),
    "lnskv_gated_append_decode": (
        C.c_int, [_P, _R, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _i32, _f32, _i32, _vp, _sz,
                  _vp]),
    "lnskv_read_units": (C.c_int, [_P, _vp, _vp, _vp, _i32, _vp, _vp]),
    "lnskv_read_stream": (C.c_int, [_vp, _sz, _i32, _i32, _vp, _vp]),
    "lnskv_q4l_prepare": (C.c_int, [_vp, _sz, _i32, _i32, _vp]),
    "lnskv_q4l_workspace_size": (C.c_int, [_i32, _i32, C.POINTER(_sz)]),
    "lnskv_q4l_gemv_accumulate": (C.c_int, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _sz, _vp]),
}

ROPE_DEFAULT, ROPE_LINEAR, ROPE_LLAMA3, ROPE_YARN = 0, 1, 2, 3

_lib = None


def lib() -> C.CDLL:
    """The loaded liblnskv.so; raises if it was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `make -C lns-ml_amd` or "
                "`python -c 'import __graft_entry__ as g; g.build()'` (no CPU fallback exists)")
        # torch first: its HIP runtime (soname libamdhip64.so.7, loaded by torch
        # under the name libamdhip64.so) then satisfies this library's
        # dependency, so the process has one runtime.  Loaded the other way
        # round, torch brings a second runtime and ours sees no device.
        import torch  # noqa: F401

        handle = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def last_error() -> str:
    return lib().lnskv_last_error().decode()


def check(status: int) -> None:
    if status != OK:
        raise LnskvError(status, last_error())
