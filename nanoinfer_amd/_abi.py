"""ctypes binding of ``include/nanoinfer_kv.h`` (the C ABI of the gfx950 path).

The library is ``nanoinfer_amd/libnanoinfer_kv.so``, built in-tree by
``nanoinfer_amd/build.py``.  Loading never falls back to anything else: if the
library is missing and cannot be built, :func:`lib` raises.
"""
from __future__ import annotations

import ctypes as C
import os
import re

from . import build as _build

HEADER = os.path.join(_build.INCLUDE, "nanoinfer_kv.h")

NI_KV_BLOCK = 16
NI_ALL_LAYERS = -1
NI_KV_HOST_ONLY = 1
NI_KV_Q8 = 2

NI_OK = 0
NI_ERR_NO_SLOT = 1
NI_ERR_CONTEXT_FULL = 2
NI_ERR_POOL_EXHAUSTED = 3
NI_ERR_NOT_LIVE = 4
NI_ERR_BAD_LEN = 5
NI_ERR_HIP = 6
NI_ERR_BAD_ARG = 7
NI_ERR_EMPTY_WORK = 8
NI_ERR_TOO_MANY_ROWS = 9
NI_ERR_NOT_RESERVED = 10
NI_ERR_NO_DEVICE = 11

NI_K_APPEND, NI_K_ATTN, NI_K_MERGE, NI_K_QKV, NI_K_COUNT = 0, 1, 2, 3, 4

NI_W_F32, NI_W_F16, NI_W_Q8_0, NI_W_Q4_0 = 0, 1, 2, 3


class ni_kv_opts(C.Structure):
    _fields_ = [
        ("n_layer", C.c_uint32),
        ("n_head", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("kv_pages", C.c_uint32),
        ("max_seqs", C.c_uint32),
        ("max_ctx", C.c_uint32),
        ("max_rows", C.c_uint32),
        ("flags", C.c_uint32),
        ("page_order", C.POINTER(C.c_uint32)),
    ]


class ni_row(C.Structure):
    _fields_ = [("seq", C.c_uint32), ("pos", C.c_uint32)]


class ni_work(C.Structure):
    _fields_ = [("seq", C.c_uint32), ("n_new", C.c_uint32), ("n_query", C.c_uint32)]


_lib = None
_vp = C.c_void_p
_i64 = C.c_int64
_u32 = C.c_uint32


def _declare(L):
    L.ni_version.restype = C.c_char_p
    L.ni_version.argtypes = []
    L.ni_kv_last_error.restype = C.c_char_p
    L.ni_kv_last_error.argtypes = [_vp]
    L.ni_kv_create.restype = C.c_int
    L.ni_kv_create.argtypes = [C.POINTER(ni_kv_opts), C.POINTER(_vp)]
    L.ni_kv_destroy.restype = None
    L.ni_kv_destroy.argtypes = [_vp]
    L.ni_kv_page_bytes.restype = C.c_size_t
    L.ni_kv_page_bytes.argtypes = [_vp]
    L.ni_kv_add_seq.restype = C.c_int
    L.ni_kv_add_seq.argtypes = [_vp, C.POINTER(_u32)]
    L.ni_kv_free_seq.restype = C.c_int
    L.ni_kv_free_seq.argtypes = [_vp, _u32]
    L.ni_kv_seq_len.restype = C.c_int
    L.ni_kv_seq_len.argtypes = [_vp, _u32, C.POINTER(_u32)]
    L.ni_kv_is_live.restype = C.c_int
    L.ni_kv_is_live.argtypes = [_vp, _u32, C.POINTER(C.c_int)]
    L.ni_kv_truncate.restype = C.c_int
    L.ni_kv_truncate.argtypes = [_vp, _u32, _u32]
    L.ni_kv_reserve.restype = C.c_int
    L.ni_kv_reserve.argtypes = [_vp, _u32, _u32]
    L.ni_kv_commit.restype = C.c_int
    L.ni_kv_commit.argtypes = [_vp, _u32, _u32]
    L.ni_kv_block_table.restype = C.c_int
    L.ni_kv_block_table.argtypes = [_vp, _u32, C.POINTER(C.POINTER(_u32)), C.POINTER(_u32)]
    L.ni_kv_blocks_used.restype = _u32
    L.ni_kv_blocks_used.argtypes = [_vp]
    L.ni_kv_free_block_count.restype = _u32
    L.ni_kv_free_block_count.argtypes = [_vp]
    L.ni_kv_append.restype = C.c_int
    L.ni_kv_append.argtypes = [_vp, C.c_int32, C.POINTER(ni_row), _u32, _vp, _vp, _i64, _i64, _vp]
    L.ni_kv_qkv_append.restype = C.c_int
    L.ni_kv_qkv_append.argtypes = [_vp, C.c_int32, C.POINTER(ni_row), _u32, _vp, _i64, _u32, _vp, _vp, _vp, _i64, _vp]
    L.ni_kv_qkv_project.restype = C.c_int
    L.ni_kv_qkv_project.argtypes = [_vp, _vp, _i64, _u32, _u32, _vp, _vp, _vp, _i64, _vp]
    L.ni_kv_qkv_append_w.restype = C.c_int
    L.ni_kv_qkv_append_w.argtypes = [_vp, C.c_int32, C.POINTER(ni_row), _u32, _vp, _i64, _u32, _vp, _u32, _vp, _vp, _i64,
                                     _vp]
    L.ni_kv_qkv_project_w.restype = C.c_int
    L.ni_kv_qkv_project_w.argtypes = [_vp, _vp, _i64, _u32, _u32, _vp, _u32, _vp, _vp, _i64, _vp]
    L.ni_kv_gather_q8.restype = C.c_int
    L.ni_kv_gather_q8.argtypes = [_vp, C.c_int32, C.POINTER(ni_row), _u32, _vp, _vp, _vp, _vp, _vp]
    L.ni_kv_gather.restype = C.c_int
    L.ni_kv_gather.argtypes = [_vp, C.c_int32, C.POINTER(ni_row), _u32, _vp, _vp, _i64, _i64, _vp]
    L.ni_paged_decode_attention.restype = C.c_int
    L.ni_paged_decode_attention.argtypes = [_vp, C.c_int32, _vp, _i64, _i64, C.POINTER(ni_row), _u32, _vp, _i64,
                                            _i64, _u32, _vp]
    L.ni_kv_step.restype = C.c_int
    L.ni_kv_step.argtypes = [_vp, C.POINTER(ni_work), _u32, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _i64, _u32, _vp]
    L.ni_stream_probe.restype = C.c_int
    L.ni_stream_probe.argtypes = [_u32, _vp, _vp, C.c_size_t, _u32, _vp]
    L.ni_kv_step_noalloc.restype = C.c_int
    L.ni_kv_step_noalloc.argtypes = L.ni_kv_step.argtypes
    L.ni_kv_step_begin.restype = C.c_int
    L.ni_kv_step_begin.argtypes = [_vp, C.POINTER(ni_work), _u32, _u32]
    L.ni_kv_step_layer.restype = C.c_int
    L.ni_kv_step_layer.argtypes = [_vp, C.c_int32, _vp, _vp, _vp, _i64, _vp, _i64, _vp]
    L.ni_kv_step_end.restype = C.c_int
    L.ni_kv_step_end.argtypes = [_vp]
    L.ni_kv_decode_steps.restype = C.c_int
    L.ni_kv_decode_steps.argtypes = [_vp, C.POINTER(_u32), _u32, _u32, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _i64, _i64,
                                     _i64, _u32, _vp]
    L.ni_kv_sync.restype = C.c_int
    L.ni_kv_sync.argtypes = [_vp, _vp]
    L.ni_kv_pools.restype = C.c_int
    L.ni_kv_pools.argtypes = [_vp, C.POINTER(_vp), C.POINTER(_vp), C.POINTER(C.c_size_t)]
    L.ni_attention.restype = C.c_int
    L.ni_attention.argtypes = [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _u32, _u32, _u32, _u32, _vp]
    L.ni_f32_to_f16.restype = C.c_int
    L.ni_f32_to_f16.argtypes = [_vp, _vp, C.c_size_t, _vp]
    L.ni_kv_profile.restype = C.c_int
    L.ni_kv_profile.argtypes = [_vp, _u32]
    L.ni_kv_profile_read.restype = C.c_int
    L.ni_kv_profile_read.argtypes = [_vp, C.c_int, C.POINTER(C.c_double), C.POINTER(C.c_uint64)]


def lib():
    """The loaded library; builds it first only if it does not exist."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_build.LIB):
        _build.build()
    L = C.CDLL(_build.LIB)
    _declare(L)
    _lib = L
    return L


def library_path() -> str:
    return _build.LIB


def declared_functions() -> list[str]:
    """Every function the public header declares (for the export check)."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ni_[a-z0-9_]+)\s*\(", text)))
