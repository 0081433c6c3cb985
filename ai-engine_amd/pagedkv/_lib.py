"""ctypes declarations of libpagedkv's C ABI (include/pagedkv.h).

The library is the product: every call here goes straight to the HIP
kernels or the C++ host code.  There is no fallback -- if the shared object
is missing, loading fails with an error that says how to build it.
"""
from __future__ import annotations

import ctypes
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("PKV_LIB", os.path.join(os.path.dirname(_PKG), "libpagedkv.so"))

PKV_OK = 0
PKV_ERR_INVALID = -1
PKV_ERR_OOM = -2
PKV_ERR_HIP = -3
PKV_ERR_UNSUPPORTED = -4
PKV_ERR_CAPACITY = -5
PKV_ERR_DEVICE_DATA = -6

F32, F16, BF16 = 0, 1, 2
K, V = 0, 1

_P = ctypes.c_void_p
_I = ctypes.c_int
_SZ = ctypes.c_size_t
_I32P = ctypes.POINTER(ctypes.c_int32)



class PrefillBatch(ctypes.Structure):
    """struct pkv_prefill_batch."""
    _fields_ = [("q", _P), ("out", _P), ("out_dtype", _I), ("cu_q_lens", _P),
                ("context_lens", _P), ("block_tables", _P), ("max_blocks_per_seq", _I),
                ("n_seqs", _I), ("max_q_len", _I), ("max_context_len", _I), ("k_new", _P),
                ("v_new", _P)]


class DecodeBatch(ctypes.Structure):
    """struct pkv_decode_batch."""
    _fields_ = [("q", _P), ("out", _P), ("out_dtype", _I), ("block_tables", _P),
                ("max_blocks_per_seq", _I), ("context_lens", _P), ("max_context_len", _I),
                ("batch", _I), ("k_new", _P), ("v_new", _P)]


_PBP = ctypes.POINTER(PrefillBatch)
_DBP = ctypes.POINTER(DecodeBatch)

# name -> (restype, argtypes); mirrors include/pagedkv.h one to one.
SIGNATURES: dict[str, tuple] = {
    "pkv_version": (ctypes.c_char_p, []),
    "pkv_last_error": (ctypes.c_char_p, [_P]),
    "pkv_pool_create": (_I, [ctypes.POINTER(_P), _I, _I, _I, _I, _I, _I, _I]),
    "pkv_pool_destroy": (_I, [_P]),
    "pkv_pool_shape": (_I, [_P] + [ctypes.POINTER(_I)] * 6),
    "pkv_pool_layer_bytes": (_SZ, [_P]),
    "pkv_pool_layer_ptrs": (_I, [_P, _I, ctypes.POINTER(_P), ctypes.POINTER(_P)]),
    "pkv_pool_read": (_I, [_P, _I, _I, _SZ, _SZ, _P]),
    "pkv_pool_write": (_I, [_P, _I, _I, _SZ, _P, _SZ]),
    "pkv_pool_fill_normal": (_I, [_P, ctypes.c_uint64, _P]),
    "pkv_pool_verify_normal": (_I, [_P, ctypes.c_uint64, _P, _P, _I,
                                    ctypes.POINTER(ctypes.c_uint64), _P]),
    "pkv_pool_read_blocks": (_I, [_P, _P, _I, _P, _P]),
    "pkv_append": (_I, [_P, _I, _P, _P, _P, _I, _P]),
    "pkv_append_rope": (_I, [_P, _I, _P, _P, _I, _P, _P, _P, _I, _P, _P, _I, _P]),
    "pkv_gather_seq": (_I, [_P, _I, _P, _I, _P, _P, _P]),
    "pkv_gather_varlen": (_I, [_P, _I, _P, _I, _P, _I, _I, _P, _P, _P]),
    "pkv_copy_blocks": (_I, [_P, _P, _P, _I, _P]),
    "pkv_compact": (_I, [_P, _I32P, _I32P, _I, _P]),
    "pkv_decode_attention": (_I, [_P, _I, _P, _P, _I, _P, _I, _P, _I, _I, _I,
                                  ctypes.c_float, _P, _P, _P]),
    "pkv_decode_attention_noalloc": (_I, [_P, _I, _P, _P, _I, _P, _I, _P, _I, _I, _I,
                                          ctypes.c_float, _P, _P, _P]),
    "pkv_decode_attention_positions": (_I, [_P, _I, _P, _P, _I, _P, _I, _P, _P, _I, _I, _I,
                                            ctypes.c_float, _P, _P, _P]),
    "pkv_decode_workspace_bytes": (_SZ, [_P, _I, _I, _I]),
    "pkv_pool_reserve_decode": (_I, [_P, _I, _I, _I]),
    "pkv_prefill_attention": (_I, [_P, _I, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I,
                                   ctypes.c_float, _P]),
    "pkv_prefill_attention_append": (_I, [_P, _I, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I,
                                          ctypes.c_float, _P, _P, _P]),
    "pkv_pool_check": (_I, [_P]),
    "pkv_prefill_workspace_bytes": (_SZ, [_P, _I, _I, _I, _I]),
    "pkv_pool_reserve_prefill": (_I, [_P, _I, _I, _I, _I]),
    "pkv_mixed_attention": (_I, [_P, _I, _PBP, _DBP, _I, ctypes.c_float, _P]),
    "pkv_mixed_workspace_bytes": (_SZ, [_P, _I, _PBP, _DBP]),
    "pkv_rope_tables_host": (_I, [_I, ctypes.c_float, _I, _P, _P]),
    "pkv_rope_create": (_I, [ctypes.POINTER(_P), _I, ctypes.c_float, _I, _I]),
    "pkv_rope_destroy": (_I, [_P]),
    "pkv_rope_tables": (_I, [_P, ctypes.POINTER(_P), ctypes.POINTER(_P)]),
    "pkv_rope_apply": (_I, [_P, _P, _I, _P, _I, _P, _I, _I, _P]),
    "pkv_rope_check": (_I, [_P]),
    "pkv_decode_attention_rope": (_I, [_P, _I, _P, _P, _I, _P, _P, _I, _P, _I, _P, _I, _I, _I,
                                       ctypes.c_float, _P, _P, _P]),
    "pkv_sched_last_error": (ctypes.c_char_p, []),
    "pkv_sched_create": (_I, [ctypes.POINTER(_P), _P]),
    "pkv_sched_destroy": (None, [_P]),
    "pkv_sched_submit": (_I, [_P, _I, _I, ctypes.POINTER(ctypes.c_int64)]),
    "pkv_sched_step": (_I, [_P, _P]),
    "pkv_sched_complete": (_I, [_P, _P, _I, ctypes.c_char_p]),
    "pkv_sched_poll": (_I, [_P, _P]),
    "pkv_sched_fork": (_I, [_P, ctypes.c_int64, _I, ctypes.POINTER(ctypes.c_int64)]),
    "pkv_sched_compact": (_I, [_P, _P, _P, _I, ctypes.POINTER(_I)]),
    "pkv_sched_counts": (_I, [_P, ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "pkv_sched_table": (_I, [_P, ctypes.c_int64, ctypes.POINTER(ctypes.POINTER(ctypes.c_uint32)),
                             ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "pkv_sample": (_I, [_P, _I, ctypes.c_longlong, _I, _I, _P, _I, ctypes.c_float,
                        ctypes.c_uint64, _P, _P]),
    "pkv_sample_exact": (_I, [_P, _I, ctypes.c_longlong, _I, _I, _P, _I, ctypes.c_float,
                              ctypes.c_uint64, _P, _P]),
    "pkv_sample_exact_routes": (_I, [_P, _I, ctypes.c_longlong, _I, _I, _P, _I, ctypes.c_float,
                                     ctypes.c_uint64, _P, _P, _P]),
    "pkv_sample_expf": (_I, [_P, _P, ctypes.c_longlong, _P]),
    "pkv_sample_draw": (ctypes.c_float, [ctypes.c_uint64]),
    "pkv_pool_profile": (_I, [_P, _I]),
    "pkv_pool_profile_read": (_I, [_P, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_I)]),
    "pkv_allocator_new": (_P, [_SZ, _SZ]),
    "pkv_allocator_free": (None, [_P]),
    "pkv_allocator_free_count": (_SZ, [_P]),
    "pkv_allocator_blocks_for": (_SZ, [_P, _SZ]),
    "pkv_allocator_ensure_capacity": (_I, [_P, _P, _SZ]),
    "pkv_allocator_release": (None, [_P, _P]),
    "pkv_allocator_locate": (_I, [_P, _P, _SZ, ctypes.POINTER(ctypes.c_uint32),
                                  ctypes.POINTER(_SZ)]),
    "pkv_table_new": (_P, []),
    "pkv_table_free": (None, [_P]),
    "pkv_table_len": (_SZ, [_P]),
    "pkv_table_blocks": (ctypes.POINTER(ctypes.c_uint32), [_P]),
}

_lib: ctypes.CDLL | None = None


class PagedKvError(RuntimeError):
    """A libpagedkv call returned a negative status."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class CapacityError(PagedKvError):
    """The allocator's free list cannot satisfy the request (the reference's
    Err(()) from ensure_capacity, block_table.rs:32-47)."""


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise OSError(
                f"libpagedkv.so not found at {LIB_PATH}; build it with "
                "`python ai-engine_amd/build.py` (or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int, pool=None) -> None:
    if rc == PKV_OK:
        return
    msg = lib().pkv_last_error(pool).decode(errors="replace")
    if rc == PKV_ERR_CAPACITY:
        raise CapacityError(rc, msg or "KV cache exhausted")
    raise PagedKvError(rc, msg)
