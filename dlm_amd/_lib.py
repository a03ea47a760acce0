"""ctypes loader for libdlmk.so and the signatures of include/dlmk.h.

There is no fallback: if the library is missing or fails to load, every entry
point raises.  Build it with ``python -m dlm_amd.build``.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

PKG = os.path.dirname(os.path.abspath(__file__))
# DLMK_LIBRARY points at another build of the same ABI (e.g. a tuning variant).
LIB_PATH = os.environ.get("DLMK_LIBRARY") or os.path.join(PKG, "libdlmk.so")

DLMK_F32, DLMK_F16, DLMK_BF16, DLMK_I8, DLMK_I4 = 0, 1, 2, 3, 4
DLMK_OK = 0
DLMK_ERR_INVALID_ARG = -1
DLMK_ERR_KV_EXHAUSTED = -2
DLMK_ERR_UNSUPPORTED = -3
DLMK_ERR_WORKSPACE = -4
DLMK_ERR_UNKNOWN_SEQ = -5


class KvCacheConfigC(C.Structure):
    _fields_ = [("num_layers", C.c_uint32), ("num_kv_heads", C.c_uint32),
                ("head_dim", C.c_uint32), ("block_size", C.c_uint32)]


class KvCacheStatsC(C.Structure):
    _fields_ = [("total_blocks", C.c_uint32), ("used_blocks", C.c_uint32),
                ("free_blocks", C.c_uint32), ("_pad", C.c_uint32),
                ("num_sequences", C.c_uint64), ("used_tokens", C.c_uint64),
                ("capacity_tokens", C.c_uint64), ("bytes_per_block", C.c_uint64)]


class KvExhaustedC(C.Structure):
    _fields_ = [("requested", C.c_uint32), ("free", C.c_uint32), ("total", C.c_uint32)]


_vp, _i32, _i64, _u32, _u64, _f32, _sz = (C.c_void_p, C.c_int, C.c_int64, C.c_uint32,
                                          C.c_uint64, C.c_float, C.c_size_t)
_cfgp = C.POINTER(KvCacheConfigC)

# name -> (restype, argtypes); one line per declaration in include/dlmk.h.
SIGNATURES = {
    "dlmk_abi_version": (_i32, []),
    "dlmk_get_last_error_string": (C.c_char_p, []),
    "dlmk_bytes_per_token": (_u64, [_cfgp]),
    "dlmk_bytes_per_block": (_u64, [_cfgp]),
    "dlmk_blocks_for_tokens": (_u64, [_cfgp, _u64]),
    "dlmk_cache_new": (_vp, [_cfgp, _u32]),
    "dlmk_cache_with_budget": (_vp, [_cfgp, _u64]),
    "dlmk_cache_new_with_free_order": (_vp, [_cfgp, _vp, _u32]),
    "dlmk_cache_destroy": (None, [_vp]),
    "dlmk_cache_append_tokens": (_i32, [_vp, _u64, _u64, C.POINTER(KvExhaustedC)]),
    "dlmk_cache_free_sequence": (None, [_vp, _u64]),
    "dlmk_cache_truncate_sequence": (_i32, [_vp, _u64, _u64]),
    "dlmk_cache_fork_sequence": (_i32, [_vp, _u64, _u64, _vp, _u32, C.POINTER(C.c_uint32),
                                        C.POINTER(KvExhaustedC)]),
    "dlmk_cache_fork_sequence_shared": (_i32, [_vp, _u64, _u64]),
    "dlmk_cache_append_tokens_cow": (_i32, [_vp, _u64, _u64, _vp, C.POINTER(C.c_uint32),
                                            C.POINTER(KvExhaustedC)]),
    "dlmk_cache_block_refcount": (_u32, [_vp, _u32]),
    "dlmk_cache_sequence_len": (_u64, [_vp, _u64]),
    "dlmk_cache_block_table": (_i64, [_vp, _u64, _vp, _u64]),
    "dlmk_cache_num_sequences": (_u64, [_vp]),
    "dlmk_cache_stats": (None, [_vp, C.POINTER(KvCacheStatsC)]),
    "dlmk_cache_free_list": (_u32, [_vp, _vp, _u32]),
    "dlmk_cache_slot_mapping": (_i32, [_vp, _u64, _u64, _u64, _vp]),
    "dlmk_cache_fill_block_tables": (_i32, [_vp, _vp, _u32, _u32, _vp, _vp]),
    "dlmk_kv_append": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i64, _i32]),
    "dlmk_paged_attention_workspace_size": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "dlmk_decode_block_workspace_size": (_sz, [_i32] * 7),
    "dlmk_decode_block_paged": (_i32, [_vp] + [_i32] * 7 + [_f32, _i32, _i32] + [_vp] * 14 +
                                [_vp, _vp, _i64, _vp, _i32, _i32, _i32, _vp, _sz]),
    "dlmk_verify_block_workspace_size": (_sz, [_i32] * 8),
    "dlmk_verify_block_paged": (_i32, [_vp] + [_i32] * 7 + [_f32, _i32, _i32] + [_vp] * 14 +
                                [_vp, _vp, _i64, _vp, _i32, _i32, _i32, _i32, _vp, _sz]),
    "dlmk_paged_decode_attention": (_i32, [_vp, _vp, _i32, _vp, _vp, _vp, _i32, _vp, _vp, _i32,
                                           _i32, _i32, _i32, _i32, _i32, _i32, _i64, _f32, _vp,
                                           _sz]),
    "dlmk_paged_decode_attention_noalloc": (_i32, [_vp, _vp, _i32, _vp, _vp, _vp, _i32, _vp, _vp,
                                                   _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i64,
                                                   _f32]),
    "dlmk_paged_decode_step": (_i32, [_vp, _vp, _i32, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _i32,
                                      _i32, _i32, _i32, _i32, _i32, _i32, _i64, _f32, _vp, _sz]),
    "dlmk_kv_append_quant": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _i64, _i32,
                                    _i32, _i32, _i64, _i32]),
    "dlmk_paged_decode_attention_quant": (_i32, [_vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _i32,
                                                 _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32,
                                                 _i32, _i64, _f32, _vp, _sz]),
    "dlmk_copy_blocks": (_i32, [_vp, _vp, _vp, _vp, _i64, _sz, _i64]),
    "dlmk_gather_blocks": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _sz, _i64]),
    "dlmk_scatter_blocks": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _sz, _i64]),
    "dlmk_swap_out": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _sz, _i64, _vp, _sz]),
    "dlmk_swap_in": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _sz, _i64, _vp, _sz]),
    "dlmk_alloc_pinned": (_i32, [C.POINTER(C.c_void_p), _sz]),
    "dlmk_free_pinned": (_i32, [_vp]),
}


class DlmkError(RuntimeError):
    """A libdlmk call failed; ``code`` is the DLMK_ERR_* or hipError_t value."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


_lib = None
_lock = threading.Lock()


def lib() -> C.CDLL:
    """The loaded libdlmk.so (raises if it was never built)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise ImportError(
                        f"{LIB_PATH} is missing: build it with `python -m dlm_amd.build` "
                        "(there is no CPU fallback)")
                L = C.CDLL(LIB_PATH)
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(L, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = L
    return _lib


def last_error() -> str:
    msg = lib().dlmk_get_last_error_string()
    return msg.decode() if msg else ""


def check(code: int) -> None:
    """Raise DlmkError for a non-zero status."""
    if code != DLMK_OK:
        raise DlmkError(code, last_error())
