"""libdlmk.so loads, exports exactly what include/dlmk.h declares, and rejects
bad arguments before touching the GPU (no compute calls here)."""
import ctypes as C
import os
import re

import pytest

from dlm_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "dlmk.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dlmk_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for must in ("dlmk_kv_append", "dlmk_paged_decode_attention", "dlmk_copy_blocks",
                 "dlmk_swap_out", "dlmk_swap_in", "dlmk_cache_append_tokens"):
        assert must in syms


def test_library_exports_every_declared_symbol(dlmk):
    missing = [s for s in declared_symbols() if not hasattr(dlmk, s)]
    assert not missing, missing


def test_python_binding_covers_the_header():
    assert sorted(_lib.SIGNATURES) == declared_symbols()


def test_exported_symbols_are_c_linkage():
    out = os.popen(f"nm -D --defined-only {_lib.LIB_PATH}").read()
    exported = set(re.findall(r"\b(dlmk_[a-z0-9_]+)\b", out))
    assert set(declared_symbols()) <= exported


def test_abi_version(dlmk):
    assert dlmk.dlmk_abi_version() == 1


def test_argument_errors_before_any_launch(dlmk):
    # Negative sizes and null pointers fail on the host with DLMK_ERR_INVALID_ARG.
    rc = dlmk.dlmk_kv_append(None, None, None, None, None, None, -1, 8, 128, 16, 10, 1)
    assert rc == _lib.DLMK_ERR_INVALID_ARG
    assert "bad sizes" in _lib.last_error()
    rc = dlmk.dlmk_kv_append(None, None, None, None, None, None, 4, 8, 128, 16, 10, 1)
    assert rc == _lib.DLMK_ERR_INVALID_ARG
    A = 4096  # a stand-in device address, 16-byte aligned (never dereferenced)
    rc = dlmk.dlmk_kv_append(None, A, A, A, A, A, 4, 8, 12, 16, 10, 1)  # 12*2 % 16 != 0
    assert rc == _lib.DLMK_ERR_UNSUPPORTED
    rc = dlmk.dlmk_kv_append(None, A, A, A + 4, A, A, 4, 8, 128, 16, 10, 1)  # k_src 4 bytes off
    assert rc == _lib.DLMK_ERR_INVALID_ARG and "aligned" in _lib.last_error()
    rc = dlmk.dlmk_copy_blocks(None, A + 8, A, A, 3, 64, 10)  # k_pool 8 bytes off
    assert rc == _lib.DLMK_ERR_INVALID_ARG and "aligned" in _lib.last_error()
    # Zero tokens is a successful no-op.
    assert dlmk.dlmk_kv_append(None, None, None, None, None, None, 0, 8, 128, 16, 10, 1) == 0
    rc = dlmk.dlmk_copy_blocks(None, 1, 1, 1, 3, 100, 10)  # block_bytes not multiple of 16
    assert rc == _lib.DLMK_ERR_INVALID_ARG
    rc = dlmk.dlmk_paged_decode_attention(None, A, 1, A, A, A, 1, A, A, 4, 1, 32, 6, 128, 16,
                                          8, 100, 0.1, None, 0)  # 32 % 6 != 0
    assert rc == _lib.DLMK_ERR_INVALID_ARG
    rc = dlmk.dlmk_paged_decode_attention(None, A, 1, A + 2, A, A, 1, A, A, 4, 1, 32, 8, 128, 16,
                                          8, 100, 0.1, None, 0)  # q 2 bytes off 16
    assert rc == _lib.DLMK_ERR_INVALID_ARG and "aligned" in _lib.last_error()
    rc = dlmk.dlmk_paged_decode_attention(None, A, 1, A, A, A, 1, A, A, 4, 1, 32, 8, 128, 32,
                                          8, 100, 0.1, None, 0)  # block_size 32
    assert rc == _lib.DLMK_ERR_UNSUPPORTED
    rc = dlmk.dlmk_paged_decode_attention(None, A, 1, A, A, A, 1, A, A, 4, 1, 32, 8, 128, 16,
                                          64, 100, 0.1, None, 0)  # needs workspace
    assert rc == _lib.DLMK_ERR_WORKSPACE
    rc = dlmk.dlmk_swap_out(None, 1, 1, 1, 1, 2, 64, 10, 1, 100)  # staging 100 < 256
    assert rc == _lib.DLMK_ERR_WORKSPACE


def test_workspace_size_formula(dlmk):
    # One partition (<= 64 tokens, the smallest any kernel uses) needs no workspace.
    assert dlmk.dlmk_paged_attention_workspace_size(64, 1, 32, 128, 16, 4) == 0
    # 4096-token tables: 64 partitions of (d + 2) floats per query row.
    rows, parts = 64 * 32, 64
    o = rows * parts * 128 * 4
    assert dlmk.dlmk_paged_attention_workspace_size(64, 1, 32, 128, 16, 256) == \
        (o + 255) // 256 * 256 + rows * parts * 8


def test_alloc_pinned_error_paths(dlmk):
    # PinnedBuffer::with_len(0) is DlmError::HostAlloc (src/memory/pinned.rs:59-66):
    # here DLMK_ERR_INVALID_ARG, *ptr NULL and a last-error string.  No GPU call
    # is made on these paths.
    p = C.c_void_p(1234)
    assert dlmk.dlmk_alloc_pinned(C.byref(p), 0) == _lib.DLMK_ERR_INVALID_ARG
    assert p.value is None
    assert "zero bytes" in _lib.last_error()
    assert dlmk.dlmk_alloc_pinned(None, 16) == _lib.DLMK_ERR_INVALID_ARG
    assert "null out pointer" in _lib.last_error()
    assert dlmk.dlmk_alloc_pinned(C.byref(p), 2**64 - 1) == _lib.DLMK_ERR_INVALID_ARG
    assert p.value is None
    assert dlmk.dlmk_free_pinned(None) == 0
    from dlm_amd import ops
    with pytest.raises(_lib.DlmkError):
        ops.PinnedBuffer(0)
