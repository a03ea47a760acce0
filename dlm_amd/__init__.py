"""dlm_amd -- MI355X (gfx950) paged KV-cache hot path for dlm.

Drop-in for vedantnimbarte/dlm's KV path: the block-table store
(src/cache/paged.rs), paged append, paged GQA decode attention, block copy and
swap gather/scatter, implemented as hand-written HIP kernels behind the C ABI
in include/dlmk.h (libdlmk.so).  This package is the Python host mirror of
that ABI.
"""
from ._lib import DlmkError, LIB_PATH
from .cache import KvCacheConfig, KvCacheExhausted, KvCacheStats, PagedKvCache, UnknownSequence

__all__ = ["DlmkError", "LIB_PATH", "KvCacheConfig", "KvCacheExhausted", "KvCacheStats",
           "PagedKvCache", "UnknownSequence"]
