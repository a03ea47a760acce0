"""Block-table KV store: the Python face of dlm's ``PagedKvCache``.

Mirrors ``src/cache/paged.rs`` (``KvCacheConfig`` :30-71, ``KvCacheStats``
:83-102, ``PagedKvCache`` :106-227) method for method, with the same error
(``KvCacheExhausted{requested, free, total}``, ``src/error.rs:70-75``) and the
same atomicity.  The books themselves live in libdlmk.so (C++), so a Rust or C
caller sees exactly the state these methods report.

Extensions needed by the paged hot path: a caller-chosen free order
(``with_free_order``), ``truncate_sequence`` (speculative rollback),
``fork_sequence`` (prefix sharing by block copy), and the device-side views
``slot_mapping`` / ``block_tables``.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Iterable, List, Optional, Sequence

import numpy as np

from ._lib import (DLMK_ERR_KV_EXHAUSTED, DLMK_ERR_UNKNOWN_SEQ, DlmkError, KvCacheConfigC,
                   KvCacheStatsC, KvExhaustedC, check, last_error, lib)


class KvCacheExhausted(DlmkError):
    """``DlmError::KvCacheExhausted``: the pool cannot supply ``requested`` blocks."""

    def __init__(self, requested: int, free: int, total: int):
        super().__init__(DLMK_ERR_KV_EXHAUSTED,
                         f"KV cache pool exhausted: need {requested} more block(s), "
                         f"{free} free of {total}")
        self.requested, self.free, self.total = requested, free, total


class UnknownSequence(DlmkError, KeyError):
    pass


@dataclass(frozen=True)
class KvCacheConfig:
    """Geometry of the KV cache (paged.rs:30-71)."""

    num_layers: int
    num_kv_heads: int
    head_dim: int
    block_size: int = 16

    def _c(self) -> KvCacheConfigC:
        return KvCacheConfigC(self.num_layers, self.num_kv_heads, self.head_dim,
                              max(self.block_size, 1))

    def bytes_per_token(self) -> int:
        """2 (K,V) x kv heads x head_dim x 2 bytes x layers (paged.rs:52-58)."""
        return lib().dlmk_bytes_per_token(C.byref(self._c()))

    def bytes_per_block(self) -> int:
        return lib().dlmk_bytes_per_block(C.byref(self._c()))

    def blocks_for_tokens(self, tokens: int) -> int:
        return lib().dlmk_blocks_for_tokens(C.byref(self._c()), tokens)


@dataclass(frozen=True)
class KvCacheStats:
    """KvCacheStats (paged.rs:83-102)."""

    total_blocks: int
    used_blocks: int
    free_blocks: int
    num_sequences: int
    used_tokens: int
    capacity_tokens: int
    bytes_per_block: int

    def utilization(self) -> float:
        return 0.0 if self.total_blocks == 0 else self.used_blocks / self.total_blocks


class PagedKvCache:
    """A block-paged KV cache over a fixed pool of physical blocks."""

    def __init__(self, config: KvCacheConfig, total_blocks: int):
        self._init(config, lib().dlmk_cache_new(C.byref(config._c()), total_blocks))

    def _init(self, config: KvCacheConfig, handle) -> None:
        if not handle:
            raise DlmkError(-1, last_error() or "dlmk_cache_new failed")
        self._config = config
        self._h = handle

    @classmethod
    def with_budget(cls, config: KvCacheConfig, kv_budget_bytes: int) -> "PagedKvCache":
        """Size the pool to fit a KV byte budget (paged.rs:130-134)."""
        self = cls.__new__(cls)
        self._init(config, lib().dlmk_cache_with_budget(C.byref(config._c()), kv_budget_bytes))
        return self

    @classmethod
    def with_free_order(cls, config: KvCacheConfig, order: Sequence[int]) -> "PagedKvCache":
        """A pool of len(order) blocks handed out in the given order."""
        arr = np.ascontiguousarray(order, dtype=np.uint32)
        self = cls.__new__(cls)
        self._init(config, lib().dlmk_cache_new_with_free_order(
            C.byref(config._c()), arr.ctypes.data_as(C.c_void_p), len(arr)))
        return self

    @classmethod
    def with_seeded_shuffle(cls, config: KvCacheConfig, total_blocks: int,
                            seed: int) -> "PagedKvCache":
        """A pool whose free order is a seeded permutation (non-contiguous tables)."""
        order = np.random.default_rng(seed).permutation(total_blocks)
        return cls.with_free_order(config, order)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            lib().dlmk_cache_destroy(h)
            self._h = None

    # -- geometry / counters (paged.rs:137-160)
    def config(self) -> KvCacheConfig:
        return self._config

    def stats(self) -> KvCacheStats:
        s = KvCacheStatsC()
        lib().dlmk_cache_stats(self._h, C.byref(s))
        return KvCacheStats(s.total_blocks, s.used_blocks, s.free_blocks, s.num_sequences,
                            s.used_tokens, s.capacity_tokens, s.bytes_per_block)

    def total_blocks(self) -> int:
        return self.stats().total_blocks

    def free_blocks(self) -> int:
        return self.stats().free_blocks

    def used_blocks(self) -> int:
        return self.stats().used_blocks

    def capacity_tokens(self) -> int:
        return self.stats().capacity_tokens

    def num_sequences(self) -> int:
        return lib().dlmk_cache_num_sequences(self._h)

    # -- mutation (paged.rs:164-197 + extensions)
    def append_tokens(self, seq_id: int, n: int) -> None:
        """Append n tokens, allocating blocks lazily; atomic on exhaustion."""
        err = KvExhaustedC()
        rc = lib().dlmk_cache_append_tokens(self._h, seq_id, n, C.byref(err))
        if rc == DLMK_ERR_KV_EXHAUSTED:
            raise KvCacheExhausted(err.requested, err.free, err.total)
        check(rc)

    def free_sequence(self, seq_id: int) -> None:
        lib().dlmk_cache_free_sequence(self._h, seq_id)

    def truncate_sequence(self, seq_id: int, new_len: int) -> None:
        """Roll back to new_len tokens; whole freed blocks go back last-first."""
        rc = lib().dlmk_cache_truncate_sequence(self._h, seq_id, new_len)
        if rc == DLMK_ERR_UNKNOWN_SEQ:
            raise UnknownSequence(rc, last_error())
        check(rc)

    def fork_sequence(self, src_seq: int, dst_seq: int) -> np.ndarray:
        """New sequence dst with private copies of src's blocks.

        Returns the int32 [n, 2] (src_block, dst_block) pairs to hand to
        ``ops.copy_blocks``."""
        table = self.block_table(src_seq)
        if table is None:
            raise UnknownSequence(DLMK_ERR_UNKNOWN_SEQ, f"unknown sequence {src_seq}")
        cap = max(len(table), 1)
        pairs = np.zeros((cap, 2), np.int32)
        n = C.c_uint32(0)
        err = KvExhaustedC()
        rc = lib().dlmk_cache_fork_sequence(self._h, src_seq, dst_seq,
                                            pairs.ctypes.data_as(C.c_void_p), cap, C.byref(n),
                                            C.byref(err))
        if rc == DLMK_ERR_KV_EXHAUSTED:
            raise KvCacheExhausted(err.requested, err.free, err.total)
        check(rc)
        return pairs[: n.value]

    def fork_sequence_shared(self, src_seq: int, dst_seq: int) -> None:
        """New sequence dst listing src's blocks (reference-counted, no copy):
        the paged prefix cache.  Append to either with ``append_tokens_cow``."""
        rc = lib().dlmk_cache_fork_sequence_shared(self._h, src_seq, dst_seq)
        if rc == DLMK_ERR_UNKNOWN_SEQ:
            raise UnknownSequence(rc, last_error())
        check(rc)

    def append_tokens_cow(self, seq_id: int, n: int) -> np.ndarray:
        """append_tokens that first gives the sequence a private copy of a shared
        partially-filled last block.  Returns the int32 [0 or 1, 2] (shared,
        private) pair to hand to ``ops.copy_blocks`` before writing the tokens."""
        pair = np.zeros((1, 2), np.int32)
        n_pairs = C.c_uint32(0)
        err = KvExhaustedC()
        rc = lib().dlmk_cache_append_tokens_cow(self._h, seq_id, n,
                                                pair.ctypes.data_as(C.c_void_p),
                                                C.byref(n_pairs), C.byref(err))
        if rc == DLMK_ERR_KV_EXHAUSTED:
            raise KvCacheExhausted(err.requested, err.free, err.total)
        check(rc)
        return pair[: n_pairs.value]

    def block_refcount(self, block: int) -> int:
        """Number of block tables listing `block` (0 when free)."""
        return lib().dlmk_cache_block_refcount(self._h, block)

    # -- queries (paged.rs:200-207)
    def sequence_len(self, seq_id: int) -> int:
        return lib().dlmk_cache_sequence_len(self._h, seq_id)

    def block_table(self, seq_id: int) -> Optional[List[int]]:
        n = lib().dlmk_cache_block_table(self._h, seq_id, None, 0)
        if n < 0:
            return None
        out = np.zeros(max(n, 1), np.uint32)
        lib().dlmk_cache_block_table(self._h, seq_id, out.ctypes.data_as(C.c_void_p), n)
        return out[:n].tolist()

    def free_list(self) -> List[int]:
        """The free stack bottom-to-top (the last entry is handed out next)."""
        n = lib().dlmk_cache_free_list(self._h, None, 0)
        out = np.zeros(max(n, 1), np.uint32)
        lib().dlmk_cache_free_list(self._h, out.ctypes.data_as(C.c_void_p), n)
        return out[:n].tolist()

    # -- device-side views
    def slot_mapping(self, seq_id: int, start_pos: int, n: int) -> np.ndarray:
        """int64 slots (block * block_size + offset) of tokens [start_pos, start_pos+n)."""
        out = np.zeros(max(n, 1), np.int64)
        rc = lib().dlmk_cache_slot_mapping(self._h, seq_id, start_pos, n,
                                           out.ctypes.data_as(C.c_void_p))
        if rc == DLMK_ERR_UNKNOWN_SEQ:
            raise UnknownSequence(rc, last_error())
        check(rc)
        return out[:n]

    def block_tables(self, seq_ids: Iterable[int], max_blocks: int):
        """(int32 [n, max_blocks] tables padded with 0, int32 [n] lengths)."""
        ids = np.ascontiguousarray(list(seq_ids), dtype=np.uint64)
        tables = np.zeros((max(len(ids), 1), max_blocks), np.int32)
        lens = np.zeros(max(len(ids), 1), np.int32)
        check(lib().dlmk_cache_fill_block_tables(
            self._h, ids.ctypes.data_as(C.c_void_p), len(ids), max_blocks,
            tables.ctypes.data_as(C.c_void_p), lens.ctypes.data_as(C.c_void_p)))
        return tables[: len(ids)], lens[: len(ids)]
