"""Prefix sharing in the block-table books: dlmk_cache_fork_sequence_shared,
dlmk_cache_append_tokens_cow, dlmk_cache_block_refcount.

dlm's prefix cache clones a whole KvSnapshot (src/batching.rs:32-72,
src/forward/orchestrator.rs:73-105); the paged form shares the prefix's blocks
by reference count and copies only a partially-filled last block, when a
sequence is about to write into it.  No reference code does this, so it is
pinned by invariants:
  * every block's count equals the number of tables listing it, the free list
    holds exactly the unlisted blocks, once each;
  * a byte-level model of the pool (NumPy, the copies the books hand out applied
    as dlmk_copy_blocks would) reads every sequence back as exactly its own
    token history, whatever the other sequences appended or truncated.
"""
import numpy as np
import pytest

from dlm_amd import DlmkError, KvCacheConfig, KvCacheExhausted, PagedKvCache

BS = 16
CFG = KvCacheConfig(num_layers=1, num_kv_heads=1, head_dim=8, block_size=BS)


def test_fork_shared_lists_the_same_blocks_and_counts_them():
    c = PagedKvCache(CFG, 10)
    c.append_tokens(1, 40)  # blocks 0 1 2, the last holding 8 tokens
    c.fork_sequence_shared(1, 2)
    assert c.block_table(2) == c.block_table(1) == [0, 1, 2]
    assert [c.block_refcount(b) for b in range(4)] == [2, 2, 2, 0]
    assert c.sequence_len(2) == 40
    assert c.stats().used_blocks == 3  # nothing allocated


def test_append_into_shared_partial_tail_needs_cow():
    c = PagedKvCache(CFG, 10)
    c.append_tokens(1, 40)
    c.fork_sequence_shared(1, 2)
    with pytest.raises(DlmkError):
        c.append_tokens(2, 1)
    assert c.sequence_len(2) == 40 and c.block_table(2) == [0, 1, 2]  # unchanged
    pair = c.append_tokens_cow(2, 5)
    assert pair.tolist() == [[2, 3]]  # shared tail 2 -> private 3 (next low id)
    assert c.block_table(2) == [0, 1, 3] and c.sequence_len(2) == 45
    assert [c.block_refcount(b) for b in range(4)] == [2, 2, 1, 1]
    # The source's tail is private again: plain append works and copies nothing.
    c.append_tokens(1, 8)
    assert c.block_table(1) == [0, 1, 2] and c.sequence_len(1) == 48
    assert c.append_tokens_cow(1, 1).size == 0 and c.block_table(1) == [0, 1, 2, 4]


def test_full_block_boundary_shares_without_copies():
    c = PagedKvCache(CFG, 10)
    c.append_tokens(1, 32)  # two full blocks
    c.fork_sequence_shared(1, 2)
    assert c.append_tokens_cow(2, 3).size == 0  # nothing to copy: writes go to a new block
    assert c.block_table(2) == [0, 1, 2]
    c.append_tokens(1, 3)  # plain append: tail is full, so it is not shared
    assert c.block_table(1) == [0, 1, 3]


def test_free_keeps_shared_blocks_until_the_last_table_goes():
    c = PagedKvCache(CFG, 6)
    c.append_tokens(1, 40)
    c.fork_sequence_shared(1, 2)
    c.append_tokens_cow(2, 10)  # 2 -> private 3, then 4 for the overflow
    assert c.block_table(2) == [0, 1, 3, 4] and c.free_list() == [5]
    c.free_sequence(1)
    # 0 and 1 are still listed by sequence 2; 2 was only sequence 1's by now.
    assert c.free_list() == [5, 2]
    c.free_sequence(2)
    assert c.free_list() == [5, 2, 0, 1, 3, 4]  # table order as they reach zero


def test_cow_is_atomic_on_exhaustion():
    c = PagedKvCache(CFG, 3)
    c.append_tokens(1, 40)  # all 3 blocks
    c.fork_sequence_shared(1, 2)
    with pytest.raises(KvCacheExhausted) as e:
        c.append_tokens_cow(2, 1)
    assert (e.value.requested, e.value.free, e.value.total) == (1, 0, 3)
    assert c.block_table(2) == [0, 1, 2] and c.sequence_len(2) == 40
    assert [c.block_refcount(b) for b in range(3)] == [2, 2, 2]


def test_truncate_into_a_shared_block_then_cow():
    c = PagedKvCache(CFG, 10)
    c.append_tokens(1, 48)  # three full blocks
    c.fork_sequence_shared(1, 2)
    c.truncate_sequence(2, 20)  # drops block 2 from sequence 2; block 1 now its partial tail
    assert c.block_table(2) == [0, 1] and c.block_refcount(2) == 1
    with pytest.raises(DlmkError):
        c.append_tokens(2, 1)
    assert c.append_tokens_cow(2, 1).tolist() == [[1, 3]]


class PoolModel:
    """Device pool stand-in: slot -> token label, copies applied like dlmk_copy_blocks."""

    def __init__(self, nb):
        self.slots = np.full(nb * BS, -1, np.int64)

    def copy(self, pairs):
        for src, dst in pairs:
            self.slots[dst * BS:(dst + 1) * BS] = self.slots[src * BS:(src + 1) * BS]

    def write(self, cache, seq, start, labels):
        sl = cache.slot_mapping(seq, start, len(labels))
        self.slots[sl] = labels

    def read(self, cache, seq):
        n = cache.sequence_len(seq)
        return self.slots[cache.slot_mapping(seq, 0, n)] if n else np.zeros(0, np.int64)


def check_books(cache, nb, live):
    tables = {s: cache.block_table(s) for s in live}
    count = np.zeros(nb, np.int64)
    for t in tables.values():
        for b in t:
            count[b] += 1
    refs = np.array([cache.block_refcount(b) for b in range(nb)])
    assert np.array_equal(refs, count), "refcounts differ from the tables"
    free = cache.free_list()
    assert len(free) == len(set(free)), "free list holds a block twice"
    assert set(free) == {b for b in range(nb) if count[b] == 0}
    assert cache.stats().used_blocks == nb - len(free)
    for s, t in tables.items():
        assert len(t) == -(-cache.sequence_len(s) // BS)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_random_sharing_storm_keeps_every_history_private(seed):
    rng = np.random.default_rng(seed)
    nb = 64
    cache = PagedKvCache(CFG, nb)
    pool = PoolModel(nb)
    hist = {}  # seq -> list of labels (its logical history)
    label = 0
    next_seq = 0
    for step in range(600):
        op = rng.choice(["new", "append", "fork_shared", "fork_copy", "truncate", "free"],
                        p=[0.1, 0.4, 0.15, 0.05, 0.15, 0.15])
        live = list(hist)
        if op == "new" or not live:
            s, next_seq = next_seq, next_seq + 1
            n = int(rng.integers(1, 40))
            try:
                cache.append_tokens_cow(s, n)
            except KvCacheExhausted:
                continue
            labs = list(range(label, label + n))
            label += n
            hist[s] = labs
            pool.write(cache, s, 0, labs)
        elif op == "append":
            s = int(rng.choice(live))
            n = int(rng.integers(1, 20))
            start = cache.sequence_len(s)
            try:
                pair = cache.append_tokens_cow(s, n)
            except KvCacheExhausted:
                continue
            pool.copy(pair)
            labs = list(range(label, label + n))
            label += n
            hist[s] += labs
            pool.write(cache, s, start, labs)
        elif op == "fork_shared":
            src, dst = int(rng.choice(live)), next_seq
            next_seq += 1
            cache.fork_sequence_shared(src, dst)
            hist[dst] = list(hist[src])
        elif op == "fork_copy":
            src, dst = int(rng.choice(live)), next_seq
            next_seq += 1
            try:
                pairs = cache.fork_sequence(src, dst)
            except KvCacheExhausted:
                continue
            pool.copy(pairs)
            hist[dst] = list(hist[src])
        elif op == "truncate":
            s = int(rng.choice(live))
            new_len = int(rng.integers(0, len(hist[s]) + 1))
            cache.truncate_sequence(s, new_len)
            hist[s] = hist[s][:new_len]
        else:
            s = int(rng.choice(live))
            cache.free_sequence(s)
            del hist[s]
        check_books(cache, nb, list(hist))
        for s, labs in hist.items():
            assert pool.read(cache, s).tolist() == labs, f"step {step}: sequence {s} corrupted"
