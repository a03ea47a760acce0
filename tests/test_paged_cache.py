"""Block-table store: the reference's known answers, run against both the
oracle restatement and the product (libdlmk.so host bookkeeping), plus
seeded op-sequence parity between the two and pool invariants.

Pins: src/cache/paged.rs:244-335 (tests/golden/reference_known_answers.json)
and tests/phase1.rs:817-845 (budget reserved per decoded token).
"""
import json
import os

import numpy as np
import pytest

from dlm_amd import KvCacheConfig, KvCacheExhausted, PagedKvCache, UnknownSequence

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                   "reference_known_answers.json")))


class OracleAdapter:
    """OracleCache behind the product's method names."""

    def __init__(self, oracle, cfg, total_blocks=None, budget=None, free_order=None):
        self.o = oracle
        c = oracle.CacheConfig(cfg.num_layers, cfg.num_kv_heads, cfg.head_dim, cfg.block_size)
        self.c = oracle.OracleCache(c, total_blocks, budget=budget, free_order=free_order)

    def append_tokens(self, s, n):
        try:
            self.c.append_tokens(s, n)
        except self.o.Exhausted as e:
            raise KvCacheExhausted(e.requested, e.free, e.total)

    def __getattr__(self, name):
        return getattr(self.c, name)

    def fork_sequence(self, s, d):
        try:
            return self.c.fork_sequence(s, d)
        except self.o.Exhausted as e:
            raise KvCacheExhausted(e.requested, e.free, e.total)


def used_tokens(c):
    return c.used_tokens() if isinstance(c, OracleAdapter) else c.stats().used_tokens


@pytest.fixture(params=["oracle", "product"])
def make(request, oracle):
    def _make(cfg, total_blocks=None, budget=None, free_order=None):
        if request.param == "oracle":
            return OracleAdapter(oracle, cfg, total_blocks, budget, free_order)
        if free_order is not None:
            return PagedKvCache.with_free_order(cfg, free_order)
        if budget is not None:
            return PagedKvCache.with_budget(cfg, budget)
        return PagedKvCache(cfg, total_blocks)
    return _make


def cfg_small():
    g = GOLD["block_sizing_math"]["config"]
    return KvCacheConfig(g["num_layers"], g["num_kv_heads"], g["head_dim"], g["block_size"])


def test_block_sizing_math(oracle):
    g = GOLD["block_sizing_math"]
    c = cfg_small()
    oc = oracle.CacheConfig(4, 2, 8, 16)
    assert c.bytes_per_token() == g["bytes_per_token"] == oracle.bytes_per_token(oc)
    assert c.bytes_per_block() == g["bytes_per_block"] == oracle.bytes_per_block(oc)
    for tokens, blocks in g["blocks_for_tokens"]:
        assert c.blocks_for_tokens(tokens) == blocks == oracle.blocks_for_tokens(oc, tokens)


def test_append_allocates_blocks_lazily(make):
    g = GOLD["append_allocates_blocks_lazily"]
    cache = make(cfg_small(), g["total_blocks"])
    for seq, n, table_len, used in g["steps"]:
        cache.append_tokens(seq, n)
        assert len(cache.block_table(seq)) == table_len
        if used is not None:
            assert cache.used_blocks() == used
    assert cache.sequence_len(1) == g["final_len"]


def test_free_returns_blocks_to_pool_without_fragmentation(make):
    g = GOLD["free_returns_blocks_to_pool_without_fragmentation"]
    cache = make(cfg_small(), g["total_blocks"])
    cache.append_tokens(*g["append"])
    assert cache.free_blocks() == g["free_after_append"]
    cache.free_sequence(g["append"][0])
    assert cache.free_blocks() == g["free_after_free"]
    assert cache.num_sequences() == 0
    cache.append_tokens(*g["reuse"])
    assert cache.used_blocks() == g["used_after_reuse"]


def test_exhaustion_is_atomic_and_reported(make):
    g = GOLD["exhaustion_is_atomic_and_reported"]
    cache = make(cfg_small(), g["total_blocks"])
    cache.append_tokens(*g["first"])
    with pytest.raises(KvCacheExhausted) as ei:
        cache.append_tokens(*g["second"])
    e = g["error"]
    assert (ei.value.requested, ei.value.free, ei.value.total) == (e["requested"], e["free"],
                                                                     e["total"])
    assert cache.sequence_len(1) == g["len_after"]
    assert len(cache.block_table(1)) == g["table_len_after"]


def test_budget_sizing_and_multi_sequence_sharing(make):
    g = GOLD["budget_sizing_and_multi_sequence_sharing"]
    c = cfg_small()
    cache = make(c, budget=c.bytes_per_block() * g["budget_blocks"])
    assert cache.total_blocks() == g["budget_blocks"]
    for s, n in g["appends"]:
        cache.append_tokens(s, n)
    assert cache.num_sequences() == g["num_sequences"]
    assert cache.used_blocks() == g["used_blocks"]
    assert cache.free_blocks() == g["free_blocks"]
    assert used_tokens(cache) == g["used_tokens"]
    assert cache.capacity_tokens() == g["capacity_tokens"]


def test_stats_utilization():
    g = GOLD["budget_sizing_and_multi_sequence_sharing"]
    c = cfg_small()
    cache = PagedKvCache.with_budget(c, c.bytes_per_block() * g["budget_blocks"])
    for s, n in g["appends"]:
        cache.append_tokens(s, n)
    st = cache.stats()
    assert abs(st.utilization() - g["utilization"]) < 1e-9
    assert st.bytes_per_block == c.bytes_per_block()


def test_budget_reserved_per_decoded_token(make):
    """ForwardOrchestrator::decode_token reserves 1 token per step (phase1.rs:817-845)."""
    g = GOLD["orchestrator_budget_then_append"]
    c = KvCacheConfig(**g["config"])
    cache = make(c, g["total_blocks"])
    for _ in range(g["tokens"]):
        cache.append_tokens(0, 1)
    assert cache.sequence_len(0) == g["sequence_len"]


def test_low_ids_first_and_lifo_reuse(make):
    """new() hands out 0,1,2,...; freed blocks are reused last-in first-out."""
    cache = make(cfg_small(), 8)
    cache.append_tokens(1, 48)
    assert cache.block_table(1) == [0, 1, 2]
    cache.append_tokens(2, 16)
    assert cache.block_table(2) == [3]
    cache.free_sequence(1)  # stack gets 0,1,2 on top, 2 on the very top
    cache.append_tokens(3, 32)
    assert cache.block_table(3) == [2, 1]


def test_unknown_sequence_queries(make):
    cache = make(cfg_small(), 4)
    assert cache.sequence_len(42) == 0
    assert cache.block_table(42) is None
    cache.free_sequence(42)  # no-op
    assert cache.free_blocks() == 4


def test_zero_token_append_creates_empty_sequence(make):
    cache = make(cfg_small(), 4)
    cache.append_tokens(5, 0)
    assert cache.block_table(5) == []
    assert cache.num_sequences() == 1


def test_free_order_injection(make):
    order = [5, 2, 7, 0, 1, 3, 6, 4]
    cache = make(cfg_small(), free_order=order)
    cache.append_tokens(1, 40)
    assert cache.block_table(1) == order[:3]


def test_free_order_must_be_permutation():
    from dlm_amd import DlmkError
    with pytest.raises(DlmkError):
        PagedKvCache.with_free_order(cfg_small(), [0, 0, 1])


def test_truncate_then_reappend_restores_table(make):
    cache = make(cfg_small(), 16)
    cache.append_tokens(1, 70)  # 5 blocks
    before = cache.block_table(1)
    cache.truncate_sequence(1, 33)  # keep 3 blocks
    assert cache.sequence_len(1) == 33
    assert cache.block_table(1) == before[:3]
    assert cache.free_blocks() == 16 - 3
    cache.append_tokens(1, 37)
    assert cache.block_table(1) == before
    cache.truncate_sequence(1, 100)  # no-op when not shorter
    assert cache.sequence_len(1) == 70


def test_truncate_unknown_sequence(make, oracle):
    cache = make(cfg_small(), 4)
    with pytest.raises((UnknownSequence, KeyError)):
        cache.truncate_sequence(9, 0)


def test_fork_copies_table_and_is_atomic(make):
    cache = make(cfg_small(), 6)
    cache.append_tokens(1, 40)  # 3 blocks
    pairs = cache.fork_sequence(1, 2)
    assert [int(p[0]) for p in pairs] == cache.block_table(1)
    assert [int(p[1]) for p in pairs] == cache.block_table(2)
    assert cache.sequence_len(2) == 40
    assert not set(cache.block_table(1)) & set(cache.block_table(2))
    with pytest.raises(KvCacheExhausted) as ei:
        cache.fork_sequence(1, 3)  # needs 3, 0 free
    assert (ei.value.requested, ei.value.free, ei.value.total) == (3, 0, 6)
    assert cache.block_table(3) is None


def test_slot_mapping_and_block_tables():
    cache = PagedKvCache.with_free_order(cfg_small(), [9, 3, 7, 1, 0, 2, 4, 5, 6, 8])
    cache.append_tokens(1, 20)
    cache.append_tokens(2, 3)
    slots = cache.slot_mapping(1, 14, 6)
    assert slots.tolist() == [9 * 16 + 14, 9 * 16 + 15, 3 * 16 + 0, 3 * 16 + 1, 3 * 16 + 2,
                              3 * 16 + 3]
    tables, lens = cache.block_tables([1, 2, 77], 4)
    assert tables.tolist() == [[9, 3, 0, 0], [7, 0, 0, 0], [0, 0, 0, 0]]
    assert lens.tolist() == [20, 3, 0]
    from dlm_amd import DlmkError
    with pytest.raises(DlmkError):
        cache.slot_mapping(1, 15, 6)  # beyond length
    with pytest.raises(DlmkError):
        cache.block_tables([1], 1)  # table longer than max_blocks


def _invariants(cache, total):
    owned = []
    for s in range(80):
        t = cache.block_table(s)
        if t is not None:
            owned += t
            assert len(t) == -(-cache.sequence_len(s) // 16)
    free = cache.free_list()
    assert len(owned) == len(set(owned)), "block owned twice"
    assert not set(owned) & set(free), "block both owned and free"
    assert sorted(owned + free) == list(range(total)), "free + owned != pool"


def _apply(cache, ops):
    outcomes = []
    for op, s, n in ops:
        try:
            if op == "append":
                cache.append_tokens(s, n)
                outcomes.append("ok")
            elif op == "free":
                cache.free_sequence(s)
                outcomes.append("ok")
            elif op == "truncate":
                if cache.block_table(s) is None:
                    outcomes.append("skip")
                else:
                    cache.truncate_sequence(s, cache.sequence_len(s) * n // 10)
                    outcomes.append("ok")
            elif op == "fork":
                if cache.block_table(s) is None or cache.block_table(s + 40) is not None:
                    outcomes.append("skip")
                else:
                    outcomes.append(np.asarray(cache.fork_sequence(s, s + 40)).tolist())
        except KvCacheExhausted as e:
            outcomes.append(("exhausted", e.requested, e.free, e.total))
    return outcomes


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_random_ops_product_matches_oracle(oracle, seed):
    """Seeded alloc/free/truncate/fork storm (config-3 style): identical books."""
    rng = np.random.default_rng(seed)
    total = 200
    order = rng.permutation(total)
    kinds = ["append", "append", "free", "truncate", "fork"]
    ops = [(kinds[rng.integers(0, 5)], int(rng.integers(0, 40)), int(rng.integers(0, 100)))
           for _ in range(800)]
    c = cfg_small()
    prod = PagedKvCache.with_free_order(c, order)
    orc = OracleAdapter(oracle, c, free_order=order)
    out_p, out_o = _apply(prod, ops), _apply(orc, ops)
    assert out_p == out_o
    assert any(isinstance(o, tuple) for o in out_p), "storm never hit exhaustion"
    assert prod.free_list() == orc.free_list()
    for s in range(80):
        assert prod.block_table(s) == orc.block_table(s)
        assert prod.sequence_len(s) == orc.sequence_len(s)
    _invariants(prod, total)
