"""End-to-end workflows of BASELINE.json configs 1, 3, 4 and 5 on the GPU.

Each test drives the product (PagedKvCache books + libdlmk kernels) and, in
lockstep, a host mirror of the pools maintained by the CPU oracle from the same
seeded inputs.  Pools must stay bit-identical to the mirror; attention must
match the oracle over the mirror within the stated tolerance.  The oracle runs
on reduced sizes where its cost would be minutes; size-independent properties
(books invariants, bit-exact pools, round trips) are checked at full size.
"""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from helpers import F16_ATOL, F16_RTOL, assert_close, to_dev

pytestmark = pytest.mark.gpu

HKV, D, BS = 8, 128, 16
X = 8  # f16 elements per 16-byte K chunk


def banner(msg):
    print(f"[gpu-test] {msg}", flush=True)


class Mirror:
    """Device pools + host mirror + books for one f16 layer."""

    def __init__(self, torch, cuda, oracle, num_blocks, seed, hq=32):
        from dlm_amd import KvCacheConfig, PagedKvCache, ops
        self.torch, self.cuda, self.oracle, self.ops = torch, cuda, oracle, ops
        self.hq = hq
        self.nb = num_blocks
        self.rng = np.random.default_rng(seed)
        self.cache = PagedKvCache.with_seeded_shuffle(KvCacheConfig(1, HKV, D, BS), num_blocks,
                                                      seed)
        # Garbage-filled pools (finite f16 bit patterns): a slot read before it
        # was written would show up in the comparison.
        def garbage(shape):
            bits = self.rng.integers(0, 2**16, shape, dtype=np.uint16)
            bits[(bits & 0x7C00) == 0x7C00] = 0
            return bits.view(np.float16)
        self.kh = garbage((num_blocks, HKV, D // X, BS, X))
        self.vh = garbage((num_blocks, HKV, D, BS))
        self.kd = to_dev(torch, self.kh, cuda)
        self.vd = to_dev(torch, self.vh, cuda)
        self.block_bytes = HKV * BS * D * 2

    def append(self, seq_tokens, sigma=0.5, outlier_frac=0.0):
        """seq_tokens: list of (seq_id, n).  Books first (atomic), then one kernel."""
        slots = []
        for s, n in seq_tokens:
            start = self.cache.sequence_len(s)
            self.cache.append_tokens(s, n)
            slots.append(self.cache.slot_mapping(s, start, n))
        slots = np.concatenate(slots) if slots else np.zeros(0, np.int64)
        n = len(slots)
        k = (self.rng.standard_normal((n, HKV, D)) * sigma).astype(np.float32)
        if outlier_frac:
            rows = self.rng.random(n) < outlier_frac
            k[rows] *= 8
        k = k.astype(np.float16)
        v = (self.rng.standard_normal((n, HKV, D)) * sigma).astype(np.float16)
        t = self.torch
        self.ops.kv_append(self.kd, self.vd, to_dev(t, k, self.cuda), to_dev(t, v, self.cuda),
                           to_dev(t, slots, self.cuda), num_kv_heads=HKV, head_dim=D)
        self.oracle.paged_append(self.kh, self.vh, k, v, slots, HKV, D, BS)

    def append_cow(self, seq_tokens, sigma=0.5):
        """append with copy-on-write of shared partial tails: books for every
        sequence, one block-copy launch for the copies they hand out, then the
        tokens (the copies run first on the stream)."""
        pairs, work = [], []
        for s, n in seq_tokens:
            start = self.cache.sequence_len(s)
            pairs.append(self.cache.append_tokens_cow(s, n))
            work.append((s, start, n))
        pairs = np.concatenate(pairs).astype(np.int32) if pairs else np.zeros((0, 2), np.int32)
        if len(pairs):
            self.ops.copy_blocks(self.kd, self.vd, to_dev(self.torch, pairs, self.cuda),
                                 self.block_bytes)
            self.oracle.copy_blocks(self.kh, self.vh, pairs, self.block_bytes)
        slots = np.concatenate([self.cache.slot_mapping(s, st, n) for s, st, n in work])
        n = len(slots)
        k = (self.rng.standard_normal((n, HKV, D)) * sigma).astype(np.float16)
        v = (self.rng.standard_normal((n, HKV, D)) * sigma).astype(np.float16)
        t = self.torch
        self.ops.kv_append(self.kd, self.vd, to_dev(t, k, self.cuda), to_dev(t, v, self.cuda),
                           to_dev(t, slots, self.cuda), num_kv_heads=HKV, head_dim=D)
        self.oracle.paged_append(self.kh, self.vh, k, v, slots, HKV, D, BS)
        return pairs

    def attention(self, seqs, nq=1, check=None, max_blocks=None):
        """Device attention for seqs; oracle check on the index subset `check`."""
        max_blocks = max_blocks or max(len(self.cache.block_table(s)) for s in seqs)
        tables, lens = self.cache.block_tables(seqs, max_blocks)
        q = (self.rng.standard_normal((len(seqs), nq, self.hq, D)) * 0.5).astype(np.float16)
        t = self.torch
        out = self.ops.paged_decode_attention(
            to_dev(t, q, self.cuda), self.kd, self.vd, to_dev(t, tables, self.cuda),
            to_dev(t, lens, self.cuda), num_kv_heads=HKV, out_dtype=t.float32)
        t.cuda.synchronize()
        out = out.cpu().numpy()
        idx = list(range(len(seqs))) if check is None else list(check)
        if idx:
            # The oracle's C call releases the GIL: sequences in parallel.
            groups = [idx[i::8] for i in range(min(8, len(idx)))]
            run = lambda g: self.oracle.paged_attention(
                q[g], self.kh, self.vh, tables[g], lens[g], nq, self.hq, HKV, D, BS,
                1.0 / np.sqrt(D))
            with ThreadPoolExecutor(len(groups)) as ex:
                refs = list(ex.map(run, groups))
            for g, ref in zip(groups, refs):
                assert_close(out[g], ref, F16_ATOL, F16_RTOL, "attention vs oracle")
        return out

    def assert_pools_equal(self, ids=None):
        self.torch.cuda.synchronize()
        if ids is None:
            assert np.array_equal(self.kd.cpu().numpy().view(np.uint16), self.kh.view(np.uint16))
            assert np.array_equal(self.vd.cpu().numpy().view(np.uint16), self.vh.view(np.uint16))
        else:
            idx = self.torch.as_tensor(np.asarray(ids), device=self.cuda).long()
            assert np.array_equal(self.kd[idx].cpu().numpy().view(np.uint16),
                                  self.kh[np.asarray(ids)].view(np.uint16))
            assert np.array_equal(self.vd[idx].cpu().numpy().view(np.uint16),
                                  self.vh[np.asarray(ids)].view(np.uint16))

    def assert_books_consistent(self, live):
        owned = []
        for s in live:
            t = self.cache.block_table(s)
            assert t is not None and len(t) == -(-self.cache.sequence_len(s) // BS)
            owned += t
        free = self.cache.free_list()
        assert len(set(owned)) == len(owned) and not set(owned) & set(free)
        assert sorted(owned + free) == list(range(self.nb))


@pytest.fixture(scope="module")
def torch_mod(cuda):
    import torch
    return torch


def test_config1_16_layer_prefill_then_decode(oracle, torch_mod, cuda):
    """BASELINE.json configs[0] as stated: Llama-3.2-1B KV (16 layers, 32 query
    heads, 8 kv heads, head_dim 64, f32), one sequence whose blocks come from a
    seeded-shuffled free list.  Each layer appends a 512-token prefill chunk,
    then 64 decode steps append 1 token per layer and attend with scale 1/8.
    Every layer of every step is compared with the oracle's attention() over
    the host mirror (1e-5), even steps through the fused decode step and odd
    steps as append + attention, and every layer's pools are bit-exact at the
    end (src/forward/cpu.rs:1126-1151, :765-795)."""
    from dlm_amd import KvCacheConfig, PagedKvCache, ops
    from helpers import F32_ATOL, F32_RTOL
    torch = torch_mod
    L, Hq, Hkv, d, prefill, steps = 16, 32, 8, 64, 512, 64
    banner(f"config-1 workflow: {L} layers, {prefill} prefill + {steps} decode steps")
    nb, max_blocks = 64, 40
    rng = np.random.default_rng(1)
    cache = PagedKvCache.with_seeded_shuffle(KvCacheConfig(L, Hkv, d, BS), nb, seed=1)
    kh = [(rng.standard_normal((nb, Hkv, d // 4, BS, 4))).astype(np.float32) for _ in range(L)]
    vh = [(rng.standard_normal((nb, Hkv, d, BS))).astype(np.float32) for _ in range(L)]
    kd = [to_dev(torch, a, cuda) for a in kh]
    vd = [to_dev(torch, a, cuda) for a in vh]
    scale = np.float32(1.0) / np.sqrt(np.float32(d))
    dv = lambda a: to_dev(torch, a, cuda)
    ws = ops.alloc_workspace(ops.attention_workspace_bytes(1, 1, Hq, d, max_blocks), cuda)

    cache.append_tokens(0, prefill)
    slots = cache.slot_mapping(0, 0, prefill)
    for layer in range(L):
        k = rng.standard_normal((prefill, Hkv, d)).astype(np.float32)
        v = rng.standard_normal((prefill, Hkv, d)).astype(np.float32)
        ops.kv_append(kd[layer], vd[layer], dv(k), dv(v), dv(slots), num_kv_heads=Hkv, head_dim=d)
        oracle.paged_append(kh[layer], vh[layer], k, v, slots, Hkv, d, BS)
    worst = 0.0
    for step in range(steps):
        cache.append_tokens(0, 1)
        pos = prefill + step
        slot = cache.slot_mapping(0, pos, 1)
        tables, lens = cache.block_tables([0], max_blocks)
        assert lens[0] == pos + 1
        t_d, l_d = dv(tables), dv(lens)
        qs, outs = [], []
        for layer in range(L):
            k = rng.standard_normal((1, Hkv, d)).astype(np.float32)
            v = rng.standard_normal((1, Hkv, d)).astype(np.float32)
            q = rng.standard_normal((1, 1, Hq, d)).astype(np.float32)
            if step % 2 == 0:
                out = ops.paged_decode_step(dv(q), dv(k), dv(v), kd[layer], vd[layer], t_d, l_d,
                                            num_kv_heads=Hkv, scale=float(scale),
                                            out_dtype=torch.float32, workspace=ws)
            else:
                ops.kv_append(kd[layer], vd[layer], dv(k), dv(v), dv(slot), num_kv_heads=Hkv,
                              head_dim=d)
                out = ops.paged_decode_attention(dv(q), kd[layer], vd[layer], t_d, l_d,
                                                 num_kv_heads=Hkv, scale=float(scale),
                                                 out_dtype=torch.float32, workspace=ws)
            oracle.paged_append(kh[layer], vh[layer], k, v, slot, Hkv, d, BS)
            qs.append(q)
            outs.append(out)
        torch.cuda.synchronize()
        for layer in range(L):
            ref = oracle.paged_attention(qs[layer], kh[layer], vh[layer], tables, lens, 1, Hq, Hkv,
                                         d, BS, scale)
            got = outs[layer].cpu().numpy()
            assert_close(got, ref, F32_ATOL, F32_RTOL, f"config-1 step {step} layer {layer}")
            worst = max(worst, float(np.abs(got - ref).max()))
        if step % 16 == 0:
            banner(f"config-1 step {step}: ctx {pos + 1}, worst abs err so far {worst:.2e}")
    torch.cuda.synchronize()
    for layer in range(L):
        assert np.array_equal(kd[layer].cpu().numpy().view(np.uint32), kh[layer].view(np.uint32))
        assert np.array_equal(vd[layer].cpu().numpy().view(np.uint32), vh[layer].view(np.uint32))
    # The single table is shared by all 16 layers and came off the shuffled list.
    table = cache.block_table(0)
    assert len(table) == -(-(prefill + steps) // BS) and table != sorted(table)


@pytest.mark.parametrize("full", [False, True])
def test_config3_continuous_batching(oracle, torch_mod, cuda, full):
    """Decode sequences + chunked-prefill sequences share one free list; sequences
    finish and are replaced; every step is checked against the oracle: all
    sequences at reduced sizes; at config-3 sizes (48 decode at U[256, 8192] +
    4 x 512-token chunks per step, all 200 steps) one sequence per step in
    rotation plus a random second one, and every sequence on every 50th step.
    Books are invariant after every step and the pools bit-exact at the end."""
    n_dec, lo, hi, n_pref, chunk, steps, pool = (
        (48, 256, 8192, 4, 512, 200, 36000) if full else (12, 64, 1024, 2, 128, 30, 4000))
    banner(f"config-3 workflow full={full} steps={steps}")
    m = Mirror(torch_mod, cuda, oracle, pool, seed=3 + full)
    rng = np.random.default_rng(33 + full)
    next_id = 0
    decode, prefill = {}, {}  # seq -> remaining decode steps / remaining prompt tokens
    for _ in range(n_dec):  # decode sequences start with a prefilled context
        m.append([(next_id, int(rng.integers(lo, hi + 1)))])
        decode[next_id] = int(rng.integers(1, steps + 1))
        next_id += 1
    for step in range(steps):
        while len(prefill) < n_pref:
            prefill[next_id] = int(rng.integers(chunk, 4 * chunk + 1))
            next_id += 1
        work = [(s, 1) for s in decode] + [(s, min(chunk, r)) for s, r in prefill.items()]
        m.append(work)
        seqs = list(decode)
        check = None
        if full and step % 50 != 49:
            check = sorted({step % len(seqs), int(rng.integers(len(seqs)))})
        if full and step % 20 == 0:
            banner(f"config-3 step {step}: {len(seqs)} decode sequences, "
                   f"{m.cache.stats().used_blocks} blocks in use")
        m.attention(seqs, check=check, max_blocks=(hi + steps + 4 * chunk) // BS + 2)
        for s in list(prefill):
            prefill[s] -= min(chunk, prefill[s])
            if prefill[s] == 0:  # prompt done: becomes a decode sequence
                del prefill[s]
                decode[s] = int(rng.integers(1, steps + 1))
        for s in list(decode):
            decode[s] -= 1
            if decode[s] == 0:  # finished: blocks go back to the shared free list
                m.cache.free_sequence(s)
                del decode[s]
        while len(decode) < n_dec:
            m.append([(next_id, int(rng.integers(lo, hi + 1)))])
            decode[next_id] = int(rng.integers(1, steps + 1))
            next_id += 1
        m.assert_books_consistent(list(decode) + list(prefill))
    m.assert_pools_equal()


def test_config4_long_context_70b(oracle, torch_mod, cuda):
    """70B shape (64 q heads, 8 kv heads), 8 x 32768 tokens on scattered blocks,
    1% of K rows x8: split-K over 64 partitions per sequence + LSE merge."""
    banner("config-4 long context")
    torch = torch_mod
    B, ctx = 8, 32768
    m = Mirror(torch, cuda, oracle, B * ctx // BS + 64, seed=4, hq=64)
    for s in range(B):
        m.append([(s, ctx)], sigma=1.0, outlier_frac=0.01)
    out = m.attention(list(range(B)), check=[0, 5])
    assert np.all(np.isfinite(out))
    m.assert_pools_equal(ids=m.cache.block_table(5)[:64])


def test_config5_verify_rollback_fork_swap(oracle, torch_mod, cuda):
    """Speculative decode on the 8B shape: append k=4 drafts, 4-query causal
    verify, roll back 0-4 rejected tokens (truncate), fork 8 sequences by block
    copy, swap 25% of blocks to pinned host memory and back.  All bit-exact."""
    banner("config-5 verify/rollback/fork/swap")
    torch = torch_mod
    B, k = 32, 4
    rng = np.random.default_rng(5)
    m = Mirror(torch, cuda, oracle, 16000, seed=5)
    from dlm_amd import ops as m_ops
    ctxs = rng.integers(1024, 8193, B)
    for s in range(B):
        m.append([(s, int(ctxs[s]))])
    for step in range(3):
        m.append([(s, k) for s in range(B)])
        m.attention(list(range(B)), nq=k, check=rng.choice(B, 3, replace=False), max_blocks=520)
        before = {s: m.cache.block_table(s) for s in range(B)}
        for s in range(B):
            r = int(rng.integers(0, k + 1))
            L = m.cache.sequence_len(s)
            m.cache.truncate_sequence(s, L - r)
            # truncate then re-append r tokens restores the same physical blocks
            m.cache.append_tokens(s, r)
            assert m.cache.block_table(s) == before[s]
            m.cache.truncate_sequence(s, L - r)
        m.assert_books_consistent(range(B))
    # Fork 8 sequences: private block copies, identical attention.
    pairs = np.concatenate([m.cache.fork_sequence(s, 100 + s) for s in range(8)])
    m_ops.copy_blocks(m.kd, m.vd, to_dev(torch, pairs, cuda), m.block_bytes)
    oracle.copy_blocks(m.kh, m.vh, pairs, m.block_bytes)
    m.assert_pools_equal(ids=pairs[:, 1])
    q = (rng.standard_normal((1, 1, 32, D)) * 0.5).astype(np.float16)
    for s in range(8):
        tables, lens = m.cache.block_tables([s, 100 + s], 520)
        o = m_ops.paged_decode_attention(to_dev(torch, np.repeat(q, 2, 0), cuda), m.kd, m.vd,
                                         to_dev(torch, tables, cuda), to_dev(torch, lens, cuda),
                                         num_kv_heads=HKV)
        assert torch.equal(o[0], o[1])
    # Swap 25% of the owned blocks out and back in through pinned host memory.
    owned = np.array(sorted(b for s in list(range(B)) + [100 + s for s in range(8)]
                            for b in m.cache.block_table(s)), np.int32)
    ids = rng.choice(owned, len(owned) // 4, replace=False).astype(np.int32)
    nbytes = 2 * len(ids) * m.block_bytes
    host = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    staging = torch.empty(nbytes, dtype=torch.uint8, device=cuda)
    ids_dev = to_dev(torch, ids, cuda)
    m_ops.swap_out(host, m.kd, m.vd, ids_dev, m.block_bytes, staging)
    torch.cuda.synchronize()
    assert np.array_equal(host.numpy(), oracle.gather_blocks(m.kh, m.vh, ids, m.block_bytes))
    m.kd[ids_dev.long()] = 0  # evicted blocks are reused by someone else meanwhile
    m.vd[ids_dev.long()] = 0
    m_ops.swap_in(m.kd, m.vd, host, ids_dev, m.block_bytes, staging)
    m.assert_pools_equal()


def test_prefix_cache_on_shared_blocks(oracle, torch_mod, cuda):
    """dlm's prefix cache (src/batching.rs:32-72: a prompt's KvSnapshot cloned
    for every request that extends it) on shared blocks: a 1000-token system
    prompt is prefilled once and forked to 6 requests by reference; every
    sequence appends its own suffix (copy-on-write of the shared partial block)
    and then decodes.  Pools stay bit-identical to the mirror, attention matches
    the oracle for every sequence, and the prompt's full blocks are stored once."""
    banner("prefix cache on shared blocks")
    m = Mirror(torch_mod, cuda, oracle, 3000, seed=9)
    rng = np.random.default_rng(99)
    prefix, n_req = 1000, 6
    m.append([(0, prefix)])
    for r in range(1, n_req + 1):
        m.cache.fork_sequence_shared(0, r)
    seqs = list(range(n_req + 1))
    used = m.cache.stats().used_blocks
    assert used == -(-prefix // BS)  # forks allocate nothing
    pairs = m.append_cow([(s, int(rng.integers(1, 300))) for s in seqs])
    # The shared partial block (8 tokens) is copied for every sequence but the
    # last one to append, which keeps it; the 62 full blocks stay shared.
    assert len(pairs) == n_req
    full = prefix // BS
    prompt_blocks = m.cache.block_table(n_req)[:full]
    for s in seqs:
        assert m.cache.block_table(s)[:full] == prompt_blocks
    assert all(m.cache.block_refcount(b) == n_req + 1 for b in prompt_blocks)
    m.assert_pools_equal()
    m.attention(seqs)
    for _ in range(4):  # decode steps: private tails now, so no copies
        assert len(m.append_cow([(s, 1) for s in seqs])) == 0
        m.attention(seqs)
    m.cache.free_sequence(0)  # the origin finishes: the prompt stays for the others
    assert all(m.cache.block_refcount(b) == n_req for b in prompt_blocks)
    assert not set(prompt_blocks) & set(m.cache.free_list())
    m.attention(seqs[1:])
    m.assert_pools_equal()
