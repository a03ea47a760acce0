"""GPU parity: every libdlmk entry point against the CPU oracle on identical
seeded inputs.  Append, block copy and swap are bit-exact; attention is within
2e-3 abs + 1e-3 rel (f16 KV) or 1e-5 (f32 KV) of the oracle's f32 restatement of
dlm's attention() (src/forward/cpu.rs:1126-1151)."""
import numpy as np
import pytest

from helpers import (BF16_ATOL, BF16_RTOL, F16_ATOL, F16_RTOL, F32_ATOL, F32_RTOL, assert_close,
                     make_workload, to_dev)

pytestmark = pytest.mark.gpu


def banner(msg):
    print(f"[gpu-test] {msg}", flush=True)


@pytest.fixture(scope="module")
def torch_mod(cuda):
    import torch
    return torch


@pytest.fixture(scope="module")
def ops(cuda):
    from dlm_amd import ops as _ops
    return _ops


# ------------------------------------------------------------------ append

@pytest.mark.parametrize("dtype,Hkv,d,ntok,chunked", [
    (np.float32, 8, 64, 64, False),   # config-1 shape, one token per sequence
    (np.float16, 8, 128, 64, False),  # config-2 shape decode step
    (np.float16, 8, 128, 2096, True), # config-3 step: 48 decode + 4 x 512 chunk
    (np.float16, 2, 64, 300, True),
    (np.float16, 2, 24, 50, True),    # 3 chunks per head row: one chunk per thread
    ("bf16", 8, 128, 100, False),
    # >= 512 tokens: 16-token runs per work-group (whole-tile stores for full
    # blocks, per-chunk stores otherwise) at 128 to 1024 threads
    (np.float32, 8, 64, 640, True),
    (np.float32, 1, 256, 520, "shifted"),  # runs straddle blocks
    (np.float16, 4, 256, 700, True),
    (np.float16, 2, 64, 600, False),     # no run fills a block
    ("bf16", 8, 128, 1024, "shifted"),
])
def test_kv_append_bit_exact(oracle, torch_mod, ops, cuda, dtype, Hkv, d, ntok, chunked):
    torch = torch_mod
    banner(f"kv_append dtype={dtype} Hkv={Hkv} d={d} ntok={ntok}")
    rng = np.random.default_rng(100 + ntok)
    bs, nb = 16, ntok // 4 + 200 if chunked else max(ntok // 4 + 200, ntok + 64)
    npdt = np.float16 if dtype == "bf16" else dtype
    X = 16 // np.dtype(npdt).itemsize
    kp = rng.integers(0, 2**16, (nb, Hkv, d // X, bs, X)).astype(np.uint16) if npdt == np.float16 \
        else rng.standard_normal((nb, Hkv, d // X, bs, X)).astype(np.float32)
    vp = rng.integers(0, 2**16, (nb, Hkv, d, bs)).astype(np.uint16) if npdt == np.float16 \
        else rng.standard_normal((nb, Hkv, d, bs)).astype(np.float32)
    if npdt == np.float16:
        kp, vp = kp.view(np.float16), vp.view(np.float16)
    ks = rng.standard_normal((ntok, Hkv, d)).astype(npdt)
    vs = rng.standard_normal((ntok, Hkv, d)).astype(npdt)
    if chunked:  # runs of consecutive slots inside shuffled blocks
        blocks = rng.permutation(nb)
        o = 5 if chunked == "shifted" else 0  # the chunk starts mid-block
        slots = np.array([blocks[(p + o) // bs] * bs + (p + o) % bs for p in range(ntok)], np.int64)
    else:  # one token per sequence, each in its own block at a random offset
        slots = rng.permutation(nb)[:ntok].astype(np.int64) * bs + rng.integers(0, bs, ntok)
    slots[::37] = -1  # skipped tokens
    tdt = torch.bfloat16 if dtype == "bf16" else None
    dev = lambda a: (to_dev(torch, a.view(np.int16), cuda).view(tdt) if tdt
                     else to_dev(torch, a, cuda))
    k_dev, v_dev = dev(kp), dev(vp)
    ops.kv_append(k_dev, v_dev, dev(ks), dev(vs), to_dev(torch, slots, cuda), num_kv_heads=Hkv,
                  head_dim=d)
    oracle.paged_append(kp, vp, ks, vs, slots, Hkv, d, bs)
    torch.cuda.synchronize()
    back = lambda t: (t.view(torch.int16).cpu().numpy().view(np.float16) if tdt
                      else t.cpu().numpy())
    assert np.array_equal(back(k_dev).view(np.uint8), kp.view(np.uint8))
    assert np.array_equal(back(v_dev).view(np.uint8), vp.view(np.uint8))


def test_kv_append_ignores_out_of_pool_slots(torch_mod, ops, cuda):
    torch = torch_mod
    banner("kv_append out-of-pool slots")
    kp = torch.zeros((2, 1, 8, 16, 8), dtype=torch.float16, device=cuda)
    vp = torch.zeros((2, 1, 64, 16), dtype=torch.float16, device=cuda)
    src = torch.ones((3, 1, 64), dtype=torch.float16, device=cuda)
    slots = torch.tensor([-5, 32, 10**9], dtype=torch.int64, device=cuda)
    ops.kv_append(kp, vp, src, src, slots, num_kv_heads=1, head_dim=64)
    torch.cuda.synchronize()
    assert kp.abs().sum().item() == 0 and vp.abs().sum().item() == 0


def test_kv_append_rejects_mismatched_shapes(torch_mod, ops, cuda):
    torch = torch_mod
    kp = torch.zeros((2, 1, 8, 16, 8), dtype=torch.float16, device=cuda)
    vp = torch.zeros_like(kp).view(2, 1, 64, 16)
    src = torch.ones((3, 1, 64), dtype=torch.float16, device=cuda)
    with pytest.raises(ValueError):
        ops.kv_append(kp, vp, src, src, torch.zeros(4, dtype=torch.int64, device=cuda),
                      num_kv_heads=1, head_dim=64)
    with pytest.raises(TypeError):
        ops.kv_append(kp, vp, src.float(), src.float(),
                      torch.zeros(3, dtype=torch.int64, device=cuda), num_kv_heads=1, head_dim=64)


# ------------------------------------------------------------------ attention

def run_attention(torch, ops, cuda, w, out_dtype=None):
    out = ops.paged_decode_attention(
        to_dev(torch, w.q, cuda), to_dev(torch, w.k_pool, cuda), to_dev(torch, w.v_pool, cuda),
        to_dev(torch, w.tables, cuda), to_dev(torch, w.ctx, cuda), num_kv_heads=w.Hkv,
        scale=float(w.scale), out_dtype=out_dtype)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def oracle_attention(oracle, w):
    return oracle.paged_attention(w.q, w.k_pool, w.v_pool, w.tables, w.ctx, w.nq, w.Hq, w.Hkv,
                                  w.d, w.bs, w.scale)


EDGE_CTX = [0, 1, 2, 15, 16, 17, 255, 256, 257, 511, 513, 1000]


@pytest.mark.parametrize("dtype,Hq,Hkv,d,nq,ctx", [
    (np.float32, 32, 8, 64, 1, [576, 1, 300]),             # config-1 shape: 64-token partitions
    (np.float32, 32, 8, 64, 1, EDGE_CTX),                   # 128-token partitions
    (np.float32, 32, 8, 64, 1, list(range(37, 1537, 37))),  # 40 seqs: 256-token partitions
    (np.float32, 32, 8, 128, 1, [2049]),                    # the decode block's 8B shape
    (np.float32, 128, 32, 128, 1, list(range(100, 4000, 197))),  # f32, 256-token partitions, d 128
    # f32 geometries of any head dim (multiple of 4) and group: the generic kernel
    (np.float32, 4, 2, 4, 1, [1, 17, 40]),                  # reference speculative tests' model
    (np.float32, 4, 2, 8, 1, [1, 5, 33]),                   # reference gpu_parity.rs:73-77 shape
    (np.float32, 6, 3, 12, 2, [2, 20, 77]),                 # 3 chunk rows
    (np.float32, 12, 4, 80, 2, [2, 130, 1000]),
    (np.float32, 32, 8, 96, 1, EDGE_CTX),
    (np.float32, 64, 2, 64, 1, [300, 900]),                 # GQA 32: two row groups
    (np.float32, 16, 4, 256, 1, [17, 900]),
    (np.float32, 8, 8, 16, 4, [4, 16, 70]),
    (np.float32, 48, 4, 20, 3, [3, 50, 600]),               # GQA 12 x 3 queries: 3 row groups
    (np.float16, 32, 8, 128, 1, EDGE_CTX),                  # config-2 shape
    (np.float16, 32, 8, 128, 1, [1023, 1024, 1025, 2048, 2049]),  # partition edges
    (np.float16, 32, 8, 128, 1, [9000, 100, 8193]),          # > 8 partitions: work-group combine
    (np.float16, 64, 8, 128, 1, [4000, 17, 2049]),          # 70B shape, GQA 8
    (np.float16, 8, 8, 128, 1, [100, 700]),                 # MHA (group 1)
    (np.float16, 16, 8, 64, 1, [100, 700]),                 # group 2, d 64
    (np.float16, 16, 8, 128, 2, [3, 1, 300, 600]),          # 2-query verify
    (np.float16, 8, 8, 128, 4, [4, 2, 513, 260]),           # 4-query verify, group 1
    (np.float16, 32, 8, 128, 2, [2, 257, 1025]),            # 2-query verify, group 4
    (np.float32, 16, 8, 64, 4, [5, 3, 400]),
    (np.float16, 32, 8, 128, 4, [4, 1030, 2100, 700]),      # config-5 verify: 4 queries x GQA 4
    (np.float16, 64, 8, 128, 2, [2, 600, 1500]),            # 2 queries x GQA 8
    (np.float16, 32, 2, 128, 1, [300, 1200]),               # GQA 16
    (np.float16, 16, 4, 256, 1, [17, 900]),                 # head_dim 256
    (np.float16, 16, 4, 256, 2, [2, 530]),
    ("bf16", 32, 8, 128, 1, EDGE_CTX),                      # bf16 KV, 8B shape
    ("bf16", 32, 8, 128, 4, [4, 777]),
    ("bf16", 16, 8, 64, 1, [33, 600]),
    # f16 / bf16 head dims and groups outside the tuned kernel's set
    (np.float16, 32, 8, 96, 1, EDGE_CTX),
    (np.float16, 16, 4, 80, 4, [4, 90, 1200]),
    (np.float16, 64, 8, 128, 4, [4, 700, 2100]),            # GQA 8 x 4 queries: 2 row groups
    (np.float16, 8, 2, 32, 1, [1, 40, 5000]),
    (np.float16, 24, 8, 200, 2, [2, 1100]),
    ("bf16", 24, 8, 96, 2, [2, 333, 1500]),
])
def test_paged_attention_matches_oracle(oracle, torch_mod, ops, cuda, dtype, Hq, Hkv, d, nq,
                                        ctx):
    name = dtype if isinstance(dtype, str) else np.dtype(dtype).name
    banner(f"attention dtype={name} Hq={Hq} Hkv={Hkv} d={d} nq={nq} ctx={ctx}")
    rng = np.random.default_rng(sum(ctx) + Hq + nq)
    sigma = 1.0 if dtype is np.float32 else 0.5
    w = make_workload(rng, ctx, Hq, Hkv, d, dtype, nq=nq, sigma=sigma)
    ref = oracle_attention(oracle, w)
    atol, rtol = {"float16": (F16_ATOL, F16_RTOL), "float32": (F32_ATOL, F32_RTOL),
                  "bf16": (BF16_ATOL, BF16_RTOL)}[name]
    got = run_attention(torch_mod, ops, cuda, w, out_dtype=torch_mod.float32)
    assert_close(got, ref, atol, rtol, "f32 out")
    if name != "float32":
        got16 = run_attention(torch_mod, ops, cuda, w)  # out in the KV dtype
        assert_close(got16, ref, atol, rtol, f"{name} out")


@pytest.mark.parametrize("dtype,d,nq", [(np.float16, 128, 1), (np.float16, 128, 4),
                                         (np.float32, 64, 1), (np.float32, 128, 1)])
def test_paged_attention_masks_out_of_pool_blocks(oracle, torch_mod, ops, cuda, dtype, d, nq):
    """A block id outside the pool inside the context is masked: the output equals
    attention over the same sequence with that block removed."""
    name = np.dtype(dtype).name
    banner(f"attention {name} out-of-pool table ids d={d} nq={nq}")
    rng = np.random.default_rng(33 + d + nq)
    w = make_workload(rng, [700, 1300, 90, 2100], 32, 8, d, dtype, nq=nq,
                      sigma=1.0 if dtype is np.float32 else 0.5)
    nb = w.k_pool.shape[0]
    tables = w.tables.copy()
    bad = tables.copy()
    ref_ctx = np.asarray(w.ctx, np.int32).copy()
    for s, (bi, bad_id) in {0: (3, -1), 1: (40, nb + 5), 3: (0, 2**30)}.items():
        bad[s, bi] = bad_id
        row = np.delete(tables[s], bi)
        tables[s] = np.concatenate([row, row[-1:]])
        ref_ctx[s] -= 16
    ref = oracle.paged_attention(w.q, w.k_pool, w.v_pool, tables, ref_ctx, w.nq, w.Hq, w.Hkv,
                                 w.d, w.bs, w.scale)
    w.tables = bad
    got = run_attention(torch_mod, ops, cuda, w, out_dtype=torch_mod.float32)
    atol, rtol = (F16_ATOL, F16_RTOL) if dtype is np.float16 else (F32_ATOL, F32_RTOL)
    assert_close(got, ref, atol, rtol, f"{name} masked blocks")


def test_paged_attention_ignores_stale_block_tails(oracle, torch_mod, ops, cuda):
    """Slots past the context (and past a verify query's limit) may hold NaN."""
    banner("attention stale NaN tails")
    rng = np.random.default_rng(21)
    w = make_workload(rng, [1, 17, 40, 300], 32, 8, 128, np.float16, nq=2, sigma=0.5,
                      fill_nan=True)
    ref = oracle_attention(oracle, w)
    got = run_attention(torch_mod, ops, cuda, w, out_dtype=torch_mod.float32)
    assert_close(got, ref, F16_ATOL, F16_RTOL)


def test_paged_attention_softmax_range_outliers(oracle, torch_mod, ops, cuda):
    """Config-4 style: 1% of K rows scaled x8 stress the running max / LSE merge."""
    banner("attention outlier K rows")
    rng = np.random.default_rng(22)
    w = make_workload(rng, [3000, 1200], 64, 8, 128, np.float16, sigma=1.0)
    X = 8
    kp = w.k_pool.astype(np.float32)
    rows = rng.random(kp.shape[0] * 16) < 0.01
    kp = kp.transpose(0, 3, 1, 2, 4)  # [blk, t, h, d/X, X]
    flat = kp.reshape(-1, *kp.shape[2:])
    flat[rows] *= 8
    w.k_pool = flat.reshape(kp.shape).transpose(0, 2, 3, 1, 4).astype(np.float16).copy()
    ref = oracle_attention(oracle, w)
    got = run_attention(torch_mod, ops, cuda, w, out_dtype=torch_mod.float32)
    assert_close(got, ref, F16_ATOL, F16_RTOL)


def test_paged_attention_full_config2_subset(oracle, torch_mod, ops, cuda):
    """Config 2 at full size (B=64, ctx U[128,4096], 20k-block pool), every sequence
    run on the GPU; 8 of them checked against the oracle."""
    torch = torch_mod
    banner("attention config-2 full size")
    rng = np.random.default_rng(2)
    ctx = rng.integers(128, 4097, 64).astype(np.int32)
    w = make_workload(rng, ctx, 32, 8, 128, np.float16, sigma=0.5, num_blocks=20000)
    got = run_attention(torch, ops, cuda, w, out_dtype=torch.float32)
    pick = rng.choice(64, 8, replace=False)
    sub = make_workload(rng, [1], 32, 8, 128, np.float16)  # placeholder container
    sub.k_pool, sub.v_pool = w.k_pool, w.v_pool
    sub.tables, sub.ctx, sub.q = w.tables[pick], w.ctx[pick], w.q[pick]
    ref = oracle_attention(oracle, sub)
    assert_close(got[pick], ref, F16_ATOL, F16_RTOL)


def test_paged_attention_is_deterministic_and_order_free(torch_mod, ops, cuda):
    """Same inputs -> bitwise same output; permuting the batch permutes the output."""
    torch = torch_mod
    banner("attention determinism / batch permutation")
    rng = np.random.default_rng(23)
    w = make_workload(rng, [50, 800, 2000, 5], 32, 8, 128, np.float16, sigma=0.5)
    a = run_attention(torch, ops, cuda, w)
    b = run_attention(torch, ops, cuda, w)
    assert np.array_equal(a, b)
    perm = np.array([2, 0, 3, 1])
    w.tables, w.ctx, w.q = w.tables[perm], w.ctx[perm], w.q[perm]
    c = run_attention(torch, ops, cuda, w)
    assert np.array_equal(c, a[perm])


def test_paged_attention_workspace_reuse_across_shapes(oracle, torch_mod, ops, cuda):
    """One workspace serves calls of different shapes back to back, twice over:
    nothing a call leaves in it disturbs the next call."""
    torch = torch_mod
    banner("attention workspace reuse across shapes")
    rng = np.random.default_rng(31)
    shapes = [([4000, 3100], 64, 8, 1), ([600, 1300, 40, 2500] * 3, 32, 8, 1),
              ([4, 1030, 2100, 700], 32, 8, 4), ([300, 1200], 32, 2, 1)]
    loads = [make_workload(rng, ctx, Hq, Hkv, 128, np.float16, nq=nq, sigma=0.5)
             for ctx, Hq, Hkv, nq in shapes]
    need = max(ops.attention_workspace_bytes(len(w.ctx), w.nq, w.Hq, w.d, w.tables.shape[1])
               for w in loads)
    ws = ops.alloc_workspace(need, cuda)
    for rep in range(2):
        for w in loads:
            out = ops.paged_decode_attention(
                to_dev(torch, w.q, cuda), to_dev(torch, w.k_pool, cuda),
                to_dev(torch, w.v_pool, cuda), to_dev(torch, w.tables, cuda),
                to_dev(torch, w.ctx, cuda), num_kv_heads=w.Hkv, scale=float(w.scale),
                out_dtype=torch.float32, workspace=ws)
            torch.cuda.synchronize()
            assert_close(out.cpu().numpy(), oracle_attention(oracle, w), F16_ATOL, F16_RTOL,
                         f"rep {rep} B={len(w.ctx)} Hq={w.Hq} nq={w.nq}")


@pytest.mark.parametrize("dtype,ctx,table_blocks", [
    (np.float16, [100, 1500, 3000], 256),      # <= 8 partitions a row: wave-per-row combine
    (np.float16, [100, 1500, 9000], 600),      # > 8: work-group-per-row combine
    (np.float32, [40, 700, 1000], 64),         # f32, 128-token partitions
])
def test_paged_attention_nan_workspace(oracle, torch_mod, ops, cuda, dtype, ctx, table_blocks):
    """The combine kernels read workspace slots past a row's partition count
    before they know it: a workspace full of NaN there changes nothing."""
    torch = torch_mod
    banner(f"attention NaN workspace dtype={np.dtype(dtype).name} ctx={ctx}")
    rng = np.random.default_rng(41 + len(ctx) + table_blocks)
    w = make_workload(rng, ctx, 32, 8, 64 if dtype is np.float32 else 128, dtype,
                      sigma=1.0 if dtype is np.float32 else 0.5)
    tables = np.zeros((len(ctx), table_blocks), np.int32)
    tables[:, :w.tables.shape[1]] = w.tables
    w.tables = tables  # wider tables: more partition slots than any row uses
    need = ops.attention_workspace_bytes(len(w.ctx), w.nq, w.Hq, w.d, table_blocks)
    ws = ops.alloc_workspace(need, cuda)
    ws.fill_(255)  # every f32 in it is a NaN
    out = ops.paged_decode_attention(
        to_dev(torch, w.q, cuda), to_dev(torch, w.k_pool, cuda), to_dev(torch, w.v_pool, cuda),
        to_dev(torch, w.tables, cuda), to_dev(torch, w.ctx, cuda), num_kv_heads=w.Hkv,
        scale=float(w.scale), out_dtype=torch.float32, workspace=ws)
    torch.cuda.synchronize()
    atol, rtol = (F32_ATOL, F32_RTOL) if dtype is np.float32 else (F16_ATOL, F16_RTOL)
    assert_close(out.cpu().numpy(), oracle_attention(oracle, w), atol, rtol, "NaN workspace")


def test_paged_attention_rejects_misaligned_operands(torch_mod, ops, cuda):
    """Q and the pools are read 16 bytes a lane: a view 2 bytes off the
    allocation is refused before any launch."""
    torch = torch_mod
    from dlm_amd import DlmkError
    kp = torch.zeros((4, 8, 16, 16, 8), dtype=torch.float16, device=cuda)
    vp = torch.zeros((4, 8, 128, 16), dtype=torch.float16, device=cuda)
    t = torch.zeros((1, 4), dtype=torch.int32, device=cuda)
    lens = torch.ones(1, dtype=torch.int32, device=cuda)
    q = torch.zeros(1 * 32 * 128 + 1, dtype=torch.float16, device=cuda)[1:].view(1, 1, 32, 128)
    with pytest.raises(DlmkError):
        ops.paged_decode_attention(q, kp, vp, t, lens, num_kv_heads=8)
    torch.cuda.synchronize()


def test_paged_attention_unsupported_shape_raises(torch_mod, ops, cuda):
    torch = torch_mod
    from dlm_amd import DlmkError
    q = torch.zeros((1, 1, 8, 264), dtype=torch.float16, device=cuda)  # head_dim above 256
    kp = torch.zeros((4, 8, 33, 16, 8), dtype=torch.float16, device=cuda)
    vp = torch.zeros((4, 8, 264, 16), dtype=torch.float16, device=cuda)
    t = torch.zeros((1, 4), dtype=torch.int32, device=cuda)
    with pytest.raises(DlmkError):
        ops.paged_decode_attention(q, kp, vp, t, t[:, 0].contiguous(), num_kv_heads=8)


# ------------------------------------------------------------------ copy / swap

def test_copy_blocks_bit_exact(oracle, torch_mod, ops, cuda):
    torch = torch_mod
    banner("copy_blocks")
    rng = np.random.default_rng(30)
    nb, bb = 300, 8 * 16 * 128 * 2
    kp = rng.integers(0, 256, nb * bb, dtype=np.uint8)
    vp = rng.integers(0, 256, nb * bb, dtype=np.uint8)
    ids = rng.permutation(nb)
    pairs = np.stack([ids[:100], ids[100:200]], 1).astype(np.int32)
    pairs[5] = [7, 1000]  # out-of-pool pair is skipped
    k_dev, v_dev = to_dev(torch, kp, cuda), to_dev(torch, vp, cuda)
    ops.copy_blocks(k_dev, v_dev, to_dev(torch, pairs, cuda), bb)
    oracle.copy_blocks(kp, vp, np.delete(pairs, 5, 0), bb)
    torch.cuda.synchronize()
    assert np.array_equal(k_dev.cpu().numpy(), kp)
    assert np.array_equal(v_dev.cpu().numpy(), vp)


def test_fork_then_attention_matches_source(oracle, torch_mod, ops, cuda):
    """Paged form of resume_from_snapshot_matches_full_prefill (src/generate.rs:659-680):
    attention over a forked table equals attention over the original."""
    torch = torch_mod
    banner("fork + attention")
    from dlm_amd import KvCacheConfig, PagedKvCache
    rng = np.random.default_rng(31)
    Hq, Hkv, d = 32, 8, 128
    cfg = KvCacheConfig(1, Hkv, d, 16)
    cache = PagedKvCache.with_seeded_shuffle(cfg, 400, seed=31)
    cache.append_tokens(0, 1000)
    w = make_workload(rng, [1000], Hq, Hkv, d, np.float16, sigma=0.5, num_blocks=400)
    w.tables, _ = cache.block_tables([0], 64)
    pairs = cache.fork_sequence(0, 1)
    k_dev, v_dev = to_dev(torch, w.k_pool, cuda), to_dev(torch, w.v_pool, cuda)
    ops.copy_blocks(k_dev, v_dev, to_dev(torch, pairs, cuda), 8 * 16 * d * 2)
    tables, lens = cache.block_tables([0, 1], 64)
    q = np.repeat(w.q, 2, 0)
    out = ops.paged_decode_attention(to_dev(torch, q, cuda), k_dev, v_dev,
                                     to_dev(torch, tables, cuda), to_dev(torch, lens, cuda),
                                     num_kv_heads=Hkv)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    assert np.array_equal(o[0], o[1])
    assert not set(tables[0][:63]) & set(tables[1][:63])


def test_gather_scatter_swap_round_trip(oracle, torch_mod, ops, cuda):
    torch = torch_mod
    banner("gather/scatter/swap")
    rng = np.random.default_rng(32)
    nb, bb = 256, 8 * 16 * 128 * 2
    kp = rng.integers(0, 256, nb * bb, dtype=np.uint8)
    vp = rng.integers(0, 256, nb * bb, dtype=np.uint8)
    ids = rng.permutation(nb)[:64].astype(np.int32)
    k_dev, v_dev = to_dev(torch, kp, cuda), to_dev(torch, vp, cuda)
    ids_dev = to_dev(torch, ids, cuda)
    staging = ops.gather_blocks(k_dev, v_dev, ids_dev, bb)
    torch.cuda.synchronize()
    assert np.array_equal(staging.cpu().numpy().reshape(-1), oracle.gather_blocks(kp, vp, ids, bb))
    # swap out to pinned host, clobber the blocks, swap back in: identity on bytes
    host = torch.empty(2 * len(ids) * bb, dtype=torch.uint8, pin_memory=True)
    stage2 = torch.empty(2 * len(ids) * bb, dtype=torch.uint8, device=cuda)
    ops.swap_out(host, k_dev, v_dev, ids_dev, bb, stage2)
    torch.cuda.synchronize()
    assert np.array_equal(host.numpy(), oracle.gather_blocks(kp, vp, ids, bb))
    zeros = torch.zeros((len(ids), 2, bb), dtype=torch.uint8, device=cuda)
    ops.scatter_blocks(k_dev, v_dev, zeros, ids_dev, bb)
    torch.cuda.synchronize()
    assert k_dev.view(nb, bb)[ids_dev.long()].sum().item() == 0
    ops.swap_in(k_dev, v_dev, host, ids_dev, bb, stage2)
    torch.cuda.synchronize()
    assert np.array_equal(k_dev.cpu().numpy(), kp)
    assert np.array_equal(v_dev.cpu().numpy(), vp)


def test_swap_through_library_pinned_buffer(oracle, torch_mod, ops, cuda):
    """Swap staging in host memory from dlmk_alloc_pinned (dlm's PinnedBuffer,
    src/memory/pinned.rs:38-112) instead of torch's pinned allocator: starts
    zeroed, rounds up to whole pages, swap-out then swap-in is the identity on
    the evicted blocks' bytes, and dlmk_free_pinned releases it."""
    torch = torch_mod
    banner("swap through dlmk_alloc_pinned")
    rng = np.random.default_rng(34)
    nb, bb = 200, 8 * 16 * 64 * 4  # f32 blocks of the config-1 shape
    kp = rng.integers(0, 256, nb * bb, dtype=np.uint8)
    vp = rng.integers(0, 256, nb * bb, dtype=np.uint8)
    ids = rng.permutation(nb)[:50].astype(np.int32)
    k_dev, v_dev = to_dev(torch, kp, cuda), to_dev(torch, vp, cuda)
    ids_dev = to_dev(torch, ids, cuda)
    nbytes = 2 * len(ids) * bb + 100  # not a page multiple
    buf = ops.PinnedBuffer(nbytes)
    assert buf.capacity % 4096 == 0 and buf.capacity >= nbytes
    host = buf.numpy()
    assert host.size == nbytes and not host.any()  # zero-initialised
    staging = torch.empty(2 * len(ids) * bb, dtype=torch.uint8, device=cuda)
    ops.swap_out(buf, k_dev, v_dev, ids_dev, bb, staging)
    torch.cuda.synchronize()
    assert np.array_equal(host[:2 * len(ids) * bb], oracle.gather_blocks(kp, vp, ids, bb))
    assert not host[2 * len(ids) * bb:].any()
    k_dev.view(nb, bb)[ids_dev.long()] = 0
    v_dev.view(nb, bb)[ids_dev.long()] = 0
    ops.swap_in(k_dev, v_dev, buf, ids_dev, bb, staging)
    torch.cuda.synchronize()
    assert np.array_equal(k_dev.cpu().numpy(), kp)
    assert np.array_equal(v_dev.cpu().numpy(), vp)
    buf.free()
    with pytest.raises(ValueError):
        buf.data_ptr()
    buf.free()  # a second free is a no-op
