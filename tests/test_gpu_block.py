"""dlmk_decode_block_paged (one decode block over the paged cache) against the
CPU oracle's decode_block over the same paged pools.

Mirrors the reference's device parity suite (tests/gpu_parity.rs): weights
drawn by its SplitMix64 generator (uniform(-1, 1) * 0.05, unit norms), the
same starting hidden states, several decode steps on two layers, and its
tolerances on the hidden state -- 1e-3, or 2e-3 for int4 / int8 weights and
the realistic width (gpu_parity.rs:114-116, :183, :218, :237).  Head dims run
from the reference's own toy configs (hidden 32 / head_dim 8,
gpu_parity.rs:73-77; hidden 16 / head_dim 4, tests/speculative.rs:33-42) to 64,
96 and 128, and GQA groups from 1 to 16.  Each case starts at a 14-token
history already in the pools so the steps cross a block boundary, on shuffled
physical blocks.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

W_F32, W_BF16, W_F16, W_INT4, W_INT8 = 0, 1, 2, 3, 4


def banner(msg):
    print(f"\n[gpu-block] {msg}", flush=True)


def make_layer(oracle, rng_seed, H, Hq, Hkv, d, I, w_dtype, biases=False):
    """Host weights (native dtype arrays) for one layer, plus their f32 values."""
    qd, kvd = Hq * d, Hkv * d
    shapes = {"q_proj": qd * H, "k_proj": kvd * H, "v_proj": kvd * H, "o_proj": H * qd,
              "gate_proj": I * H, "up_proj": I * H, "down_proj": H * I}
    w = {}
    for i, (name, n) in enumerate(shapes.items()):
        f = oracle.rng_uniform(rng_seed * 131 + i, n, 0.05)
        if w_dtype == W_F32:
            w[name] = f
        elif w_dtype == W_BF16:
            w[name] = oracle.bf16_bits(f)
        elif w_dtype == W_F16:
            w[name] = f.astype(np.float16).view(np.uint16)
        else:
            w[name] = oracle.quantize_weights(f, w_dtype)
    w["in_norm"] = np.ones(H, np.float32)
    w["post_norm"] = np.ones(H, np.float32)
    if biases:
        w["q_bias"] = oracle.rng_uniform(rng_seed * 7 + 1, qd, 0.1)
        w["k_bias"] = oracle.rng_uniform(rng_seed * 7 + 2, kvd, 0.1)
        w["v_bias"] = oracle.rng_uniform(rng_seed * 7 + 3, kvd, 0.1)
    return w


def to_layer(torch, w, cuda):
    from dlm_amd.block import LayerWeights
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    raw = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).ravel()).to(cuda)
    return LayerWeights(
        q_proj=raw(w["q_proj"]), k_proj=raw(w["k_proj"]), v_proj=raw(w["v_proj"]),
        o_proj=raw(w["o_proj"]), gate_proj=raw(w["gate_proj"]), up_proj=raw(w["up_proj"]),
        down_proj=raw(w["down_proj"]), input_layernorm=t(w["in_norm"]),
        post_attention_layernorm=t(w["post_norm"]), q_bias=t(w.get("q_bias")),
        k_bias=t(w.get("k_bias")), v_bias=t(w.get("v_bias")))


CASES = [
    # name, (hidden, heads, kv heads, head_dim, inter), w_dtype, tol, biases, rope (theta, scaling)
    ("f32", (256, 4, 2, 64, 512), W_F32, 1e-3, False, (10000.0, None)),
    ("bf16", (256, 4, 2, 64, 512), W_BF16, 1e-3, False, (10000.0, None)),
    ("f16", (256, 4, 2, 64, 512), W_F16, 1e-3, False, (10000.0, None)),
    ("int4", (256, 4, 2, 64, 512), W_INT4, 2e-3, False, (10000.0, None)),
    ("int8", (256, 4, 2, 64, 512), W_INT8, 2e-3, False, (10000.0, None)),
    ("hidden2048", (2048, 16, 4, 128, 512), W_F32, 2e-3, False, (10000.0, None)),
    ("qkv-bias+llama3-rope", (256, 4, 2, 64, 512), W_F32, 1e-3, True,
     (500000.0, ("llama3", 8.0, 1.0, 4.0, 8192.0))),
    ("gqa8-bf16", (512, 8, 1, 64, 1024), W_BF16, 1e-3, False, (10000.0, None)),
    ("gpu_parity-hidden32-d8", (32, 4, 2, 8, 64), W_F32, 1e-3, False, (10000.0, None)),
    ("speculative-hidden16-d4", (16, 4, 2, 4, 32), W_F32, 1e-3, False, (10000.0, None)),
    ("d96-gqa3", (384, 6, 2, 96, 512), W_F32, 1e-3, False, (10000.0, None)),
    ("d80-bf16", (320, 4, 4, 80, 640), W_BF16, 1e-3, False, (10000.0, None)),
    ("gqa16", (1024, 16, 1, 64, 512), W_F32, 1e-3, False, (10000.0, None)),
]


def run_case(oracle, cuda, name, shape, w_dtype, tol, biases, rope, hist=14, max_blocks=8,
             steps=4, poison=False):
    """Runs `steps` decode steps of two layers from a `hist`-token history on
    shuffled blocks and checks the hidden state and the appended K/V."""
    import torch
    from dlm_amd.block import BlockConfig, PagedGpuKernel, rope_inv_freqs

    H, Hq, Hkv, d, I = shape
    banner(f"decode block {name}: hidden={H} heads={Hq}/{Hkv} d={d} inter={I} w_dtype={w_dtype} "
           f"hist={hist}")
    cfg = BlockConfig(H, Hq, Hkv, d, I, rope_theta=rope[0], rms_eps=1e-5, rope_scaling=rope[1])
    gs = 128 if w_dtype in (W_INT4, W_INT8) else 0
    host = [make_layer(oracle, 17 + L, H, Hq, Hkv, d, I, w_dtype, biases) for L in range(2)]
    kern = PagedGpuKernel(cfg, [to_layer(torch, w, cuda) for w in host], w_dtype, gs,
                          max_blocks_per_seq=max_blocks, device=cuda)
    if poison:  # the block must not rely on a zeroed workspace
        kern.workspace.fill_(0x7f)
    inv = rope_inv_freqs(d, rope[0], rope[1])  # the host-side frequencies the device reads

    used = (hist + steps + 15) // 16
    nb = used + 9
    rng = np.random.default_rng(5)
    table = np.full(max_blocks, 0, np.int32)
    table[:used] = rng.permutation(nb)[:used]
    pools_h = []
    for L in range(2):
        kp = np.zeros((nb, Hkv, d * 16), np.float32)
        vp = np.zeros((nb, Hkv, d * 16), np.float32)
        # a prior history in both pools
        k = (rng.standard_normal((hist, Hkv, d)) * 0.5).astype(np.float32)
        v = (rng.standard_normal((hist, Hkv, d)) * 0.5).astype(np.float32)
        p = np.arange(hist)
        slots = (table[p // 16].astype(np.int64) * 16 + p % 16).astype(np.int64)
        oracle.paged_append(kp.reshape(nb, Hkv, d // 4, 16, 4), vp.reshape(nb, Hkv, d, 16),
                            k, v, slots, Hkv, d, 16)
        pools_h.append((kp, vp))
    pools_d = [(torch.from_numpy(kp.copy()).to(cuda), torch.from_numpy(vp.copy()).to(cuda))
               for kp, vp in pools_h]
    table_d = torch.from_numpy(table).to(cuda)

    c = dict(hidden_size=H, num_heads=Hq, num_kv_heads=Hkv, head_dim=d, inter=I, rms_eps=1e-5,
             w_dtype=w_dtype, w_group_size=gs)
    x_ref = (np.arange(H) % 17 * 0.03 - 0.25).astype(np.float32)  # gpu_parity.rs:143-145
    x_dev = torch.from_numpy(x_ref.copy()).to(cuda)
    for step in range(steps):
        p = hist + step
        for L in range(2):
            x_ref = oracle.decode_block_paged(c, host[L], x_ref, pools_h[L][0], pools_h[L][1],
                                              table, p, p, inv)
            kern.run_block(L, x_dev, pools_d[L], table_d, p, p)
        torch.cuda.synchronize()
        got = x_dev.cpu().numpy()
        diff = float(np.abs(got - x_ref).max())
        assert diff < tol, f"{name} step {step}: GPU diverged from the oracle by {diff}"
    for L in range(2):  # the appended K/V (after RoPE) match too
        for dev_pool, host_pool in zip(pools_d[L], pools_h[L]):
            np.testing.assert_allclose(dev_pool.cpu().numpy(), host_pool, atol=tol, rtol=0)


@pytest.mark.parametrize("name,shape,w_dtype,tol,biases,rope", CASES, ids=[c[0] for c in CASES])
def test_decode_block_matches_oracle(oracle, cuda, name, shape, w_dtype, tol, biases, rope):
    run_case(oracle, cuda, name, shape, w_dtype, tol, biases, rope)


LONG = [
    # name, shape, w_dtype, tol, hist, max_blocks: several split-K partitions
    # and the combine launch, on a workspace that starts as garbage
    ("f32-hist700", (256, 4, 2, 64, 512), W_F32, 1e-3, 700, 64),
    ("hidden2048-d128-hist1000", (2048, 16, 4, 128, 512), W_F32, 2e-3, 1000, 80),
    ("gqa16-hist330", (1024, 16, 1, 64, 512), W_F32, 1e-3, 330, 32),
    ("d96-gqa3-hist200", (384, 6, 2, 96, 512), W_F32, 1e-3, 200, 16),
    ("hidden32-d8-hist150", (32, 4, 2, 8, 64), W_F32, 1e-3, 150, 16),
]


@pytest.mark.parametrize("name,shape,w_dtype,tol,hist,max_blocks", LONG, ids=[c[0] for c in LONG])
def test_decode_block_long_context(oracle, cuda, name, shape, w_dtype, tol, hist, max_blocks):
    run_case(oracle, cuda, name, shape, w_dtype, tol, False, (10000.0, None), hist=hist,
             max_blocks=max_blocks, steps=3, poison=True)


def test_decode_token_books_and_pools(oracle, cuda):
    """decode_token: the books reserve each token (KvCacheExhausted when the
    pool runs out, before any launch) and the layers run at that position."""
    import torch
    from dlm_amd import KvCacheConfig, KvCacheExhausted, PagedKvCache
    from dlm_amd.block import BlockConfig, PagedGpuKernel, decode_token, rope_inv_freqs

    banner("decode_token over the books")
    H, Hq, Hkv, d, I = 256, 4, 2, 64, 512
    cfg = BlockConfig(H, Hq, Hkv, d, I)
    host = [make_layer(oracle, 3 + L, H, Hq, Hkv, d, I, W_F32) for L in range(2)]
    kern = PagedGpuKernel(cfg, [to_layer(torch, w, cuda) for w in host], W_F32,
                          max_blocks_per_seq=4, device=cuda)
    cache = PagedKvCache.with_seeded_shuffle(KvCacheConfig(2, Hkv, d, 16), 3, seed=9)
    pools_d = [(torch.zeros((3, Hkv, d * 16), device=cuda), torch.zeros((3, Hkv, d * 16), device=cuda))
               for _ in range(2)]
    pools_h = [(np.zeros((3, Hkv, d * 16), np.float32), np.zeros((3, Hkv, d * 16), np.float32))
               for _ in range(2)]
    inv = rope_inv_freqs(d, 10000.0)
    c = dict(hidden_size=H, num_heads=Hq, num_kv_heads=Hkv, head_dim=d, inter=I, rms_eps=1e-5,
             w_dtype=W_F32, w_group_size=0)
    x_ref = (np.arange(H) * 0.03 - 0.5).astype(np.float32)  # gpu_parity.rs:95-97
    x_dev = torch.from_numpy(x_ref.copy()).to(cuda)
    for step in range(48):  # 3 blocks of 16 tokens
        pos = decode_token(kern, cache, 7, x_dev, pools_d)
        assert pos == step
        table = np.array(cache.block_table(7) + [0] * (4 - len(cache.block_table(7))), np.int32)
        for L in range(2):
            x_ref = oracle.decode_block_paged(c, host[L], x_ref, *pools_h[L], table, pos, pos, inv)
    torch.cuda.synchronize()
    assert float(np.abs(x_dev.cpu().numpy() - x_ref).max()) < 2e-3
    with pytest.raises(KvCacheExhausted):
        decode_token(kern, cache, 7, x_dev, pools_d)
    assert cache.sequence_len(7) == 48


def test_decode_block_rejects_bad_arguments(oracle, cuda):
    """Host checks run before any launch: operand sizes, row widths the
    16-byte loads need, and positions beyond the block table."""
    import torch
    from dlm_amd._lib import DlmkError
    from dlm_amd.block import BlockConfig, PagedGpuKernel

    banner("decode block argument errors")
    pools = (torch.zeros((2, 1, 64 * 16), device=cuda), torch.zeros((2, 1, 64 * 16), device=cuda))
    table = torch.zeros(2, dtype=torch.int32, device=cuda)
    # A weight of the wrong size never reaches a kernel.
    good = to_layer(torch, make_layer(oracle, 1, 64, 1, 1, 64, 64, W_F32), cuda)
    bad = to_layer(torch, make_layer(oracle, 1, 64, 1, 1, 64, 64, W_F32), cuda)
    bad.o_proj = bad.o_proj[:-4]
    with pytest.raises(ValueError):
        PagedGpuKernel(BlockConfig(64, 1, 1, 64, 64), [bad], W_F32, device=cuda)
    # hidden 36 bf16: rows are read 16 bytes (8 elements) at a time.
    lw = to_layer(torch, make_layer(oracle, 1, 36, 1, 1, 64, 64, W_BF16), cuda)
    kern = PagedGpuKernel(BlockConfig(36, 1, 1, 64, 64), [lw], W_BF16, max_blocks_per_seq=2,
                          device=cuda)
    with pytest.raises(DlmkError):
        kern.run_block(0, torch.zeros(36, device=cuda), pools, table, 0, 0)
    # Position 32 needs a third block; the table has two.
    kern = PagedGpuKernel(BlockConfig(64, 1, 1, 64, 64), [good], W_F32, max_blocks_per_seq=2,
                          device=cuda)
    with pytest.raises(DlmkError):
        kern.run_block(0, torch.zeros(64, device=cuda), pools, table, 32, 32)
