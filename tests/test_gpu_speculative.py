"""Batched verify block and speculative rounds on the GPU.

dlmk_verify_block_paged (n tokens through a layer in one pass) against the
CPU oracle's decode_block run one token at a time over the same paged pools
(dlm verifies sequentially, src/speculative.rs:133-141, decode_block
src/forward/cpu.rs:1156-1219), at the decode block's tolerances (1e-3, 2e-3
for int8 weights and wide layers; gpu_parity.rs:114-116, :183, :237).

Speculative rounds (dlm_amd.speculative) over the paged path against
target-greedy decoding computed by the oracle, with the reference's own test
models (tests/speculative.rs:29-64: 1 layer, hidden 16, 4/2 heads, head_dim
4, inter 32, vocab 32, SplitMix64 weights * 0.05, unit norms, target seed 1,
draft seed 2) and its properties (speculative.rs:77-171): output == target
greedy, an identical draft is fully accepted, round-by-round sessions respect
the budget, the scheduler (max_batch 2, staggered admission) matches greedy
per request and stops at EOS.  A 2-layer head_dim-64 model with a perturbed draft adds
mixed acceptance and rollbacks across block boundaries.
"""
import numpy as np
import pytest

from test_gpu_block import W_BF16, W_F32, W_INT8, make_layer, to_layer

pytestmark = pytest.mark.gpu


def banner(msg):
    print(f"\n[gpu-spec] {msg}", flush=True)


VERIFY_CASES = [
    # name, (hidden, heads, kv heads, head_dim, inter), w_dtype, n tokens, tol
    ("f32-n2", (256, 4, 2, 64, 512), W_F32, 2, 1e-3),
    ("f32-n5", (256, 4, 2, 64, 512), W_F32, 5, 1e-3),
    ("f32-n8", (256, 4, 2, 64, 512), W_F32, 8, 1e-3),
    ("f32-n11", (256, 4, 2, 64, 512), W_F32, 11, 1e-3),   # launches of 8 + 3 tokens
    ("bf16-n5-gqa4", (512, 8, 2, 64, 1024), W_BF16, 5, 1e-3),
    ("int8-n4", (256, 4, 2, 64, 512), W_INT8, 4, 2e-3),
    ("wide-inter-n3", (512, 8, 2, 64, 12288), W_F32, 3, 2e-3),  # down_proj one token a launch
    ("hidden2048-n5", (2048, 16, 4, 128, 512), W_F32, 5, 2e-3),
    ("speculative-model-n5", (16, 4, 2, 4, 32), W_F32, 5, 1e-3),
    ("gpu_parity-d8-n3", (32, 4, 2, 8, 64), W_F32, 3, 1e-3),
    # Long histories: several split-K partitions and the combine launch;
    # gqa16 x 5 tokens is 5 row groups of 16 rows.
    ("f32-n2-hist500", (256, 4, 2, 64, 512), W_F32, 2, 1e-3, 500, 40),
    ("f32-n5-hist600", (256, 4, 2, 64, 512), W_F32, 5, 1e-3, 600, 48),
    ("hidden2048-n5-hist900", (2048, 16, 4, 128, 512), W_F32, 5, 2e-3, 900, 64),
    ("gqa16-n5-hist300", (1024, 16, 1, 64, 512), W_F32, 5, 1e-3, 300, 32),
]


@pytest.mark.parametrize("name,shape,w_dtype,n,tol,hist,max_blocks",
                         [c if len(c) == 7 else c + (13, 4) for c in VERIFY_CASES],
                         ids=[c[0] for c in VERIFY_CASES])
def test_verify_block_matches_sequential_oracle(oracle, cuda, name, shape, w_dtype, n, tol, hist,
                                                max_blocks):
    """hist 13: 13 + n crosses the first block boundary for n >= 4."""
    import torch
    from dlm_amd.block import BlockConfig, PagedGpuKernel, rope_inv_freqs

    H, Hq, Hkv, d, I = shape
    banner(f"verify block {name}: hidden={H} heads={Hq}/{Hkv} d={d} inter={I} n={n} hist={hist}")
    cfg = BlockConfig(H, Hq, Hkv, d, I)
    gs = 128 if w_dtype == W_INT8 else 0
    host = [make_layer(oracle, 41 + L, H, Hq, Hkv, d, I, w_dtype) for L in range(2)]
    kern = PagedGpuKernel(cfg, [to_layer(torch, w, cuda) for w in host], w_dtype, gs,
                          max_blocks_per_seq=max_blocks, device=cuda)
    inv = rope_inv_freqs(d, 10000.0)
    used = (hist + n + 15) // 16
    nb = used + 7
    rng = np.random.default_rng(n)
    table = np.zeros(max_blocks, np.int32)
    table[:used] = rng.permutation(nb)[:used]
    pools_h = []
    for L in range(2):
        kp = np.zeros((nb, Hkv, d * 16), np.float32)
        vp = np.zeros((nb, Hkv, d * 16), np.float32)
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
    x = (rng.uniform(-0.5, 0.5, (n, H))).astype(np.float32)
    x_dev = torch.from_numpy(x.copy()).to(cuda)
    kern.verify_workspace(n).fill_(0x7f)  # the block must not rely on a zeroed workspace
    for L in range(2):
        kern.run_tokens(L, x_dev, pools_d[L], table_d, hist, hist)
    ref = np.empty_like(x)
    for j in range(n):  # the reference's way: one token at a time, every layer
        xr = x[j].copy()
        for L in range(2):
            xr = oracle.decode_block_paged(c, host[L], xr, pools_h[L][0], pools_h[L][1], table,
                                           hist + j, hist + j, inv)
        ref[j] = xr
    torch.cuda.synchronize()
    got = x_dev.cpu().numpy()
    err = np.abs(got - ref).max(axis=1)
    assert err.max() < tol, f"{name}: per-token max errors {err}"
    for L in range(2):
        for dev_pool, host_pool in zip(pools_d[L], pools_h[L]):
            np.testing.assert_allclose(dev_pool.cpu().numpy(), host_pool, atol=tol, rtol=0)


# --------------------------------------------------------------- models

def reference_model(oracle, seed, hidden=16, heads=4, kv_heads=2, head_dim=4, inter=32, vocab=32):
    """build_generator (tests/speculative.rs:30-64): one SplitMix64 stream
    drawn in the order q, k, v, o, gate, up, down, embedding, lm_head."""
    qd, kvd = heads * head_dim, kv_heads * head_dim
    sizes = [("q_proj", qd * hidden), ("k_proj", kvd * hidden), ("v_proj", kvd * hidden),
             ("o_proj", hidden * qd), ("gate_proj", inter * hidden), ("up_proj", inter * hidden),
             ("down_proj", hidden * inter), ("embedding", vocab * hidden),
             ("lm_head", vocab * hidden)]
    stream = oracle.rng_uniform(seed, sum(n for _, n in sizes), 0.05)
    m, off = {}, 0
    for name, n in sizes:
        m[name] = stream[off:off + n].copy()
        off += n
    m["in_norm"] = np.ones(hidden, np.float32)
    m["post_norm"] = np.ones(hidden, np.float32)
    shape = (hidden, heads, kv_heads, head_dim, inter, vocab)
    return shape, [m]


def perturbed_model(oracle, seed, base_seed, noise, shape=(256, 4, 2, 64, 512, 64), layers=2):
    """A multi-layer model (seed base_seed) whose weights are moved by
    noise * a second stream (seed): noise 0 is the same model."""
    H, Hq, Hkv, d, I, V = shape
    out = []
    for L in range(layers):
        m = make_layer(oracle, base_seed * 10 + L, H, Hq, Hkv, d, I, W_F32)
        for i, k in enumerate(("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj",
                               "down_proj")):
            m[k] = m[k] + np.float32(noise) * oracle.rng_uniform(seed * 1000 + L * 10 + i,
                                                                 m[k].size, 0.05)
        out.append(m)
    emb = oracle.rng_uniform(base_seed * 7 + 1, V * H, 0.5)
    head = oracle.rng_uniform(base_seed * 7 + 2, V * H, 0.5)
    head = head + np.float32(noise) * oracle.rng_uniform(seed * 7 + 3, V * H, 0.5)
    out[0]["embedding"], out[0]["lm_head"] = emb, head
    return shape, out


def gpu_generator(torch, cuda, shape, layers, max_blocks, total_blocks, seed):
    from dlm_amd.block import BlockConfig, PagedGpuKernel
    from dlm_amd.speculative import PagedGenerator
    H, Hq, Hkv, d, I, V = shape
    kern = PagedGpuKernel(BlockConfig(H, Hq, Hkv, d, I), [to_layer(torch, m, cuda) for m in layers],
                          W_F32, max_blocks_per_seq=max_blocks, device=cuda)
    return PagedGenerator(kern, layers[0]["embedding"], np.ones(H, np.float32),
                          layers[0]["lm_head"], V, 1e-5, total_blocks, seed)


def oracle_greedy(oracle, shape, layers, prompt, n):
    """Target-greedy decoding on the oracle: the prompt, then n tokens, each
    through every layer's decode_block at its position (Generator::generate,
    src/generate.rs:338-380).  Logits in f64.  Returns (tokens, the smallest
    top-1 / top-2 logit gap seen)."""
    from dlm_amd.block import rope_inv_freqs
    H, Hq, Hkv, d, I, V = shape
    inv = rope_inv_freqs(d, 10000.0)
    c = dict(hidden_size=H, num_heads=Hq, num_kv_heads=Hkv, head_dim=d, inter=I, rms_eps=1e-5,
             w_dtype=W_F32, w_group_size=0)
    nb = -(-(len(prompt) + n) // 16)
    pools = [(np.zeros((nb, Hkv, d * 16), np.float32), np.zeros((nb, Hkv, d * 16), np.float32))
             for _ in layers]
    table = np.arange(nb, dtype=np.int32)
    emb = layers[0]["embedding"].reshape(V, H)
    head = layers[0]["lm_head"].reshape(V, H).astype(np.float64)
    pos, x, out, gap = 0, None, [], np.inf

    def feed(tok):
        nonlocal pos
        xr = emb[tok].copy()
        for L, m in enumerate(layers):
            xr = oracle.decode_block_paged(c, m, xr, pools[L][0], pools[L][1], table, pos, pos, inv)
        pos += 1
        return xr

    for t in prompt:
        x = feed(t)
    for _ in range(n):
        xd = x.astype(np.float64)
        normed = xd / np.sqrt((xd * xd).mean() + 1e-5)
        logits = head @ normed
        top = np.sort(logits)[-2:]
        gap = min(gap, float(top[1] - top[0]))
        tok = int(np.argmax(logits))
        out.append(tok)
        x = feed(tok)
    return out, gap


def test_speculative_reference_models_equal_target_greedy(oracle, cuda):
    """tests/speculative.rs:77-107 on the reference's own models, over the
    paged GPU path: draft seed 2 against target seed 1, and an identical
    draft fully accepted; gamma 1 and 4; several prompts."""
    import torch
    from dlm_amd.speculative import SpeculativeDecoder
    banner("speculative rounds: reference models (hidden 16, head_dim 4, vocab 32)")
    shape, t_layers = reference_model(oracle, 1)
    _, d_layers = reference_model(oracle, 2)
    target = gpu_generator(torch, cuda, shape, t_layers, 8, 24, seed=11)
    draft = gpu_generator(torch, cuda, shape, d_layers, 8, 24, seed=12)
    same = gpu_generator(torch, cuda, shape, t_layers, 8, 24, seed=13)
    for prompt, n in (([1, 2, 3], 8), ([5, 6], 6), ([7], 5), ([4, 5], 30)):
        ref, gap = oracle_greedy(oracle, shape, t_layers, prompt, n)
        assert gap > 1e-6, f"prompt {prompt}: ambiguous greedy choice (gap {gap:.2e})"
        assert target.generate(prompt, n) == ref, f"prompt {prompt}: paged greedy diverged"
        for gamma in (1, 4):
            dec = SpeculativeDecoder(target, draft, gamma)
            assert dec.generate(prompt, n) == ref, f"prompt {prompt} gamma {gamma}: diverged"
            assert len(ref) == n and dec.accepted <= dec.proposed
            full = SpeculativeDecoder(target, same, gamma)
            assert full.generate(prompt, n) == ref
            assert full.proposed > 0 and full.accepted == full.proposed
    for g in (target, draft, same):  # every session released its blocks
        assert g.cache.num_sequences() == 0 and g.cache.free_blocks() == g.cache.total_blocks()


def test_speculative_session_rounds_with_rollback(oracle, cuda):
    """tests/speculative.rs:109-131 round by round on a 2-layer head_dim-64
    model with a perturbed draft (mixed acceptance): every round emits
    1..=gamma+1 tokens within the budget, both books are rolled back to the
    sequence minus its last token (rollbacks cross block boundaries), and the
    output equals the oracle's target greedy."""
    import torch
    from dlm_amd.speculative import SpeculativeSession
    banner("speculative session: 2 layers, d 64, perturbed draft")
    shape, t_layers = perturbed_model(oracle, 0, base_seed=3, noise=0.0)
    _, d_layers = perturbed_model(oracle, 5, base_seed=3, noise=0.35)
    target = gpu_generator(torch, cuda, shape, t_layers, 8, 40, seed=21)
    draft = gpu_generator(torch, cuda, shape, d_layers, 8, 40, seed=22)
    prompt, n = [3, 1, 4, 1, 5, 9, 2, 6, 5, 3, 5, 8, 9], 60
    ref, gap = oracle_greedy(oracle, shape, t_layers, prompt, n)
    assert gap > 1e-5, f"ambiguous greedy choice (gap {gap:.2e})"
    for gamma in (4, 3):
        s = SpeculativeSession(target, draft, gamma, prompt)
        out, rounds, partial = [], 0, 0
        while len(out) < n:
            emitted = s.step(n - len(out))
            assert 1 <= len(emitted) <= min(gamma + 1, n - len(out))
            partial += len(emitted) < gamma + 1
            out.extend(emitted)
            rounds += 1
            held = len(s.seq) - 1
            assert target.cache.sequence_len(s.t_seq) == held
            assert draft.cache.sequence_len(s.d_seq) == held
            assert len(target.cache.block_table(s.t_seq)) == -(-held // 16)
        assert out == ref, f"gamma {gamma}: speculative diverged from target greedy"
        assert 0 < s.accepted < s.proposed and partial > 0, (s.accepted, s.proposed)
        assert rounds < n  # fewer target passes than tokens
        banner(f"gamma {gamma}: {rounds} rounds for {n} tokens, "
               f"acceptance {s.accepted}/{s.proposed}")
        s.close()
    assert target.cache.free_blocks() == target.cache.total_blocks()


def test_speculative_scheduler_reference_models(oracle, cuda):
    """tests/speculative.rs:133-171 on the reference's models over the paged
    path: max_batch 2 forces staggered admission while speculating, every
    request equals its target greedy; then an identical draft stops at EOS
    (included), as plain decoding does."""
    import torch
    from dlm_amd.speculative import SpeculativeScheduler
    banner("speculative scheduler: reference models")
    shape, t_layers = reference_model(oracle, 1)
    _, d_layers = reference_model(oracle, 2)
    target = gpu_generator(torch, cuda, shape, t_layers, 8, 24, seed=31)
    draft = gpu_generator(torch, cuda, shape, d_layers, 8, 24, seed=32)
    reqs = [(1, [1, 2, 3], 7), (2, [7], 5), (3, [4, 5], 6)]
    sched = SpeculativeScheduler(target, draft, 2, 4)
    for rid, prompt, n in reqs:
        sched.submit(rid, prompt, n)
    results = dict(sched.run())
    assert set(results) == {1, 2, 3}
    for rid, prompt, n in reqs:
        ref, gap = oracle_greedy(oracle, shape, t_layers, prompt, n)
        assert gap > 1e-6
        assert results[rid] == ref, f"request {rid} diverged"
    proposed, accepted = sched.speculative_stats()
    assert proposed > 0 and accepted <= proposed
    # EOS: the token plain decoding emits second (speculative.rs:157-171).
    same = gpu_generator(torch, cuda, shape, t_layers, 8, 24, seed=33)
    two, _ = oracle_greedy(oracle, shape, t_layers, [1, 2], 2)
    sched = SpeculativeScheduler(target, same, 4, 4)
    sched.submit(1, [1, 2], 10, [two[1]])
    (rid, toks), = sched.run()
    assert rid == 1 and toks[-1] == two[1] and toks == two[:len(toks)]
    for g in (target, draft, same):
        assert g.cache.num_sequences() == 0
