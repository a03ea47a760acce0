"""Seeded random-shape parity sweep of paged attention against the oracle.

Each case draws a pool dtype (f16, bf16, f32, int8, int4), head dim, KV heads,
GQA group and verify-query count from the combinations the kernels support,
a batch of 1-10 sequences with contexts from 0 to 2500 tokens, and a block
table wider than the longest context by a random margin, so that the
partition counts -- and with them the split-K combine kernels and the f32
partition sizes -- vary from case to case.  The same tolerances as the
targeted tests apply: 2e-3 abs + 1e-3 rel for f16 / bf16 / int8 / int4 pools
(f16 queries), 1e-5 for f32.
"""
import numpy as np
import pytest

from helpers import (BF16_ATOL, BF16_RTOL, F16_ATOL, F16_RTOL, F32_ATOL, F32_RTOL, assert_close,
                     make_workload, to_dev)

pytestmark = pytest.mark.gpu

BS = 16
MFMA_ROWS = [(1, 1), (1, 2), (1, 4), (2, 1), (2, 2), (2, 4), (4, 1), (4, 2), (4, 4), (8, 1),
             (8, 2), (16, 1)]  # (GQA group, queries per sequence)
VALU_ROWS = [(1, 1), (1, 2), (1, 4), (2, 1), (2, 2), (2, 4), (4, 1), (4, 2), (8, 1)]


def banner(msg):
    print(f"\n[gpu-fuzz] {msg}", flush=True)


def draw_case(seed):
    rng = np.random.default_rng(1000 + seed)
    kind = ["f16", "bf16", "f32", "int8", "int4"][seed % 5]
    d = int(rng.choice([64, 128] if kind == "f32" else [64, 128, 256]))
    gqa, nq = VALU_ROWS[rng.integers(len(VALU_ROWS))] if kind == "f32" else \
        MFMA_ROWS[rng.integers(len(MFMA_ROWS))]
    hkv = int(rng.choice([1, 2, 4, 8]))
    B = int(rng.integers(1, 11))
    ctx = rng.integers(0, 2501, B)
    ctx[rng.random(B) < 0.15] = 0
    ctx = np.maximum(ctx, 0).astype(np.int32)
    extra = int(rng.choice([0, int(rng.integers(1, 600))]))
    return rng, kind, d, gqa * hkv, hkv, nq, ctx, extra


def widen(tables, extra):
    out = np.zeros((tables.shape[0], tables.shape[1] + extra), np.int32)
    out[:, :tables.shape[1]] = tables
    return out


@pytest.mark.parametrize("seed", range(25))
def test_attention_random_shapes(oracle, cuda, seed):
    import torch
    from dlm_amd import ops

    rng, kind, d, hq, hkv, nq, ctx, extra = draw_case(seed)
    banner(f"seed {seed}: {kind} d={d} Hq={hq} Hkv={hkv} nq={nq} ctx={ctx.tolist()} "
           f"extra_blocks={extra}")
    scale = np.float32(1.0) / np.sqrt(np.float32(d))
    if kind in ("f16", "bf16", "f32"):
        dt = {"f16": np.float16, "f32": np.float32, "bf16": "bf16"}[kind]
        w = make_workload(rng, ctx, hq, hkv, d, dt, nq=nq, sigma=1.0 if kind == "f32" else 0.5)
        w.tables = widen(w.tables, extra)
        ref = oracle.paged_attention(w.q, w.k_pool, w.v_pool, w.tables, w.ctx, w.nq, w.Hq, w.Hkv,
                                     w.d, w.bs, w.scale)
        got = ops.paged_decode_attention(
            to_dev(torch, w.q, cuda), to_dev(torch, w.k_pool, cuda), to_dev(torch, w.v_pool, cuda),
            to_dev(torch, w.tables, cuda), to_dev(torch, w.ctx, cuda), num_kv_heads=hkv,
            scale=float(w.scale), out_dtype=torch.float32)
        atol, rtol = {"f16": (F16_ATOL, F16_RTOL), "f32": (F32_ATOL, F32_RTOL),
                      "bf16": (BF16_ATOL, BF16_RTOL)}[kind]
    else:
        quant = oracle.I8 if kind == "int8" else oracle.I4
        need = [-(-int(c) // BS) for c in ctx]
        nb = sum(need) + 4
        perm = rng.permutation(nb)
        tables = np.zeros((len(ctx), max(max(need), 1)), np.int32)
        off = 0
        for s, n in enumerate(need):
            tables[s, :n] = perm[off:off + n]
            off += n
        ks, vs = oracle.quant_pool_shapes(nb, hkv, d, quant)
        kp = rng.integers(0, 256, ks, dtype=np.uint8)  # bytes nobody wrote
        vp = rng.integers(0, 256, vs, dtype=np.uint8)
        ksc = np.full((nb, BS), np.nan, np.float32)
        vsc = np.full((nb, BS), np.nan, np.float32)
        slots = np.array([tables[s, p // BS] * BS + p % BS for s, c in enumerate(ctx)
                          for p in range(int(c))], np.int64)
        n = len(slots)
        k = rng.standard_normal((n, hkv * d)).astype(np.float32)
        v = rng.standard_normal((n, hkv * d)).astype(np.float32)
        if n:
            oracle.paged_append_quant(kp, vp, ksc, vsc, k, v, slots, hkv, d, quant)
        tables = widen(tables, extra)
        q = rng.standard_normal((len(ctx), nq, hq, d)).astype(np.float16)
        ref = oracle.paged_attention_quant(q.astype(np.float32), kp, vp, ksc, vsc, quant, tables,
                                           ctx, nq, hq, hkv, d, scale)
        kv = ops.QuantKv(torch.from_numpy(kp).to(cuda), torch.from_numpy(vp).to(cuda),
                         torch.from_numpy(ksc).to(cuda), torch.from_numpy(vsc).to(cuda), kind)
        got = ops.paged_decode_attention_quant(
            to_dev(torch, q, cuda), kv, to_dev(torch, tables, cuda), to_dev(torch, ctx, cuda),
            num_kv_heads=hkv, scale=float(scale), out_dtype=torch.float32)
        atol, rtol = F16_ATOL, F16_RTOL
    torch.cuda.synchronize()
    assert_close(got.cpu().numpy(), ref, atol, rtol, f"seed {seed} {kind}")
