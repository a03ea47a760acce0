"""Fused decode step (dlmk_paged_decode_step) against its definition:
dlmk_kv_append of the newest num_q_per_seq tokens followed by
dlmk_paged_decode_attention.  Pools and outputs must be bitwise identical, and
both must match the oracle (append bit-exact, attention within tolerance)."""
import numpy as np
import pytest

from helpers import (BF16_ATOL, BF16_RTOL, F16_ATOL, F16_RTOL, F32_ATOL, F32_RTOL, assert_close,
                     make_workload, to_dev)

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,Hq,Hkv,d,nq,ctx", [
    (np.float16, 32, 8, 128, 1, [1, 16, 17, 512, 513, 4096, 700]),   # 8B shape decode
    (np.float16, 32, 8, 128, 4, [2, 4, 510, 513, 515, 1000]),        # verify, drafts across a partition edge
    (np.float16, 64, 8, 128, 1, [3000, 33]),                         # 70B shape
    (np.float32, 32, 8, 64, 1, [544, 1, 257]),                       # config-1 shape (VALU kernel)
    (np.float32, 16, 8, 64, 4, [3, 258, 600]),
    ("bf16", 32, 8, 128, 2, [2, 600, 1025]),
    (np.float32, 4, 2, 8, 1, [1, 16, 17, 40]),                       # generic kernel, head_dim 8
    (np.float32, 32, 8, 128, 2, [2, 300, 2049]),
    (np.float16, 32, 8, 96, 2, [2, 17, 1100]),                       # generic f16, head_dim 96
    (np.float16, 64, 8, 128, 4, [4, 513, 1030]),                     # two row groups
])
def test_fused_step_equals_append_then_attention(oracle, cuda, dtype, Hq, Hkv, d, nq, ctx):
    import torch
    from dlm_amd import ops
    name = dtype if isinstance(dtype, str) else np.dtype(dtype).name
    print(f"[gpu-test] fused step {name} Hq={Hq} Hkv={Hkv} d={d} nq={nq} ctx={ctx}", flush=True)
    rng = np.random.default_rng(len(ctx) * 7 + nq)
    sigma = 1.0 if dtype is np.float32 else 0.5
    w = make_workload(rng, ctx, Hq, Hkv, d, dtype, nq=nq, sigma=sigma)
    B = len(ctx)
    newk = make_workload(rng, [nq] * B, 1, Hkv, d, dtype, nq=1, sigma=sigma)  # donor of new tokens
    # new tokens [B][nq][Hkv][d] taken from the donor's logical view, same dtype bits
    npdt = w.k_pool.dtype
    k_new = np.zeros((B, nq, Hkv, d), npdt)
    v_new = np.zeros((B, nq, Hkv, d), npdt)
    X = 16 // npdt.itemsize
    for s in range(B):
        for j in range(nq):
            blk, t = newk.tables[s, j // 16], j % 16
            k_new[s, j] = newk.k_pool[blk, :, :, t, :].reshape(Hkv, d)
            v_new[s, j] = newk.v_pool[blk, :, :, t]
    slots, src = [], []
    for s, c in enumerate(ctx):
        for j in range(nq):
            p = c - nq + j
            if p >= 0:
                slots.append(int(w.tables[s, p // 16]) * 16 + p % 16)
                src.append((s, j))
    slots = np.array(slots, np.int64)
    ks = np.stack([k_new[s, j] for s, j in src]) if src else np.zeros((0, Hkv, d), npdt)
    vs = np.stack([v_new[s, j] for s, j in src]) if src else np.zeros((0, Hkv, d), npdt)

    dv = lambda a: to_dev(torch, a, cuda)
    kA, vA, kB, vB = dv(w.k_pool), dv(w.v_pool), dv(w.k_pool), dv(w.v_pool)
    tables, lens, q = dv(w.tables), dv(w.ctx), dv(w.q)
    ops.kv_append(kA, vA, dv(ks), dv(vs), dv(slots), num_kv_heads=Hkv, head_dim=d)
    outA = ops.paged_decode_attention(q, kA, vA, tables, lens, num_kv_heads=Hkv,
                                      out_dtype=torch.float32)
    outB = ops.paged_decode_step(q, dv(k_new), dv(v_new), kB, vB, tables, lens, num_kv_heads=Hkv,
                                 out_dtype=torch.float32)
    torch.cuda.synchronize()
    raw = lambda t: t.view(torch.int16).cpu().numpy() if t.element_size() == 2 else t.cpu().numpy()
    assert np.array_equal(raw(kA), raw(kB)) and np.array_equal(raw(vA), raw(vB)), "pools differ"
    assert torch.equal(outA, outB), "fused output differs from append + attention"

    oracle.paged_append(w.k_pool, w.v_pool, ks, vs, slots, Hkv, d, 16)
    assert np.array_equal(raw(kB).view(np.uint8), w.k_pool.view(np.uint8))
    ref = oracle.paged_attention(w.q, w.k_pool, w.v_pool, w.tables, w.ctx, nq, Hq, Hkv, d, 16,
                                 w.scale)
    atol, rtol = {"float16": (F16_ATOL, F16_RTOL), "float32": (F32_ATOL, F32_RTOL),
                  "bf16": (BF16_ATOL, BF16_RTOL)}[name]
    assert_close(outB.cpu().numpy(), ref, atol, rtol, "fused step vs oracle")
