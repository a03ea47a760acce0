"""Shared builders for the GPU parity tests: seeded paged workloads that exist
both as NumPy arrays (for the oracle) and as device tensors (for libdlmk)."""
from dataclasses import dataclass

import numpy as np

F16_ATOL, F16_RTOL = 2e-3, 1e-3  # tolerance stated for f16 KV
F32_ATOL, F32_RTOL = 1e-5, 1e-5  # tolerance stated for f32 KV


def assert_close(got, ref, atol, rtol, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    bad = err > bound
    assert not bad.any(), (f"{what}: {bad.sum()} of {bad.size} outside atol={atol} rtol={rtol}; "
                           f"max abs err {err.max():.3e} at {np.unravel_index(err.argmax(), err.shape)}")


@dataclass
class Workload:
    """A batch of sequences laid out in shuffled physical blocks."""

    k_pool: np.ndarray
    v_pool: np.ndarray
    tables: np.ndarray  # int32 [B, max_blocks]
    ctx: np.ndarray  # int32 [B]
    q: np.ndarray  # [B, nq, Hq, d]
    Hq: int
    Hkv: int
    d: int
    nq: int
    bs: int = 16

    @property
    def scale(self):
        return np.float32(1.0) / np.sqrt(np.float32(self.d))


BF16_ATOL, BF16_RTOL = 1.6e-2, 8e-3  # bf16 KV: 8x the f16 bound (3 fewer mantissa bits)


def _bf16(a):
    from oracle.oracle import bf16_bits
    return bf16_bits(a)


def make_workload(rng, ctx, Hq, Hkv, d, dtype, nq=1, sigma=1.0, num_blocks=None, spare=8,
                  fill_nan=False, bs=16):
    """Pools filled through the logical view: token p of seq s at table[s][p//bs].

    dtype "bf16" stores bf16 bit patterns in uint16 arrays (NumPy has no bf16)."""
    if isinstance(dtype, str) and dtype == "bf16":
        w = make_workload(rng, ctx, Hq, Hkv, d, np.float32, nq, sigma, num_blocks, spare,
                          fill_nan, bs)
        X = 8
        nb = w.k_pool.shape[0]
        # re-chunk K for 8-element (16-byte) bf16 chunks: [nb][Hkv][d/4][bs][4] -> logical -> [d/8][bs][8]
        k = w.k_pool.transpose(0, 1, 3, 2, 4).reshape(nb, Hkv, bs, d)
        k = k.reshape(nb, Hkv, bs, d // X, X).transpose(0, 1, 3, 2, 4)
        w.k_pool = _bf16(np.ascontiguousarray(k))
        w.v_pool = _bf16(w.v_pool)
        w.q = _bf16(w.q)
        return w
    ctx = np.asarray(ctx, np.int32)
    B = len(ctx)
    need = [-(-int(c) // bs) for c in ctx]
    max_blocks = max(max(need), 1)
    total = sum(need) + spare
    num_blocks = num_blocks or total
    X = 16 // np.dtype(dtype).itemsize
    if fill_nan:
        k_pool = np.full((num_blocks, Hkv, d // X, bs, X), np.nan, dtype)
        v_pool = np.full((num_blocks, Hkv, d, bs), np.nan, dtype)
    else:
        k_pool = (rng.standard_normal((num_blocks, Hkv, d // X, bs, X)) * sigma).astype(dtype)
        v_pool = (rng.standard_normal((num_blocks, Hkv, d, bs)) * sigma).astype(dtype)
    perm = rng.permutation(num_blocks)
    tables = np.zeros((B, max_blocks), np.int32)
    off = 0
    for s, n in enumerate(need):
        tables[s, :n] = perm[off:off + n]
        off += n
    if fill_nan:
        # Only the visible tokens get finite values; block tails stay NaN.
        for s, c in enumerate(ctx):
            for p in range(int(c)):
                blk, t = tables[s, p // bs], p % bs
                k_pool[blk, :, :, t, :] = (rng.standard_normal((Hkv, d // X, X)) * sigma)
                v_pool[blk, :, :, t] = (rng.standard_normal((Hkv, d)) * sigma)
    q = (rng.standard_normal((B, nq, Hq, d)) * sigma).astype(dtype)
    return Workload(k_pool, v_pool, tables, ctx, q, Hq, Hkv, d, nq, bs)


def to_dev(torch, arr, device):
    """NumPy -> device tensor; uint16 arrays become bfloat16 (bit patterns kept)."""
    arr = np.ascontiguousarray(arr)
    if arr.dtype == np.uint16:
        return torch.from_numpy(arr.view(np.int16)).to(device).view(torch.bfloat16)
    return torch.from_numpy(arr).to(device)
