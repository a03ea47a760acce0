"""GPU parity for the int8 / int4 KV pools (dlm's --kv-quant, KvLayerCache at
src/forward/cpu.rs:622-846).  Quantizing append is bit-exact against the oracle
(codes and scales); attention over quantized pools is within 2e-3 abs + 1e-3
rel of the oracle's f32 restatement (the kernel rounds q and code * scale to
f16 operands, as the f16-pool path rounds its stored values)."""
import numpy as np
import pytest

from helpers import F16_ATOL, F16_RTOL, assert_close, to_dev

pytestmark = pytest.mark.gpu

BS = 16


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


def _quant(oracle, name):
    return oracle.I8 if name == "int8" else oracle.I4


def layout(rng, ctx, spare=8):
    """Shuffled block tables for lengths ctx, and every token's slot."""
    need = [-(-int(c) // BS) for c in ctx]
    nb = sum(need) + spare
    perm = rng.permutation(nb)
    tables = np.zeros((len(ctx), max(max(need), 1)), np.int32)
    off = 0
    for s, n in enumerate(need):
        tables[s, :n] = perm[off:off + n]
        off += n
    slots = np.array([tables[s, p // BS] * BS + p % BS for s, c in enumerate(ctx)
                      for p in range(int(c))], np.int64)
    return nb, tables, slots


def tokens(rng, n, Hkv, d, outliers=True):
    x = rng.standard_normal((n, Hkv, d)).astype(np.float32)
    if outliers and n:
        x[rng.integers(0, n, max(1, n // 50))] *= 8.0  # a few large-norm tokens
    return x


def halfway_rows(rng, x, rows, qmax):
    """Tokens whose quotients x / scale sit on or within a few ulps of the
    half-integers, where the append's reciprocal-multiply rounding test must
    fall back to the division (scale = max / qmax, with the max in element 0)."""
    for r in rows:
        flat = x[r].reshape(-1)
        mx = np.float32(rng.uniform(0.5, 3.0))
        scale = np.float32(mx / np.float32(qmax))
        k = rng.integers(-qmax, qmax, flat.size)
        vals = (k + 0.5).astype(np.float32) * scale
        for step in (-2, -1, 1, 2):  # nudge some by a few ulps either way
            sel = rng.random(flat.size) < 0.15
            toward = np.float32(np.inf) if step > 0 else np.float32(-np.inf)
            for _ in range(abs(step)):
                vals[sel] = np.nextafter(vals[sel], toward)
        vals[0] = mx
        flat[:] = vals


def tie_rows(rng, x, rows, qmax):
    """Tokens whose quotients are exact half-integers (scale a power of two:
    max = qmax / 8, so scale = 1/8 and x = (k + 1/2) / 8, exact in f16 and
    bf16), some nudged by one f16 ulp: round half away from zero and its
    neighbours, for every source dtype."""
    for r in rows:
        flat = x[r].reshape(-1)
        k = rng.integers(-qmax, qmax, flat.size)
        vals = ((k + 0.5) / 8.0).astype(np.float16)
        for toward in (np.float16(np.inf), np.float16(-np.inf)):
            sel = rng.random(flat.size) < 0.2
            vals[sel] = np.nextafter(vals[sel], toward)
        vals[0] = np.float16(qmax / 8.0)
        flat[:] = vals.astype(np.float32)


def garbage_pools(rng, oracle, nb, Hkv, d, quant):
    """Pools holding random bytes and NaN scales: slots nobody wrote."""
    ks, vs = oracle.quant_pool_shapes(nb, Hkv, d, quant)
    kp = rng.integers(0, 256, ks, dtype=np.uint8)
    vp = rng.integers(0, 256, vs, dtype=np.uint8)
    ksc = np.full((nb, BS), np.nan, np.float32)
    vsc = np.full((nb, BS), np.nan, np.float32)
    return kp, vp, ksc, vsc


def upload(torch, ops, cuda, kp, vp, ksc, vsc, qname):
    return ops.QuantKv(torch.from_numpy(kp.copy()).to(cuda), torch.from_numpy(vp.copy()).to(cuda),
                       torch.from_numpy(ksc.copy()).to(cuda), torch.from_numpy(vsc.copy()).to(cuda),
                       qname)


def src_dev(torch, x, src, cuda):
    """Token source on the device in src dtype, and its exact f32 value."""
    if src == "f32":
        return to_dev(torch, x, cuda), x
    if src == "f16":
        h = x.astype(np.float16)
        return to_dev(torch, h, cuda), h.astype(np.float32)
    from oracle.oracle import bf16_bits, bf16_to_f32
    b = bf16_bits(x)
    return to_dev(torch, b, cuda), bf16_to_f32(b)


def assert_pools_equal(kv, kp, vp, ksc, vsc, what):
    got = [kv.k.cpu().numpy(), kv.v.cpu().numpy(), kv.k_scales.cpu().numpy(),
           kv.v_scales.cpu().numpy()]
    for g, r, nm in zip(got, (kp, vp, ksc, vsc), ("K codes", "V codes", "K scales", "V scales")):
        same = (g.view(np.uint8) == r.view(np.uint8))
        assert same.all(), f"{what}: {nm} differ at {(~same).sum()} bytes"


# ------------------------------------------------------------------ append

@pytest.mark.parametrize("qname", ["int8", "int4"])
@pytest.mark.parametrize("src,Hkv,d,ntok,ordered", [
    ("f32", 8, 64, 200, False),    # config-1 geometry
    ("f16", 8, 128, 700, False),   # config-2 geometry, prefill chunk + decode tokens
    ("bf16", 2, 256, 90, False),
    ("f16", 1, 64, 33, False),     # one head, smallest head dim
    # tokens in sequence order: waves whose 4 tokens fill a block's quad
    # (transposed V words) next to waves broken by skipped slots
    ("f16", 8, 128, 700, True),    # kv_dim 1024
    ("f32", 8, 64, 600, True),     # kv_dim 512
    ("bf16", 4, 128, 530, True),   # kv_dim 512, ragged last run
    ("f32", 2, 64, 80, True),      # kv_dim 128: one chunk per lane
    ("f32", 4, 64, 130, True),     # kv_dim 256
    ("f16", 16, 64, 66, True),     # kv_dim 1024 at d 64 (int4: 4-dim V lane groups)
])
def test_kv_append_quant_bit_exact(oracle, torch_mod, ops, cuda, qname, src, Hkv, d, ntok, ordered):
    torch = torch_mod
    banner(f"kv_append_quant {qname} src={src} Hkv={Hkv} d={d} ntok={ntok} ordered={ordered}")
    quant = _quant(oracle, qname)
    rng = np.random.default_rng(7 * ntok + d)
    nb, _, slots = layout(rng, [ntok])
    if not ordered:
        slots = slots[rng.permutation(ntok)]  # tokens land in any order
    slots[::29] = -1                      # skipped tokens
    slots[5] = nb * BS + 3                # out-of-pool slot: skipped
    k = tokens(rng, ntok, Hkv, d)
    v = tokens(rng, ntok, Hkv, d)
    qmax = 127 if qname == "int8" else 7
    halfway_rows(rng, k, [10, 11], qmax)
    halfway_rows(rng, v, [12, 13], qmax)
    tie_rows(rng, k, [14, 15], qmax)
    tie_rows(rng, v, [16, 17], qmax)
    for base in ((0, 32) if ntok >= 64 else (0,)):
        # Also inside the run of tokens 32..47, which fills a whole block when
        # ordered (no skipped or out-of-pool slot there).
        k[base + 3] = 0.0                 # all-zero token: scale 0, codes 0
        v[base + 4] = 0.0
        k[base + 6, 0, 1] = np.nan        # NaN element: skipped by the max, code 0
        v[base + 7, 0, 2] = np.inf        # inf element: scale inf, every code 0
        if base:
            halfway_rows(rng, k, [base + 8], qmax)
            halfway_rows(rng, v, [base + 9], qmax)
            tie_rows(rng, k, [base + 10], qmax)
            tie_rows(rng, v, [base + 11], qmax)
    kd, kf = src_dev(torch, k, src, cuda)
    vd, vf = src_dev(torch, v, src, cuda)
    kp, vp, ksc, vsc = garbage_pools(rng, oracle, nb, Hkv, d, quant)
    kv = upload(torch, ops, cuda, kp, vp, ksc, vsc, qname)
    oracle.paged_append_quant(kp, vp, ksc, vsc, kf.reshape(ntok, -1), vf.reshape(ntok, -1), slots,
                              Hkv, d, quant)
    ops.kv_append_quant(kv, kd, vd, torch.from_numpy(slots).to(cuda), num_kv_heads=Hkv,
                        head_dim=d)
    torch.cuda.synchronize()
    assert_pools_equal(kv, kp, vp, ksc, vsc, f"{qname}/{src}")
    # all-zero tokens stored scale 0 exactly
    if slots[3] >= 0:
        assert ksc.reshape(-1)[slots[3]] == 0.0


def test_kv_append_quant_rejects_bad_shapes(torch_mod, ops, cuda):
    torch = torch_mod
    kv = ops.alloc_quant_pools(4, 2, 64, "int8", cuda)
    k = torch.zeros((3, 2, 64), dtype=torch.float16, device=cuda)
    with pytest.raises(ValueError):
        ops.kv_append_quant(kv, k, k, torch.zeros(2, dtype=torch.int64, device=cuda),
                            num_kv_heads=2, head_dim=64)
    with pytest.raises(ValueError):
        ops.kv_append_quant(kv, k, k, torch.zeros(3, dtype=torch.int64, device=cuda),
                            num_kv_heads=2, head_dim=128)
    with pytest.raises(ValueError):  # the 16-byte tiles need head_dim % 64 == 0
        ops.alloc_quant_pools(4, 2, 32, "int4", cuda)
    from dlm_amd._lib import DlmkError, check, lib
    k32 = torch.zeros((3, 2, 32), dtype=torch.float16, device=cuda)
    with pytest.raises(DlmkError):
        check(lib().dlmk_kv_append_quant(None, kv.k.data_ptr(), kv.v.data_ptr(),
                                         kv.k_scales.data_ptr(), kv.v_scales.data_ptr(),
                                         k32.data_ptr(), k32.data_ptr(), 1,
                                         torch.zeros(3, dtype=torch.int64, device=cuda).data_ptr(),
                                         3, 2, 32, 16, 4, 3))


# --------------------------------------------------------------- attention

def quant_workload(oracle, rng, ctx, Hkv, d, quant):
    nb, tables, slots = layout(rng, ctx)
    kp, vp, ksc, vsc = garbage_pools(rng, oracle, nb, Hkv, d, quant)
    n = len(slots)
    oracle.paged_append_quant(kp, vp, ksc, vsc, tokens(rng, n, Hkv, d).reshape(n, -1),
                              tokens(rng, n, Hkv, d).reshape(n, -1), slots, Hkv, d, quant)
    return kp, vp, ksc, vsc, tables


@pytest.mark.parametrize("qname", ["int8", "int4"])
@pytest.mark.parametrize("ctx,Hq,Hkv,d,nq", [
    ([1, 17, 300, 64], 32, 8, 64, 1),        # config-1 heads, ragged
    ([700, 1, 1300, 513, 2100], 32, 8, 128, 1),  # split over 1024-token partitions
    ([2100, 45], 64, 8, 128, 1),             # GQA 8
    ([600, 4, 90], 16, 4, 128, 4),           # 4-query verify
    ([777, 16], 32, 2, 256, 1),              # GQA 16, d 256
    ([333], 8, 8, 64, 2),                    # MHA, 2 queries
    # Groups of up to 8 rows run the packed kernel (several blocks per score tile):
    ([900, 20, 1500], 32, 8, 128, 2),        # GQA 4 x 2 queries: 8 rows, 2 blocks a tile (int4)
    ([640, 33], 16, 8, 64, 2),               # GQA 2 x 2 queries: 4 rows, d 64
    ([1100, 7], 8, 8, 256, 4),               # GQA 1 x 4 queries: 4 rows, d 256
    ([1030, 300], 64, 8, 64, 1),             # GQA 8 at d 64 (int4: 8-byte code loads)
])
def test_attention_quant_matches_oracle(oracle, torch_mod, ops, cuda, qname, ctx, Hq, Hkv, d, nq):
    torch = torch_mod
    banner(f"attention_quant {qname} ctx={ctx} Hq={Hq} Hkv={Hkv} d={d} nq={nq}")
    quant = _quant(oracle, qname)
    rng = np.random.default_rng(sum(ctx) + d + nq)
    kp, vp, ksc, vsc, tables = quant_workload(oracle, rng, ctx, Hkv, d, quant)
    q = rng.standard_normal((len(ctx), nq, Hq, d)).astype(np.float16)
    scale = np.float32(1.0) / np.sqrt(np.float32(d))
    ref = oracle.paged_attention_quant(q.astype(np.float32), kp, vp, ksc, vsc, quant, tables,
                                       np.asarray(ctx, np.int32), nq, Hq, Hkv, d, scale)
    kv = upload(torch, ops, cuda, kp, vp, ksc, vsc, qname)
    out = ops.paged_decode_attention_quant(
        to_dev(torch, q, cuda), kv, to_dev(torch, tables, cuda),
        to_dev(torch, np.asarray(ctx, np.int32), cuda), num_kv_heads=Hkv, scale=float(scale),
        out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), ref, F16_ATOL, F16_RTOL, f"attention {qname}")


@pytest.mark.parametrize("qname", ["int8", "int4"])
def test_append_then_attention_quant(oracle, torch_mod, ops, cuda, qname):
    """The serving order: GPU prefill chunk, GPU decode token, GPU attention,
    all against the oracle (pools bit-exact, output within tolerance)."""
    torch = torch_mod
    banner(f"append->attention {qname}")
    quant = _quant(oracle, qname)
    rng = np.random.default_rng(11)
    Hq, Hkv, d = 32, 8, 128
    ctx = [520, 33, 1029]
    nb, tables, _ = layout(rng, ctx)
    kp, vp, ksc, vsc = garbage_pools(rng, oracle, nb, Hkv, d, quant)
    kv = upload(torch, ops, cuda, kp, vp, ksc, vsc, qname)
    for phase in ("prefill", "decode"):
        ss = []  # prefill: all but each sequence's last token; decode: that token
        for s, c in enumerate(ctx):
            ps = range(c - 1) if phase == "prefill" else [c - 1]
            ss += [tables[s, p // BS] * BS + p % BS for p in ps]
        slots = np.asarray(ss, np.int64)
        n = len(slots)
        k = tokens(rng, n, Hkv, d).astype(np.float16)
        v = tokens(rng, n, Hkv, d).astype(np.float16)
        oracle.paged_append_quant(kp, vp, ksc, vsc, k.astype(np.float32).reshape(n, -1),
                                  v.astype(np.float32).reshape(n, -1), slots, Hkv, d, quant)
        ops.kv_append_quant(kv, to_dev(torch, k, cuda), to_dev(torch, v, cuda),
                            torch.from_numpy(slots).to(cuda), num_kv_heads=Hkv, head_dim=d)
    torch.cuda.synchronize()
    assert_pools_equal(kv, kp, vp, ksc, vsc, qname)
    q = rng.standard_normal((len(ctx), 1, Hq, d)).astype(np.float16)
    scale = np.float32(1.0) / np.sqrt(np.float32(d))
    ref = oracle.paged_attention_quant(q.astype(np.float32), kp, vp, ksc, vsc, quant, tables,
                                       np.asarray(ctx, np.int32), 1, Hq, Hkv, d, scale)
    out = ops.paged_decode_attention_quant(
        to_dev(torch, q, cuda), kv, to_dev(torch, tables, cuda),
        to_dev(torch, np.asarray(ctx, np.int32), cuda), num_kv_heads=Hkv, scale=float(scale),
        out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), ref, F16_ATOL, F16_RTOL, f"append->attention {qname}")


@pytest.mark.parametrize("qname", ["int8", "int4"])
def test_fork_quant_pools(oracle, torch_mod, ops, cuda, qname):
    """copy_blocks_quant copies codes and scales of each (src, dst) pair."""
    torch = torch_mod
    banner(f"fork quant {qname}")
    quant = _quant(oracle, qname)
    rng = np.random.default_rng(5)
    nb, Hkv, d = 40, 8, 128
    kp, vp, ksc, vsc = garbage_pools(rng, oracle, nb, Hkv, d, quant)
    ksc[:] = rng.standard_normal(ksc.shape)
    vsc[:] = rng.standard_normal(vsc.shape)
    kv = upload(torch, ops, cuda, kp, vp, ksc, vsc, qname)
    pairs = np.stack([np.arange(0, 10), np.arange(20, 30)], 1).astype(np.int32)
    ops.copy_blocks_quant(kv, torch.from_numpy(pairs).to(cuda))
    torch.cuda.synchronize()
    for a in (kp, vp, ksc, vsc):
        a[20:30] = a[0:10]
    assert_pools_equal(kv, kp, vp, ksc, vsc, f"fork {qname}")


@pytest.mark.parametrize("qname", ["int8", "int4"])
@pytest.mark.parametrize("Hq,nq", [(32, 1), (32, 2), (32, 4)])  # 4 / 8 / 16 rows
def test_attention_quant_masks_out_of_pool_blocks(oracle, torch_mod, ops, cuda, qname, Hq, nq):
    """A block id outside the pool (negative or >= num_blocks) inside the context is
    masked: the output equals attention over the same sequence with that block
    removed (the remaining tokens keep their order; the causal limits of the last
    nq positions are unchanged), and nothing outside the pool is read."""
    torch = torch_mod
    banner(f"attention_quant {qname} out-of-pool table ids Hq={Hq} nq={nq}")
    quant = _quant(oracle, qname)
    Hkv, d = 8, 128
    ctx = [700, 1300, 90, 2100]
    rng = np.random.default_rng(77 + nq)
    kp, vp, ksc, vsc, tables = quant_workload(oracle, rng, ctx, Hkv, d, quant)
    nb = kp.shape[0]
    bad = tables.copy()
    ref_tables = tables.copy()
    ref_ctx = np.asarray(ctx, np.int32).copy()
    for s, (bi, bad_id) in {0: (3, -1), 1: (40, nb + 5), 3: (0, 2**30)}.items():
        bad[s, bi] = bad_id
        row = np.delete(tables[s], bi)
        ref_tables[s] = np.concatenate([row, row[-1:]])
        ref_ctx[s] -= BS
    q = rng.standard_normal((len(ctx), nq, Hq, d)).astype(np.float16)
    scale = np.float32(1.0) / np.sqrt(np.float32(d))
    ref = oracle.paged_attention_quant(q.astype(np.float32), kp, vp, ksc, vsc, quant, ref_tables,
                                       ref_ctx, nq, Hq, Hkv, d, scale)
    kv = upload(torch, ops, cuda, kp, vp, ksc, vsc, qname)
    out = ops.paged_decode_attention_quant(
        to_dev(torch, q, cuda), kv, to_dev(torch, bad, cuda),
        to_dev(torch, np.asarray(ctx, np.int32), cuda), num_kv_heads=Hkv, scale=float(scale),
        out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), ref, F16_ATOL, F16_RTOL, f"attention {qname} masked blocks")
