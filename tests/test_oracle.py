"""Pins for the CPU oracle (oracle/oracle.c) before it is trusted as a checker.

Each function is checked against something independent of its own formula:
the reference's known answers (tests/golden/reference_known_answers.json), a
float64 NumPy brute force, closed forms (single position, uniform scores,
one-hot scores, convex hull), library routines (NumPy's IEEE f16 decoder),
published SplitMix64 outputs, and round-trip identities for the byte moves.
"""
import json
import os

import numpy as np
import pytest

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                   "reference_known_answers.json")))


def brute_attention_f64(q, keys, values, Hq, Hkv, d, scale):
    """Textbook softmax attention in float64 (independent of the oracle)."""
    q = q.astype(np.float64).reshape(Hq, d)
    k = keys.astype(np.float64).reshape(-1, Hkv, d)
    v = values.astype(np.float64).reshape(-1, Hkv, d)
    out = np.zeros((Hq, d))
    g = Hq // Hkv
    for h in range(Hq):
        s = k[:, h // g, :] @ q[h] * scale
        if len(s) == 0:
            continue
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p @ v[:, h // g, :]
    return out.reshape(-1)


# ---------------------------------------------------------------- primitives

def test_splitmix64_published_outputs(oracle):
    # SplitMix64 from state 0 yields 0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, ...;
    # Rng::new(seed) starts from seed ^ golden (tests/gpu_parity.rs:34-36).
    import ctypes as C
    L = oracle.lib()
    L.orc_rng_next.restype = C.c_uint64
    L.orc_rng_next.argtypes = [C.POINTER(C.c_uint64)]
    st = C.c_uint64(0)
    assert L.orc_rng_next(C.byref(st)) == 0xE220A8397B1DCDAF
    assert L.orc_rng_next(C.byref(st)) == 0x6E789E6AA1B965F4
    assert L.orc_rng_next(C.byref(st)) == 0x06C45D188009454F
    u = oracle.rng_uniform(0x9E3779B97F4A7C15, 1, 1.0)  # state 0 -> first draw
    assert u[0] == np.float32((0xE220A8397B1DCDAF >> 40) / 2**24 * 2 - 1)


def test_f16_decoder_matches_ieee_for_every_pattern(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


# ---------------------------------------------------------------- attention

@pytest.mark.parametrize("name", ["attention_single_position_returns_its_value",
                                  "attention_gqa_shares_kv_head_across_query_heads"])
def test_attention_reference_known_answers(oracle, name):
    g = GOLD[name]
    out = oracle.attention(np.array(g["q"]), np.array(g["keys"]), np.array(g["values"]),
                           g["num_heads"], g["num_kv_heads"], g["head_dim"])
    assert np.allclose(out, g["expected"], atol=g["tol"], rtol=0)


@pytest.mark.parametrize("Hq,Hkv,d,P,seed", [(4, 2, 8, 1, 0), (4, 2, 8, 37, 1), (8, 2, 16, 200, 2),
                                             (3, 1, 4, 5, 3), (32, 8, 64, 64, 4)])
def test_attention_matches_f64_brute_force(oracle, Hq, Hkv, d, P, seed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(Hq * d).astype(np.float32)
    k = rng.standard_normal((P, Hkv, d)).astype(np.float32)
    v = rng.standard_normal((P, Hkv, d)).astype(np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(d))
    got = oracle.attention(q, k, v, Hq, Hkv, d, scale)
    ref = brute_attention_f64(q, k, v, Hq, Hkv, d, float(scale))
    assert np.abs(got - ref).max() < 1e-5


def test_attention_uniform_scores_give_mean_of_values(oracle):
    rng = np.random.default_rng(5)
    P, Hkv, d, Hq = 24, 2, 8, 4
    k = rng.standard_normal((P, Hkv, d)).astype(np.float32)
    v = rng.standard_normal((P, Hkv, d)).astype(np.float32)
    out = oracle.attention(np.zeros(Hq * d, np.float32), k, v, Hq, Hkv, d).reshape(Hq, d)
    for h in range(Hq):
        assert np.allclose(out[h], v[:, h // 2].mean(0), atol=1e-6)


def test_attention_one_hot_score_selects_that_value(oracle):
    P, d = 10, 4
    k = np.zeros((P, 1, d), np.float32)
    k[6, 0, 0] = 1000.0
    v = np.arange(P * d, dtype=np.float32).reshape(P, 1, d)
    q = np.array([1.0, 0, 0, 0], np.float32)
    out = oracle.attention(q, k, v, 1, 1, d, 1.0)
    assert np.array_equal(out, v[6, 0])


def test_attention_is_a_convex_combination(oracle):
    rng = np.random.default_rng(6)
    P, Hkv, d, Hq = 50, 2, 16, 8
    k = (rng.standard_normal((P, Hkv, d)) * 3).astype(np.float32)
    v = rng.standard_normal((P, Hkv, d)).astype(np.float32)
    q = rng.standard_normal(Hq * d).astype(np.float32)
    out = oracle.attention(q, k, v, Hq, Hkv, d).reshape(Hq, d)
    for h in range(Hq):
        vh = v[:, h // 4]
        assert np.all(out[h] >= vh.min(0) - 1e-6) and np.all(out[h] <= vh.max(0) + 1e-6)


def test_attention_empty_history_gives_zeros(oracle):
    out = oracle.attention(np.ones(8, np.float32), np.zeros((0, 1, 8), np.float32),
                           np.zeros((0, 1, 8), np.float32), 1, 1, 8)
    assert np.array_equal(out, np.zeros(8, np.float32))


# ---------------------------------------------------------------- paging

def make_pools(num_blocks, Hkv, d, bs, dtype, rng):
    X = 16 // np.dtype(dtype).itemsize
    # Fill with garbage so an unwritten slot would be visible.
    k = rng.standard_normal((num_blocks, Hkv, d // X, bs, X)).astype(dtype)
    v = rng.standard_normal((num_blocks, Hkv, d, bs)).astype(dtype)
    return k, v


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_paged_append_then_gather_reproduces_tokens(oracle, dtype):
    rng = np.random.default_rng(7)
    Hkv, d, bs, nb, ntok = 2, 16, 16, 12, 70
    kp, vp = make_pools(nb, Hkv, d, bs, dtype, rng)
    table = rng.permutation(nb)[: -(-ntok // bs)].astype(np.int32)
    ks = rng.standard_normal((ntok, Hkv, d)).astype(dtype)
    vs = rng.standard_normal((ntok, Hkv, d)).astype(dtype)
    slots = np.array([table[p // bs] * bs + p % bs for p in range(ntok)], np.int64)
    # Split into a chunk and single-token appends; the result must not care.
    oracle.paged_append(kp, vp, ks[:50], vs[:50], slots[:50], Hkv, d, bs)
    for i in range(50, ntok):
        oracle.paged_append(kp, vp, ks[i:i + 1], vs[i:i + 1], slots[i:i + 1], Hkv, d, bs)
    gk, gv = oracle.gather_logical(kp, vp, table, ntok, Hkv, d, bs, dtype)
    assert np.array_equal(gk, ks.astype(np.float32))
    assert np.array_equal(gv, vs.astype(np.float32))
    # Physical layout: K[blk][h][j // X][t][j % X], V[blk][h][j][t].
    X = 16 // np.dtype(dtype).itemsize
    p, h, j = 37, 1, 13
    blk, t = table[p // bs], p % bs
    assert kp[blk, h, j // X, t, j % X] == ks[p, h, j]
    assert vp[blk, h, j, t] == vs[p, h, j]


def test_paged_append_skips_negative_and_out_of_pool_slots(oracle):
    rng = np.random.default_rng(8)
    kp, vp = make_pools(2, 1, 8, 16, np.float32, rng)
    k0, v0 = kp.copy(), vp.copy()
    src = np.ones((3, 1, 8), np.float32)
    oracle.paged_append(kp, vp, src, src, np.array([-1, 32, 1000], np.int64), 1, 8, 16)
    assert np.array_equal(kp, k0) and np.array_equal(vp, v0)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_paged_attention_equals_contiguous_attention_bitwise(oracle, dtype):
    """paged result == the reference's contiguous result on the same sequence."""
    rng = np.random.default_rng(9)
    Hq, Hkv, d, bs, nb = 8, 2, 16, 16, 40
    kp, vp = make_pools(nb, Hkv, d, bs, dtype, rng)
    ctx = np.array([1, 15, 16, 17, 100, 0], np.int32)
    maxb = 8
    perm = rng.permutation(nb)
    tables = np.zeros((len(ctx), maxb), np.int32)
    off = 0
    for s, c in enumerate(ctx):
        n = -(-c // bs)
        tables[s, :n] = perm[off:off + n]
        off += n
    q = rng.standard_normal((len(ctx), 1, Hq, d)).astype(dtype)
    scale = np.float32(1.0) / np.sqrt(np.float32(d))
    out = oracle.paged_attention(q, kp, vp, tables, ctx, 1, Hq, Hkv, d, bs, scale)
    for s, c in enumerate(ctx):
        keys, values = oracle.gather_logical(kp, vp, tables[s], c, Hkv, d, bs, dtype)
        ref = oracle.attention(q[s, 0].astype(np.float32), keys, values, Hq, Hkv, d, scale)
        assert np.array_equal(out[s, 0].reshape(-1), ref)
        bf = brute_attention_f64(q[s, 0].astype(np.float32), keys, values, Hq, Hkv, d,
                                 float(scale))
        assert np.abs(out[s, 0].reshape(-1) - bf).max() < 1e-5


def test_multi_query_verify_is_causal_prefix_attention(oracle):
    rng = np.random.default_rng(10)
    Hq, Hkv, d, bs, nb, nq = 4, 1, 8, 16, 10, 4
    kp, vp = make_pools(nb, Hkv, d, bs, np.float32, rng)
    ctx = np.array([35, 3], np.int32)  # second sequence: first query sees 0 tokens
    tables = np.array([[4, 7, 1, 0], [9, 0, 0, 0]], np.int32)
    q = rng.standard_normal((2, nq, Hq, d)).astype(np.float32)
    out = oracle.paged_attention(q, kp, vp, tables, ctx, nq, Hq, Hkv, d, bs, 0.3)
    for s in range(2):
        for j in range(nq):
            n = max(int(ctx[s]) - nq + j + 1, 0)
            keys, values = oracle.gather_logical(kp, vp, tables[s], n, Hkv, d, bs, np.float32)
            ref = oracle.attention(q[s, j], keys, values, Hq, Hkv, d, 0.3)
            assert np.array_equal(out[s, j].reshape(-1), ref)
    assert np.array_equal(out[1, 0], np.zeros((Hq, d), np.float32))


# ---------------------------------------------------------------- block moves

def test_copy_gather_scatter_round_trips(oracle):
    rng = np.random.default_rng(11)
    bb = 256
    kp = rng.integers(0, 256, 10 * bb, dtype=np.uint8)
    vp = rng.integers(0, 256, 10 * bb, dtype=np.uint8)
    ids = np.array([7, 2, 5], np.int32)
    st = oracle.gather_blocks(kp, vp, ids, bb)
    for i, b in enumerate(ids):
        assert np.array_equal(st[(2 * i) * bb:(2 * i + 1) * bb], kp[b * bb:(b + 1) * bb])
        assert np.array_equal(st[(2 * i + 1) * bb:(2 * i + 2) * bb], vp[b * bb:(b + 1) * bb])
    k0, v0 = kp.copy(), vp.copy()
    kp[:] = 0
    vp[:] = 0
    oracle.scatter_blocks(kp, vp, st, ids, bb)
    for b in ids:
        assert np.array_equal(kp[b * bb:(b + 1) * bb], k0[b * bb:(b + 1) * bb])
    oracle.copy_blocks(kp, vp, np.array([[7, 0], [2, 9]], np.int32), bb)
    assert np.array_equal(kp[0:bb], k0[7 * bb:8 * bb])
    assert np.array_equal(vp[9 * bb:10 * bb], v0[2 * bb:3 * bb])


# ---------------------------------------------------------------- int8 / int4 KV

def test_quantize_i8_round_trips_within_a_quantum(oracle):
    g = GOLD["quantize_i8_round_trips_within_a_quantum"]
    x = np.array(g["x"], np.float32)
    q, s = oracle.quantize_i8(x)
    assert np.all(np.abs(x - q.astype(np.float32) * s) <= s)
    assert s == np.float32(3.0) / np.float32(127.0)
    qz, sz = oracle.quantize_i8(np.array(g["zero_input"], np.float32))
    assert sz == 0 and not qz.any()


def test_quantize_i4_round_trips_within_a_quantum(oracle):
    g = GOLD["quantize_i4_round_trips_within_a_quantum"]
    x = np.array(g["x"], np.float32)
    packed, s = oracle.quantize_i4(x)
    assert len(packed) == g["packed_len"]
    for i, xi in enumerate(x):
        assert abs(xi - oracle.read_i4(packed, 0, i) * s) <= s
    pz, sz = oracle.quantize_i4(np.array(g["zero_input"], np.float32))
    assert sz == 0 and not pz.any()
    # round half away from zero (f32::round): 0.5 * scale -> code 1, -0.5 -> -1
    p2, s2 = oracle.quantize_i4(np.array([7.0, 0.5, -0.5], np.float32))
    assert [oracle.read_i4(p2, 0, i) for i in range(3)] == [7.0, 1.0, -1.0]


def test_quantize_nan_and_inf_follow_rust_casts(oracle):
    """`(v / scale).round().clamp(..) as i8` (cpu.rs:680, :696): f32::max skips
    NaN when taking max|x|, and the saturating cast sends NaN to 0, so a NaN
    element gets code 0 and an inf element makes scale inf with every code 0
    (finite / inf = 0, inf / inf = NaN -> 0)."""
    x = np.array([np.nan, 1.0, -2.0, 0.0], np.float32)
    q, s = oracle.quantize_i8(x)
    assert s == np.float32(2.0) / np.float32(127.0)
    assert q.tolist() == [0, 64, -127, 0]  # 1 / (2/127) = 63.5 -> 64 (half away from zero)
    p4, s4 = oracle.quantize_i4(x)
    assert [oracle.read_i4(p4, 0, i) for i in range(4)] == [0.0, 3.0, -7.0, 0.0]
    for fn in (oracle.quantize_i8, oracle.quantize_i4):
        codes, sc = fn(np.array([np.inf, 1.0, -np.inf], np.float32))
        assert sc == np.inf and not codes.any()


def test_bf16_decode_matches_torch(oracle):
    """The oracle's bf16 widening (used for bf16 pools) equals torch's bf16 -> f32."""
    import torch
    bits = np.arange(0, 65536, 7, dtype=np.uint16)
    ref = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float().numpy()
    n = len(bits) - len(bits) % 128
    v = bits[:n].reshape(-1, 1, 8, 16)  # [blocks][1 head][d=8][16]
    k = np.zeros((v.shape[0], 1, 1, 16, 8), np.uint16)
    table = np.arange(v.shape[0], dtype=np.int32)
    _, vals = oracle.gather_logical(k, v, table, v.shape[0] * 16, 1, 8, 16, np.uint16)
    got = vals.reshape(v.shape[0], 16, 8).transpose(0, 2, 1).reshape(-1)
    finite = np.isfinite(ref[:n])
    assert np.array_equal(got[finite], ref[:n][finite])
    assert np.array_equal(np.isnan(got), np.isnan(ref[:n]))
    assert np.array_equal(oracle.bf16_bits(ref[:n][finite]), bits[:n][finite])


# ---------------------------------------------------------------- quantized KV attention

def _ref_quant_case():
    """The inputs of cpu.rs:1480-1544 (int8_/int4_kv_attention_close_to_full)."""
    g = GOLD["kv_quant_attention_close_to_full"]
    Hq, Hkv, d, P = g["num_heads"], g["num_kv_heads"], g["head_dim"], g["positions"]
    kv = Hkv * d
    k = np.array([[((p + i) % 7) * 0.3 - 1.0 for i in range(kv)] for p in range(P)], np.float32)
    v = np.array([[((p * 2 + i) % 5) * 0.5 for i in range(kv)] for p in range(P)], np.float32)
    q = np.array([(i % 3) * 0.2 for i in range(Hq * d)], np.float32)
    return g, Hq, Hkv, d, k, v, q


@pytest.mark.parametrize("quant,tol_key", [(3, "tol_int8"), (4, "tol_int4")])
def test_quant_attention_close_to_full_reference_case(oracle, quant, tol_key):
    g, Hq, Hkv, d, k, v, q = _ref_quant_case()
    full = oracle.attention(q, k, v, Hq, Hkv, d)
    kc, ks = oracle.quantize_tokens(k, quant)
    vc, vs = oracle.quantize_tokens(v, quant)
    qa = oracle.attention_quant(q, kc, ks, vc, vs, Hq, Hkv, d, quant)
    assert np.abs(full - qa).max() <= g[tol_key]


@pytest.mark.parametrize("quant", [3, 4])
def test_quant_attention_matches_dequantized_f64(oracle, quant):
    """Quantized attention == textbook attention over the dequantized codes."""
    rng = np.random.default_rng(50 + quant)
    Hq, Hkv, d, P = 8, 2, 16, 40
    k = rng.standard_normal((P, Hkv * d)).astype(np.float32)
    v = rng.standard_normal((P, Hkv * d)).astype(np.float32)
    q = rng.standard_normal(Hq * d).astype(np.float32)
    kc, ks = oracle.quantize_tokens(k, quant)
    vc, vs = oracle.quantize_tokens(v, quant)
    if quant == 3:
        kd, vd = kc.astype(np.float32) * ks[:, None], vc.astype(np.float32) * vs[:, None]
    else:
        dq = lambda c, s: np.array([[oracle.read_i4(c[p], 0, i) for i in range(Hkv * d)]
                                    for p in range(P)], np.float32) * s[:, None]
        kd, vd = dq(kc, ks), dq(vc, vs)
    got = oracle.attention_quant(q, kc, ks, vc, vs, Hq, Hkv, d, quant)
    ref = brute_attention_f64(q, kd, vd, Hq, Hkv, d, 1 / np.sqrt(d))
    assert np.abs(got - ref).max() < 1e-5


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("quant", [3, 4])
def test_paged_quant_round_trip_and_attention(oracle, quant, d):
    """Paged quantized append -> gather reproduces the contiguous codes and scales
    byte for byte; paged attention equals contiguous quantized attention bitwise."""
    rng = np.random.default_rng(60 + quant + d)
    Hq, Hkv, nb, ntok = 8, 2, 12, 70
    ks_shape, vs_shape = oracle.quant_pool_shapes(nb, Hkv, d, quant)
    dt = np.int8 if quant == 3 else np.uint8
    kp = rng.integers(-100, 100, ks_shape).astype(dt)
    vp = rng.integers(-100, 100, vs_shape).astype(dt)
    ksc = rng.standard_normal(nb * 16).astype(np.float32)
    vsc = rng.standard_normal(nb * 16).astype(np.float32)
    table = rng.permutation(nb)[: -(-ntok // 16)].astype(np.int32)
    k = rng.standard_normal((ntok, Hkv * d)).astype(np.float32)
    v = rng.standard_normal((ntok, Hkv * d)).astype(np.float32)
    slots = np.array([table[p // 16] * 16 + p % 16 for p in range(ntok)], np.int64)
    oracle.paged_append_quant(kp, vp, ksc, vsc, k[:33], v[:33], slots[:33], Hkv, d, quant)
    oracle.paged_append_quant(kp, vp, ksc, vsc, k[33:], v[33:], slots[33:], Hkv, d, quant)
    kc, ks = oracle.quantize_tokens(k, quant)
    vc, vs = oracle.quantize_tokens(v, quant)
    gkc, gks, gvc, gvs = oracle.paged_gather_quant(kp, vp, ksc, vsc, table, ntok, Hkv, d, quant)
    assert np.array_equal(gkc, kc) and np.array_equal(gvc, vc)
    assert np.array_equal(gks, ks) and np.array_equal(gvs, vs)
    q = rng.standard_normal((1, 2, Hq, d)).astype(np.float32)
    tables = np.zeros((1, 8), np.int32)
    tables[0, :len(table)] = table
    out = oracle.paged_attention_quant(q, kp, vp, ksc, vsc, quant, tables, np.array([ntok], np.int32),
                                       2, Hq, Hkv, d, 0.25)
    for j in range(2):
        n = ntok - 2 + j + 1
        ref = oracle.attention_quant(q[0, j], kc[:n], ks[:n], vc[:n], vs[:n], Hq, Hkv, d, quant, 0.25)
        assert np.array_equal(out[0, j].reshape(-1), ref)


def _unpack_codes(c, quant):
    """Contiguous codes [n, row_bytes] -> signed values [n, kv_dim]."""
    if quant == 3:
        return c.astype(np.int16)
    u = c.view(np.uint8)
    lo, hi = (u & 15).astype(np.int16), (u >> 4).astype(np.int16)
    x = np.stack([lo, hi], -1).reshape(len(c), -1)
    return np.where(x >= 8, x - 16, x)


def _pack_tile_codes(vals, quant):
    """Signed codes whose last axis runs over consecutive elements -> pool bytes
    (offset binary: the byte c + 128, the nibble c + 8)."""
    if quant == 3:
        return (vals + 128).astype(np.uint8)
    u = (vals + 8).astype(np.uint8)
    return u[..., 0::2] | (u[..., 1::2] << 4)


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("quant", [3, 4])
def test_paged_quant_layout_by_axes(oracle, quant, d):
    """The paged quantized layout, restated as numpy axis permutations of the
    [token][head][dim] codes and compared with the oracle's append byte for
    byte over one full block per head, codes stored offset binary:
      K [d/KG][16 tokens][KG dims];  V [d/(16 VG)][4 quads][16][VG dims][4 tokens],
    with KG, VG = 16, 4 (int8) and 32, 8 or 16, 4 (int4, d % 128 == 0 or not)."""
    Hkv, bs = 2, 16
    kg, vg = (16, 4) if quant == 3 else ((32, 8) if d % 128 == 0 else (16, 4))
    assert oracle.quant_groups(d, quant) == (kg, vg)
    rng = np.random.default_rng(d + quant)
    k = rng.standard_normal((bs, Hkv * d)).astype(np.float32)
    v = rng.standard_normal((bs, Hkv * d)).astype(np.float32)
    ks_shape, vs_shape = oracle.quant_pool_shapes(2, Hkv, d, quant)
    kp, vp = np.zeros(ks_shape, np.uint8), np.zeros(vs_shape, np.uint8)
    ksc, vsc = np.zeros(2 * bs, np.float32), np.zeros(2 * bs, np.float32)
    oracle.paged_append_quant(kp, vp, ksc, vsc, k, v, np.arange(bs, 2 * bs), Hkv, d, quant)
    kc, _ = oracle.quantize_tokens(k, quant)
    vc, _ = oracle.quantize_tokens(v, quant)
    kx = _unpack_codes(kc, quant).reshape(bs, Hkv, d)
    vx = _unpack_codes(vc, quant).reshape(bs, Hkv, d)
    # K: [h][t][d] -> [h][d/KG][t][KG]
    kt = kx.transpose(1, 0, 2).reshape(Hkv, bs, d // kg, kg).transpose(0, 2, 1, 3)
    # V: dim j = (qq * 16 + n) * VG + kk, token t = 4 * quad + tt
    vt = vx.transpose(1, 0, 2).reshape(Hkv, 4, 4, d // (16 * vg), 16, vg)  # h, quad, tt, qq, n, kk
    vt = vt.transpose(0, 3, 1, 4, 5, 2)                                      # h, qq, quad, n, kk, tt
    if quant == 4:  # an int4 byte holds one token's dims kk, kk + 1
        vt = vt.reshape(Hkv, d // (16 * vg), 4, 16, vg // 2, 2, 4).transpose(0, 1, 2, 3, 4, 6, 5)
    assert np.array_equal(kp[1], _pack_tile_codes(kt, quant).reshape(kp[1].shape))
    assert np.array_equal(vp[1], _pack_tile_codes(vt, quant).reshape(vp[1].shape))
    assert not kp[0].any() and not vp[0].any()
