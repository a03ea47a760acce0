"""Pins for the decode-block part of the CPU oracle (oracle/oracle.c: weight
decode and quantization, matvec, rmsnorm, silu, RoPE, decode_block over a paged
pool) before it is trusted as the checker of dlmk_decode_block_paged.

Each function is checked against something independent of its own formula:
the reference's own unit tests (src/forward/cpu.rs:1282-1465,
src/quant/dequant.rs tests), closed forms (rotation preserves norms, position 0
is the identity, silu(0) = 0, zero weights give the identity block), NumPy's
IEEE decoders, hand-built quantized blobs, and a float64 NumPy restatement of
the whole block over a contiguous KV history.
"""
import math

import numpy as np
import pytest

W_F32, W_BF16, W_F16, W_INT4, W_INT8 = 0, 1, 2, 3, 4


# ----------------------------------------------------------- primitives

def test_matvec_known_answer(oracle):
    # cpu.rs:1282 matvec_basic: [[1,2],[3,4]] . [1,1] = [3,7]
    y = oracle.matvec(np.array([1, 2, 3, 4], np.float32), W_F32, [1, 1], 2, 2)
    assert y.tolist() == [3.0, 7.0]


def test_rmsnorm_known_answer(oracle):
    # cpu.rs:1289 rmsnorm_normalizes: x=[3,4] -> [0.848528, 1.131371]
    y = oracle.rmsnorm([3.0, 4.0], [1.0, 1.0], 0.0)
    np.testing.assert_allclose(y, [0.848528, 1.131371], atol=1e-4)


def test_rmsnorm_f64_brute_force(oracle):
    rng = np.random.default_rng(1)
    x = rng.standard_normal(777).astype(np.float32)
    w = rng.standard_normal(777).astype(np.float32)
    ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5) * w
    np.testing.assert_allclose(oracle.rmsnorm(x, w, 1e-5), ref, rtol=1e-5, atol=1e-6)


def test_silu_known_answers_and_closed_form(oracle):
    # cpu.rs:1304 silu_values
    assert abs(oracle.silu(0.0)) < 1e-6
    assert oracle.silu(20.0) > 19.9
    for x in np.linspace(-30, 30, 241):
        ref = x / (1 + math.exp(-x))
        assert abs(oracle.silu(float(x)) - ref) <= 1e-6 * max(1.0, abs(ref))


def test_rope_preserves_norm_and_is_identity_at_zero(oracle):
    # cpu.rs:1310
    inv = oracle.rope_inv_freqs(4, 10000.0)
    v = np.array([1, 2, 3, 4], np.float32)
    r = oracle.rope(v, 1, 4, 5, inv)
    assert abs(float((v ** 2).sum()) - float((r ** 2).sum())) < 1e-3
    np.testing.assert_allclose(oracle.rope(v, 1, 4, 0, inv), v, atol=1e-6)


def test_rope_is_the_neox_split_half_rotation(oracle):
    """f64 rotation of each (i, i + d/2) pair by position * inv_freq[i]."""
    rng = np.random.default_rng(2)
    H, d, pos = 3, 16, 37
    inv = oracle.rope_inv_freqs(d, 10000.0)
    v = rng.standard_normal(H * d).astype(np.float32)
    got = oracle.rope(v, H, d, pos, inv)
    ref = v.astype(np.float64).reshape(H, d).copy()
    half = d // 2
    ang = pos * inv.astype(np.float64)
    a, b = ref[:, :half].copy(), ref[:, half:].copy()
    ref[:, :half] = a * np.cos(ang) - b * np.sin(ang)
    ref[:, half:] = a * np.sin(ang) + b * np.cos(ang)
    np.testing.assert_allclose(got, ref.ravel(), atol=2e-5)


def test_inv_freqs_plain_linear_llama3(oracle):
    # cpu.rs:1325: freq_i = theta^(-2i/d)
    np.testing.assert_allclose(oracle.rope_inv_freqs(8, 10000.0),
                               [1.0, 10000 ** -0.25, 10000 ** -0.5, 10000 ** -0.75], rtol=1e-6)
    # cpu.rs:1336: linear scaling divides every frequency
    plain = oracle.rope_inv_freqs(8, 10000.0)
    np.testing.assert_allclose(oracle.rope_inv_freqs(8, 10000.0, ("linear", 4.0)), plain / 4,
                               rtol=1e-7)
    # cpu.rs:1344: Llama-3 scaling is piecewise in wavelength
    plain = oracle.rope_inv_freqs(128, 500000.0)
    sc = oracle.rope_inv_freqs(128, 500000.0, ("llama3", 8.0, 1.0, 4.0, 8192.0))
    bands = set()
    for p, s in zip(plain, sc):
        wl = 2 * math.pi / p
        if wl < 8192 / 4:
            assert s == p
            bands.add("high")
        elif wl > 8192:
            assert abs(s - p / 8) <= 1e-9 + 1e-7 * p
            bands.add("low")
        else:
            assert p / 8 - 1e-9 <= s <= p + 1e-9
            bands.add("mid")
    assert bands == {"high", "mid", "low"}


# ----------------------------------------------------------- weights

def test_float_weight_decode(oracle):
    rng = np.random.default_rng(3)
    x = rng.standard_normal(64).astype(np.float32)
    h = x.astype(np.float16)
    for i in range(64):
        assert oracle.weight_get(x, W_F32, 64, i) == x[i]
        assert oracle.weight_get(h.view(np.uint16), W_F16, 64, i) == float(h[i])
    bits = oracle.bf16_bits(x)
    widened = oracle.bf16_to_f32(bits)  # bf16 is the top half of an f32
    for i in range(64):
        assert oracle.weight_get(bits, W_BF16, 64, i) == widened[i]


def _blob(codes, scales, zeros, w_dtype, group):
    """Weights blob built by hand: [codes][pad to 4][scales][zeros] (cpu.rs:132-159)."""
    n = len(codes)
    code_bytes = (n + 1) // 2 if w_dtype == W_INT4 else n
    so = (code_bytes + 3) // 4 * 4
    g = -(-n // group)
    blob = np.zeros(so + 8 * g, np.uint8)
    for i, c in enumerate(codes):
        if w_dtype == W_INT4:
            blob[i // 2] |= (c & 15) << (4 * (i % 2))
        else:
            blob[i] = c
    blob[so:so + 4 * g] = np.asarray(scales, np.float32).view(np.uint8)
    blob[so + 4 * g:] = np.asarray(zeros, np.float32).view(np.uint8)
    return blob


def test_quant_blob_layout_and_decode(oracle):
    # dequant.rs dequantizes_known_example: codes 0, 15 with scale 2, zero 0 -> 0, 30
    b = _blob([0, 15], [2.0], [0.0], W_INT4, 2)
    assert oracle.quant_blob_bytes(W_INT4, 2, 2) == b.size
    assert [oracle.weight_get(b, W_INT4, 2, i, 2) for i in range(2)] == [0.0, 30.0]
    # dequant.rs pack_unpack_round_trips: odd length, low nibble holds the even index
    codes = [0, 15, 1, 8, 7, 3, 9]
    b = _blob(codes, [1.0], [0.0], W_INT4, 8)
    assert b[:4].tolist() == [0xF0, 0x81, 0x37, 0x09]
    assert [oracle.weight_get(b, W_INT4, 7, i, 8) for i in range(7)] == codes
    # Two groups, nonzero zero-points, int8 (one code a byte, scales 4-byte aligned).
    codes = [3, 250, 17, 0, 128, 255, 9]
    b = _blob(codes, [0.5, 0.25], [10.0, 100.0], W_INT8, 4)
    assert oracle.quant_blob_bytes(W_INT8, 7, 4) == b.size == 8 + 16
    got = [oracle.weight_get(b, W_INT8, 7, i, 4) for i in range(7)]
    want = [(c - (10.0 if i < 4 else 100.0)) * (0.5 if i < 4 else 0.25) for i, c in enumerate(codes)]
    assert got == want


@pytest.mark.parametrize("w_dtype,levels", [(W_INT4, 15), (W_INT8, 255)])
def test_quantize_round_trip_within_half_a_step(oracle, w_dtype, levels):
    rng = np.random.default_rng(4 + w_dtype)
    v = (rng.standard_normal(1000) * 0.3).astype(np.float32)
    v[256:384] = 0.125  # a degenerate (constant) group: scale 1, code 0 reconstructs it
    blob = oracle.quantize_weights(v, w_dtype, 128)
    got = np.array([oracle.weight_get(blob, w_dtype, v.size, i) for i in range(v.size)])
    for g in range(-(-v.size // 128)):
        seg = v[g * 128:(g + 1) * 128]
        step = (seg.max() - seg.min()) / levels
        err = np.abs(got[g * 128:(g + 1) * 128] - seg)
        assert err.max() <= (step / 2 if step > 0 else 0) + 1e-6, g
    assert np.all(got[256:384] == np.float32(0.125))


@pytest.mark.parametrize("w_dtype", [W_F32, W_BF16, W_F16, W_INT4, W_INT8])
def test_matvec_native_matches_f64(oracle, w_dtype):
    rng = np.random.default_rng(10 + w_dtype)
    out_dim, in_dim = 24, 256
    w = (rng.standard_normal(out_dim * in_dim) * 0.05).astype(np.float32)
    x = rng.standard_normal(in_dim).astype(np.float32)
    if w_dtype == W_F32:
        wn, dense = w, w
    elif w_dtype == W_F16:
        wn = w.astype(np.float16).view(np.uint16)
        dense = w.astype(np.float16).astype(np.float32)
    elif w_dtype == W_BF16:
        wn = oracle.bf16_bits(w)
        dense = oracle.bf16_to_f32(wn)
    else:
        wn = oracle.quantize_weights(w, w_dtype)
        dense = np.array([oracle.weight_get(wn, w_dtype, w.size, i) for i in range(w.size)],
                         np.float32)
    ref = dense.reshape(out_dim, in_dim).astype(np.float64) @ x.astype(np.float64)
    got = oracle.matvec(wn, w_dtype, x, out_dim, in_dim)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


# ----------------------------------------------------------- the block

def small_cfg(**kw):
    c = dict(hidden_size=4, num_heads=2, num_kv_heads=1, head_dim=2, inter=6, rms_eps=1e-5,
             w_dtype=W_F32, w_group_size=0)
    c.update(kw)
    return c


def zero_weights(c):
    H, qd, kvd, I = c["hidden_size"], c["num_heads"] * c["head_dim"], \
        c["num_kv_heads"] * c["head_dim"], c["inter"]
    z = lambda n: np.zeros(n, np.float32)
    return dict(q_proj=z(qd * H), k_proj=z(kvd * H), v_proj=z(kvd * H), o_proj=z(H * qd),
                gate_proj=z(I * H), up_proj=z(I * H), down_proj=z(H * I),
                in_norm=np.ones(H, np.float32), post_norm=np.ones(H, np.float32))


def empty_pools(c, nb=4, bs=16):
    d, Hkv = c["head_dim"], c["num_kv_heads"]
    return np.zeros((nb, Hkv, d * bs), np.float32), np.zeros((nb, Hkv, d * bs), np.float32)


def test_decode_block_zero_weights_is_identity(oracle):
    # cpu.rs:1447: zero projections => both residual deltas are zero
    c = small_cfg()
    kp, vp = empty_pools(c)
    hidden = np.array([1.5, -2.0, 0.5, 3.0], np.float32)
    inv = oracle.rope_inv_freqs(2, 10000.0)
    out = oracle.decode_block_paged(c, zero_weights(c), hidden, kp, vp, [2, 0, 1, 3], 0, 0, inv)
    np.testing.assert_allclose(out, hidden, atol=1e-6)


def test_decode_block_v_bias_reaches_the_output(oracle):
    # cpu.rs:1373 qkv_bias_shifts_the_block_output
    c = small_cfg()
    w = zero_weights(c)
    qd = c["num_heads"] * c["head_dim"]
    o = np.zeros((c["hidden_size"], qd), np.float32)
    for i in range(min(c["hidden_size"], qd)):
        o[i, i] = 1.0
    w["o_proj"] = o.ravel()
    hidden = np.array([1.5, -2.0, 0.5, 3.0], np.float32)
    inv = oracle.rope_inv_freqs(2, 10000.0)
    kp, vp = empty_pools(c)
    base = oracle.decode_block_paged(c, w, hidden, kp, vp, [0, 1, 2, 3], 0, 0, inv)
    w["v_bias"] = np.ones(c["num_kv_heads"] * c["head_dim"], np.float32)
    kp, vp = empty_pools(c)
    biased = oracle.decode_block_paged(c, w, hidden, kp, vp, [0, 1, 2, 3], 0, 0, inv)
    assert np.abs(base - biased).max() > 1e-6
    # With one position the context is that value (the bias): o_proj copies it.
    np.testing.assert_allclose(biased - hidden, [1, 1, 1, 1], atol=1e-6)


def ref_block_f64(c, w, dense, hidden, keys, values, position, inv):
    """decode_block in float64 NumPy over a contiguous [pos][Hkv][d] history."""
    H, Hq, Hkv, d, I = c["hidden_size"], c["num_heads"], c["num_kv_heads"], c["head_dim"], c["inter"]
    f = lambda n: dense[n].astype(np.float64)
    x = hidden.astype(np.float64)

    def norm(v, g):
        return v / np.sqrt(np.mean(v * v) + c["rms_eps"]) * g.astype(np.float64)

    def rot(v, heads):
        v = v.reshape(heads, d).copy()
        a, b = v[:, :d // 2].copy(), v[:, d // 2:].copy()
        ang = position * inv.astype(np.float64)
        v[:, :d // 2] = a * np.cos(ang) - b * np.sin(ang)
        v[:, d // 2:] = a * np.sin(ang) + b * np.cos(ang)
        return v.ravel()

    n1 = norm(x, w["in_norm"])
    q = f("q_proj").reshape(Hq * d, H) @ n1 + (w["q_bias"] if w.get("q_bias") is not None else 0)
    k = f("k_proj").reshape(Hkv * d, H) @ n1 + (w["k_bias"] if w.get("k_bias") is not None else 0)
    v = f("v_proj").reshape(Hkv * d, H) @ n1 + (w["v_bias"] if w.get("v_bias") is not None else 0)
    q, k = rot(q, Hq), rot(k, Hkv)
    keys.append(k.reshape(Hkv, d))
    values.append(v.reshape(Hkv, d))
    K, V = np.array(keys), np.array(values)
    ctx = np.zeros(Hq * d)
    g = Hq // Hkv
    for h in range(Hq):
        s = K[:, h // g, :] @ q[h * d:(h + 1) * d] / math.sqrt(d)
        p = np.exp(s - s.max())
        ctx[h * d:(h + 1) * d] = (p / p.sum()) @ V[:, h // g, :]
    x = x + f("o_proj").reshape(H, Hq * d) @ ctx
    n2 = norm(x, w["post_norm"])
    gt = f("gate_proj").reshape(I, H) @ n2
    up = f("up_proj").reshape(I, H) @ n2
    act = gt / (1 + np.exp(-gt)) * up
    return x + f("down_proj").reshape(H, I) @ act


@pytest.mark.parametrize("w_dtype", [W_F32, W_BF16, W_INT4])
def test_decode_block_matches_f64_over_steps(oracle, w_dtype):
    """Five decode steps on shuffled physical blocks (crossing a block boundary
    after a 14-token history), GQA 2, biases, Llama-3 RoPE scaling."""
    rng = np.random.default_rng(40 + w_dtype)
    c = small_cfg(hidden_size=64, num_heads=4, num_kv_heads=2, head_dim=16, inter=96,
                  w_dtype=w_dtype, w_group_size=128 if w_dtype >= W_INT4 else 0)
    H, qd, kvd, I = 64, 64, 32, 96
    dense, w = {}, {}
    for name, n in (("q_proj", qd * H), ("k_proj", kvd * H), ("v_proj", kvd * H),
                    ("o_proj", H * qd), ("gate_proj", I * H), ("up_proj", I * H),
                    ("down_proj", H * I)):
        f = (rng.uniform(-1, 1, n) * 0.2).astype(np.float32)
        if w_dtype == W_BF16:
            w[name] = oracle.bf16_bits(f)
            dense[name] = oracle.bf16_to_f32(w[name])
        elif w_dtype == W_INT4:
            w[name] = oracle.quantize_weights(f, W_INT4)
            dense[name] = np.array([oracle.weight_get(w[name], W_INT4, n, i) for i in range(n)],
                                   np.float32)
        else:
            w[name] = dense[name] = f
    w["in_norm"] = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    w["post_norm"] = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    for name, n in (("q_bias", qd), ("k_bias", kvd), ("v_bias", kvd)):
        w[name] = (0.1 * rng.standard_normal(n)).astype(np.float32)
    inv = oracle.rope_inv_freqs(16, 500000.0, ("llama3", 8.0, 1.0, 4.0, 8192.0))

    # A 14-token history already in the pool, mirrored contiguously for the reference.
    kp, vp = empty_pools(c, nb=6)
    table = np.array([4, 1, 5, 0], np.int32)
    keys, values = [], []
    for p in range(14):
        k = rng.standard_normal((2, 16)).astype(np.float32)
        v = rng.standard_normal((2, 16)).astype(np.float32)
        oracle.paged_append(kp.reshape(6, 2, 4, 16, 4), vp.reshape(6, 2, 16, 16), k[None], v[None],
                            np.array([table[p // 16] * 16 + p % 16], np.int64), 2, 16, 16)
        keys.append(k.astype(np.float64))
        values.append(v.astype(np.float64))
    x = (rng.standard_normal(H)).astype(np.float32)
    xr = x.astype(np.float64)
    for step in range(5):
        p = 14 + step
        x = oracle.decode_block_paged(c, w, x, kp, vp, table, p, p, inv)
        xr = ref_block_f64(c, w, dense, xr.astype(np.float32), keys, values, p, inv)
        np.testing.assert_allclose(x, xr, rtol=2e-4, atol=2e-4, err_msg=f"step {step}")
