"""ctypes binding of the CPU oracle (``oracle/oracle.c``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg, always as the checker.  The product
(``dlm_amd``) never imports this module.

Every function mirrors one in ``oracle.c``; see that file for the reference
file:line each one restates.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

F32, F16, BF16, I8, I4 = 0, 1, 2, 3, 4
ERR_EXHAUSTED = -2
ERR_UNKNOWN_SEQ = -5


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    src = os.path.join(_HERE, "oracle.c")
    if force or not os.path.exists(_LIB_PATH) or os.path.getmtime(src) > os.path.getmtime(_LIB_PATH):
        subprocess.run(["make", "-B" if force else "-s", "-C", _HERE, "liboracle.so"], check=True)
    return _LIB_PATH


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


class CacheConfig(C.Structure):
    _fields_ = [("num_layers", C.c_uint32), ("num_kv_heads", C.c_uint32),
                ("head_dim", C.c_uint32), ("block_size", C.c_uint32)]


class BlockConfigC(C.Structure):
    _fields_ = [("hidden_size", C.c_int), ("num_heads", C.c_int), ("num_kv_heads", C.c_int),
                ("head_dim", C.c_int), ("inter", C.c_int), ("rms_eps", C.c_float),
                ("w_dtype", C.c_int), ("w_group_size", C.c_int64)]


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def _declare(L):
    vp, i64, u64, u32, i32, f32 = C.c_void_p, C.c_int64, C.c_uint64, C.c_uint32, C.c_int, C.c_float
    cfgp = C.POINTER(CacheConfig)
    sig = {
        "orc_rng_uniform": (None, [u64, f32, vp, i64]),
        "orc_f16_to_f32": (f32, [C.c_uint16]),
        "orc_bytes_per_token": (u64, [cfgp]),
        "orc_bytes_per_block": (u64, [cfgp]),
        "orc_blocks_for_tokens": (u64, [cfgp, u64]),
        "orc_cache_new": (vp, [cfgp, u32]),
        "orc_cache_new_with_free_order": (vp, [cfgp, vp, u32]),
        "orc_cache_with_budget": (vp, [cfgp, u64]),
        "orc_cache_destroy": (None, [vp]),
        "orc_cache_append_tokens": (i32, [vp, u64, u64, vp]),
        "orc_cache_free_sequence": (None, [vp, u64]),
        "orc_cache_truncate_sequence": (i32, [vp, u64, u64]),
        "orc_cache_fork_sequence": (i32, [vp, u64, u64, vp, u32, vp, vp]),
        "orc_cache_sequence_len": (u64, [vp, u64]),
        "orc_cache_block_table": (i64, [vp, u64, vp, u64]),
        "orc_cache_total_blocks": (u32, [vp]),
        "orc_cache_free_blocks": (u32, [vp]),
        "orc_cache_used_blocks": (u32, [vp]),
        "orc_cache_capacity_tokens": (u64, [vp]),
        "orc_cache_num_sequences": (u64, [vp]),
        "orc_cache_used_tokens": (u64, [vp]),
        "orc_cache_free_list": (u32, [vp, vp]),
        "orc_attention": (None, [vp, vp, vp, i64, i32, i32, i32, f32, vp]),
        "orc_paged_append": (None, [vp, vp, vp, vp, vp, i64, i32, i32, i32, i32, i64]),
        "orc_paged_gather_logical": (None, [vp, vp, vp, i64, i32, i32, i32, i32, vp, vp]),
        "orc_paged_attention": (None, [vp, vp, vp, vp, i32, vp, vp, i32, i32, i32, i32, i32,
                                       i32, i32, f32]),
        "orc_copy_blocks": (None, [vp, vp, vp, i64, i64]),
        "orc_gather_blocks": (None, [vp, vp, vp, vp, i64, i64]),
        "orc_scatter_blocks": (None, [vp, vp, vp, vp, i64, i64]),
        "orc_quantize_i8": (f32, [vp, i64, vp]),
        "orc_quantize_i4": (f32, [vp, i64, vp]),
        "orc_read_i4": (f32, [vp, i64, i64]),
        "orc_attention_quant": (None, [vp, vp, vp, vp, vp, i64, i32, i32, i32, f32, i32, vp]),
        "orc_quantize_tokens": (None, [vp, i64, i64, i32, vp, vp]),
        "orc_paged_append_quant": (None, [vp, vp, vp, vp, vp, vp, vp, i64, i32, i32, i32, i32,
                                          i64]),
        "orc_paged_gather_quant": (None, [vp, vp, vp, vp, vp, i64, i32, i32, i32, i32, vp, vp, vp,
                                          vp]),
        "orc_paged_attention_quant": (None, [vp, vp, vp, vp, vp, vp, i32, vp, vp, i32, i32, i32,
                                             i32, i32, i32, i32, f32]),
    }
    sig.update({
        "orc_quant_blob_bytes": (i64, [i32, i64, i64]),
        "orc_weight_get": (f32, [vp, i32, i64, i64, i64]),
        "orc_quantize_weights": (i32, [vp, i64, i64, i32, vp]),
        "orc_matvec": (None, [vp, i32, i64, vp, i64, i64, vp]),
        "orc_rmsnorm": (None, [vp, vp, i64, f32, vp]),
        "orc_silu": (f32, [f32]),
        "orc_rope_inv_freqs": (None, [i32, f32, i32, f32, f32, f32, f32, vp]),
        "orc_rope": (None, [vp, i32, i32, i64, vp]),
        "orc_decode_block_paged": (i32, [C.POINTER(BlockConfigC)] + [vp] * 14 +
                                   [vp, vp, vp, i32, i64, i32, i64, i64]),
    })
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def dtype_code(dt) -> int:
    """float32 -> F32, float16 -> F16; raw uint16 arrays are bf16 bit patterns."""
    dt = np.dtype(dt)
    if dt == np.float32:
        return F32
    if dt == np.float16:
        return F16
    if dt == np.uint16:
        return BF16
    raise ValueError(f"unsupported dtype {dt}")


def bf16_bits(x) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def bf16_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- RNG / f16

def rng_uniform(seed: int, n: int, scale: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_rng_uniform(seed, scale, _p(out), n)
    return out


def f16_to_f32(bits: int) -> float:
    return lib().orc_f16_to_f32(bits)


# ---------------------------------------------------------------- geometry

def bytes_per_token(cfg: CacheConfig) -> int:
    return lib().orc_bytes_per_token(C.byref(cfg))


def bytes_per_block(cfg: CacheConfig) -> int:
    return lib().orc_bytes_per_block(C.byref(cfg))


def blocks_for_tokens(cfg: CacheConfig, tokens: int) -> int:
    return lib().orc_blocks_for_tokens(C.byref(cfg), tokens)


# ---------------------------------------------------------------- bookkeeping

class Exhausted(Exception):
    def __init__(self, requested, free, total):
        super().__init__(f"need {requested} more block(s), {free} free of {total}")
        self.requested, self.free, self.total = requested, free, total


class OracleCache:
    """Restatement of PagedKvCache (src/cache/paged.rs:106-227) + extensions."""

    def __init__(self, cfg: CacheConfig, total_blocks: int = None, *, budget: int = None,
                 free_order=None):
        L = lib()
        self.cfg = cfg
        if free_order is not None:
            order = np.ascontiguousarray(free_order, dtype=np.uint32)
            self.h = L.orc_cache_new_with_free_order(C.byref(cfg), _p(order), len(order))
        elif budget is not None:
            self.h = L.orc_cache_with_budget(C.byref(cfg), budget)
        else:
            self.h = L.orc_cache_new(C.byref(cfg), total_blocks)

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_cache_destroy(self.h)
            self.h = None

    def append_tokens(self, seq_id: int, n: int) -> None:
        err = np.zeros(3, np.uint32)
        rc = lib().orc_cache_append_tokens(self.h, seq_id, n, _p(err))
        if rc == ERR_EXHAUSTED:
            raise Exhausted(*map(int, err))
        assert rc == 0, rc

    def free_sequence(self, seq_id: int) -> None:
        lib().orc_cache_free_sequence(self.h, seq_id)

    def truncate_sequence(self, seq_id: int, new_len: int) -> None:
        rc = lib().orc_cache_truncate_sequence(self.h, seq_id, new_len)
        if rc == ERR_UNKNOWN_SEQ:
            raise KeyError(seq_id)
        assert rc == 0, rc

    def fork_sequence(self, src: int, dst: int) -> np.ndarray:
        n = len(self.block_table(src) or [])
        pairs = np.zeros((max(n, 1), 2), np.int32)
        npairs = np.zeros(1, np.uint32)
        err = np.zeros(3, np.uint32)
        rc = lib().orc_cache_fork_sequence(self.h, src, dst, _p(pairs), max(n, 1), _p(npairs),
                                           _p(err))
        if rc == ERR_EXHAUSTED:
            raise Exhausted(*map(int, err))
        if rc == ERR_UNKNOWN_SEQ:
            raise KeyError(src)
        assert rc == 0, rc
        return pairs[: int(npairs[0])]

    def sequence_len(self, seq_id: int) -> int:
        return lib().orc_cache_sequence_len(self.h, seq_id)

    def block_table(self, seq_id: int):
        n = lib().orc_cache_block_table(self.h, seq_id, None, 0)
        if n < 0:
            return None
        out = np.zeros(max(n, 1), np.uint32)
        lib().orc_cache_block_table(self.h, seq_id, _p(out), n)
        return [int(x) for x in out[:n]]

    def free_list(self):
        out = np.zeros(max(self.total_blocks(), 1), np.uint32)
        n = lib().orc_cache_free_list(self.h, _p(out))
        return [int(x) for x in out[:n]]

    def total_blocks(self):
        return lib().orc_cache_total_blocks(self.h)

    def free_blocks(self):
        return lib().orc_cache_free_blocks(self.h)

    def used_blocks(self):
        return lib().orc_cache_used_blocks(self.h)

    def capacity_tokens(self):
        return lib().orc_cache_capacity_tokens(self.h)

    def num_sequences(self):
        return lib().orc_cache_num_sequences(self.h)

    def used_tokens(self):
        return lib().orc_cache_used_tokens(self.h)


# ---------------------------------------------------------------- attention & paging

def attention(q, keys, values, num_heads, num_kv_heads, head_dim, scale=None) -> np.ndarray:
    """attention() over a contiguous [pos][Hkv][d] f32 history (cpu.rs:1126-1151)."""
    q = np.ascontiguousarray(q, np.float32)
    keys = np.ascontiguousarray(keys, np.float32)
    values = np.ascontiguousarray(values, np.float32)
    positions = keys.size // (num_kv_heads * head_dim)
    if scale is None:
        scale = np.float32(1.0) / np.sqrt(np.float32(head_dim))
    ctx = np.zeros(num_heads * head_dim, np.float32)
    lib().orc_attention(_p(q), _p(keys), _p(values), positions, num_heads, num_kv_heads,
                        head_dim, float(scale), _p(ctx))
    return ctx


def paged_append(k_pool, v_pool, k_src, v_src, slots, num_kv_heads, head_dim, block_size):
    """In-place append into numpy pools (uint8 views allowed) through slot mapping."""
    dt = dtype_code(k_src.dtype)
    slots = np.ascontiguousarray(slots, np.int64)
    eb = 4 if dt == F32 else 2
    num_blocks = k_pool.nbytes // (num_kv_heads * head_dim * block_size * eb)
    lib().orc_paged_append(_p(k_pool), _p(v_pool), _p(np.ascontiguousarray(k_src)),
                           _p(np.ascontiguousarray(v_src)), _p(slots), len(slots),
                           num_kv_heads, head_dim, block_size, dt, num_blocks)


def gather_logical(k_pool, v_pool, table, ctx, num_kv_heads, head_dim, block_size, dtype):
    dt = dtype_code(dtype)
    table = np.ascontiguousarray(table, np.int32)
    keys = np.zeros((ctx, num_kv_heads, head_dim), np.float32)
    values = np.zeros_like(keys)
    lib().orc_paged_gather_logical(_p(k_pool), _p(v_pool), _p(table), ctx, num_kv_heads,
                                   head_dim, block_size, dt, _p(keys), _p(values))
    return keys, values


def paged_attention(q, k_pool, v_pool, tables, ctx_lens, nq, num_heads, num_kv_heads,
                    head_dim, block_size, scale) -> np.ndarray:
    """Paged (multi-query causal) attention; returns f32 [B][nq][Hq][d]."""
    dt = dtype_code(q.dtype)
    q = np.ascontiguousarray(q)
    tables = np.ascontiguousarray(tables, np.int32)
    ctx_lens = np.ascontiguousarray(ctx_lens, np.int32)
    B = len(ctx_lens)
    out = np.zeros((B, nq, num_heads, head_dim), np.float32)
    lib().orc_paged_attention(_p(out), _p(q), _p(k_pool), _p(v_pool), dt, _p(tables),
                              _p(ctx_lens), B, nq, num_heads, num_kv_heads, head_dim,
                              block_size, tables.shape[1], float(scale))
    return out


def copy_blocks(k_pool, v_pool, pairs, block_bytes):
    pairs = np.ascontiguousarray(pairs, np.int32)
    lib().orc_copy_blocks(_p(k_pool), _p(v_pool), _p(pairs), len(pairs), block_bytes)


def gather_blocks(k_pool, v_pool, ids, block_bytes) -> np.ndarray:
    ids = np.ascontiguousarray(ids, np.int32)
    staging = np.zeros(2 * len(ids) * block_bytes, np.uint8)
    lib().orc_gather_blocks(_p(staging), _p(k_pool), _p(v_pool), _p(ids), len(ids), block_bytes)
    return staging


def scatter_blocks(k_pool, v_pool, staging, ids, block_bytes):
    ids = np.ascontiguousarray(ids, np.int32)
    lib().orc_scatter_blocks(_p(k_pool), _p(v_pool), _p(np.ascontiguousarray(staging)), _p(ids),
                             len(ids), block_bytes)


def quantize_i8(x):
    x = np.ascontiguousarray(x, np.float32)
    q = np.zeros(x.size, np.int8)
    s = lib().orc_quantize_i8(_p(x), x.size, _p(q))
    return q, np.float32(s)


def quantize_i4(x):
    x = np.ascontiguousarray(x, np.float32)
    packed = np.zeros((x.size + 1) // 2, np.uint8)
    s = lib().orc_quantize_i4(_p(x), x.size, _p(packed))
    return packed, np.float32(s)


def read_i4(packed, base, i) -> float:
    packed = np.ascontiguousarray(packed, np.uint8)
    return lib().orc_read_i4(_p(packed), base, i)


# ---------------------------------------------------------------- quantized KV (int8 / int4)

def quant_row_bytes(kv_dim, quant):
    return kv_dim if quant == I8 else (kv_dim + 1) // 2


def quantize_tokens(src, quant):
    """KvLayerCache::append for Int8/Int4 (cpu.rs:780-793): src [n, kv_dim] f32 ->
    (codes [n, row_bytes] int8|uint8, scales [n] f32)."""
    src = np.ascontiguousarray(src, np.float32)
    n, kv_dim = src.shape
    codes = np.zeros((n, quant_row_bytes(kv_dim, quant)), np.int8 if quant == I8 else np.uint8)
    scales = np.zeros(n, np.float32)
    lib().orc_quantize_tokens(_p(src), n, kv_dim, quant, _p(codes), _p(scales))
    return codes, scales


def attention_quant(q, kcodes, kscales, vcodes, vscales, num_heads, num_kv_heads, head_dim,
                    quant, scale=None):
    """attention() over an Int8/Int4 KvLayerCache (cpu.rs:1126-1151 with :798-846)."""
    q = np.ascontiguousarray(q, np.float32)
    if scale is None:
        scale = np.float32(1.0) / np.sqrt(np.float32(head_dim))
    ctx = np.zeros(num_heads * head_dim, np.float32)
    lib().orc_attention_quant(_p(q), _p(np.ascontiguousarray(kcodes)),
                              _p(np.ascontiguousarray(kscales, np.float32)),
                              _p(np.ascontiguousarray(vcodes)),
                              _p(np.ascontiguousarray(vscales, np.float32)), len(kscales),
                              num_heads, num_kv_heads, head_dim, float(scale), quant, _p(ctx))
    return ctx


def quant_groups(d, quant):
    """(KG, VG): dims per K chunk and per V lane group of the paged quantized
    tiles (orc_quant_k_group / orc_quant_v_group)."""
    if d % 64:
        raise ValueError("quantized pools need head_dim % 64 == 0")
    if quant == I8:
        return 16, 4
    return (32, 8) if d % 128 == 0 else (16, 4)


def quant_pool_shapes(num_blocks, Hkv, d, quant, bs=16):
    """K [nb][Hkv][d/KG][16][KG codes], V [nb][Hkv][d/(16 VG)][4][16][VG * 4 codes]
    (int4 codes two to a byte)."""
    kg, vg = quant_groups(d, quant)
    per = 2 if quant == I4 else 1
    return ((num_blocks, Hkv, d // kg, bs, kg // per),
            (num_blocks, Hkv, d // (16 * vg), 4, 16, 4 * vg // per))


def paged_append_quant(k_pool, v_pool, k_scales, v_scales, k_src, v_src, slots, Hkv, d, quant,
                       bs=16):
    quant_groups(d, quant)
    slots = np.ascontiguousarray(slots, np.int64)
    k_src = np.ascontiguousarray(k_src, np.float32)
    v_src = np.ascontiguousarray(v_src, np.float32)
    num_blocks = k_scales.size // bs
    lib().orc_paged_append_quant(_p(k_pool), _p(v_pool), _p(k_scales), _p(v_scales), _p(k_src),
                                 _p(v_src), _p(slots), len(slots), Hkv, d, bs, quant, num_blocks)


def paged_gather_quant(k_pool, v_pool, k_scales, v_scales, table, ctx, Hkv, d, quant, bs=16):
    quant_groups(d, quant)
    rb = quant_row_bytes(Hkv * d, quant)
    dt = np.int8 if quant == I8 else np.uint8
    kc, vc = np.zeros((ctx, rb), dt), np.zeros((ctx, rb), dt)
    ks, vs = np.zeros(ctx, np.float32), np.zeros(ctx, np.float32)
    lib().orc_paged_gather_quant(_p(k_pool), _p(v_pool), _p(k_scales), _p(v_scales),
                                 _p(np.ascontiguousarray(table, np.int32)), ctx, Hkv, d, bs, quant,
                                 _p(kc), _p(ks), _p(vc), _p(vs))
    return kc, ks, vc, vs


def paged_attention_quant(q, k_pool, v_pool, k_scales, v_scales, quant, tables, ctx_lens, nq,
                          Hq, Hkv, d, scale, bs=16):
    q = np.ascontiguousarray(q, np.float32)
    tables = np.ascontiguousarray(tables, np.int32)
    ctx_lens = np.ascontiguousarray(ctx_lens, np.int32)
    out = np.zeros((len(ctx_lens), nq, Hq, d), np.float32)
    lib().orc_paged_attention_quant(_p(out), _p(q), _p(k_pool), _p(v_pool), _p(k_scales),
                                    _p(v_scales), quant, _p(tables), _p(ctx_lens), len(ctx_lens),
                                    nq, Hq, Hkv, d, bs, tables.shape[1], float(scale))
    return out


# ---------------------------------------------------------------- decode block

W_F32, W_BF16, W_F16, W_INT4, W_INT8 = 0, 1, 2, 3, 4
QUANT_GROUP_SIZE = 128  # src/forward/cpu.rs:161


def quant_blob_bytes(w_dtype, n, group_size=QUANT_GROUP_SIZE) -> int:
    return lib().orc_quant_blob_bytes(w_dtype, n, group_size)


def quantize_weights(values, w_dtype, group_size=QUANT_GROUP_SIZE) -> np.ndarray:
    """Weights::quantize_int4 / quantize_int8 blob (codes, pad, scales, zeros)."""
    v = np.ascontiguousarray(values, np.float32).ravel()
    blob = np.zeros(quant_blob_bytes(w_dtype, v.size, group_size), np.uint8)
    rc = lib().orc_quantize_weights(_p(v), v.size, group_size, w_dtype, _p(blob))
    if rc != 0:
        raise ValueError("bad quantization arguments")
    return blob


def weight_get(w, w_dtype, n, i, group_size=QUANT_GROUP_SIZE) -> float:
    return lib().orc_weight_get(_p(np.ascontiguousarray(w)), w_dtype, n, group_size, i)


def matvec(w, w_dtype, x, out_dim, in_dim, group_size=QUANT_GROUP_SIZE) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(out_dim, np.float32)
    lib().orc_matvec(_p(np.ascontiguousarray(w)), w_dtype, group_size, _p(x), out_dim, in_dim,
                     _p(y))
    return y


def rmsnorm(x, w, eps) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros_like(x)
    lib().orc_rmsnorm(_p(x), _p(np.ascontiguousarray(w, np.float32)), x.size, eps, _p(out))
    return out


def silu(x: float) -> float:
    return lib().orc_silu(x)


def rope_inv_freqs(head_dim, theta, scaling=None) -> np.ndarray:
    """scaling: None, ("linear", factor) or ("llama3", factor, low, high, original_max)."""
    out = np.zeros(head_dim // 2, np.float32)
    kind, args = 0, (1.0, 1.0, 1.0, 1.0)
    if scaling is not None and scaling[0] == "linear":
        kind, args = 1, (scaling[1], 1.0, 1.0, 1.0)
    elif scaling is not None:
        kind, args = 2, tuple(scaling[1:5])
    lib().orc_rope_inv_freqs(head_dim, theta, kind, *args, _p(out))
    return out


def rope(v, num_heads, head_dim, position, inv_freq) -> np.ndarray:
    v = np.array(v, np.float32)
    lib().orc_rope(_p(v), num_heads, head_dim, position,
                   _p(np.ascontiguousarray(inv_freq, np.float32)))
    return v


def decode_block_paged(cfg, weights, x, k_pool, v_pool, table, num_positions, position,
                       inv_freq, bs=16):
    """decode_block over a paged f32 pool (pools updated in place); returns the new hidden.

    cfg: dict with hidden_size, num_heads, num_kv_heads, head_dim, inter, rms_eps, w_dtype,
    w_group_size.  weights: dict q_proj k_proj v_proj o_proj gate_proj up_proj down_proj
    in_norm post_norm and optional q_bias k_bias v_bias."""
    c = BlockConfigC(cfg["hidden_size"], cfg["num_heads"], cfg["num_kv_heads"], cfg["head_dim"],
                     cfg["inter"], cfg["rms_eps"], cfg["w_dtype"], cfg.get("w_group_size", 0))
    x = np.array(x, np.float32)
    table = np.ascontiguousarray(table, np.int32)
    names = ["q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj",
             "in_norm", "post_norm", "q_bias", "k_bias", "v_bias"]
    ptrs = [_p(np.ascontiguousarray(weights[n])) if weights.get(n) is not None else None
            for n in names]
    num_blocks = k_pool.shape[0]
    rc = lib().orc_decode_block_paged(C.byref(c), *ptrs, _p(np.ascontiguousarray(inv_freq,
                                      np.float32)), _p(x), _p(k_pool), _p(v_pool), _p(table),
                                      table.size, num_blocks, bs, num_positions, position)
    if rc != 0:
        raise ValueError("decode_block_paged: table too short")
    return x
