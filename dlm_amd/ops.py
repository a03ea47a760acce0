"""Device entry points over torch tensors.

Each function validates shapes, dtypes and devices on the host (so a kernel
never sees an operand its grid does not expect), then calls the matching
``dlmk_*`` C entry point of libdlmk.so on torch's current HIP stream.  torch is
used only for device memory and the stream handle; all device work is the
hand-written HIP in ``dlm_amd/csrc``.  There is no fallback path: a missing
library raises on the first call.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch

from ._lib import DLMK_BF16, DLMK_F16, DLMK_F32, DLMK_I4, DLMK_I8, check, lib

BLOCK_SIZE = 16  # tokens per block; dlm hard-codes 16 (src/main.rs:455, src/loader.rs:597)

_DT = {torch.float32: DLMK_F32, torch.float16: DLMK_F16, torch.bfloat16: DLMK_BF16}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DT[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt} (float32, float16, bfloat16)") from None


def _stream(stream=None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _dev(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must live on the GPU (got {t.device})")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


@dataclass(frozen=True)
class PoolGeometry:
    """Shape of one layer's K and V pools."""

    num_blocks: int
    num_kv_heads: int
    head_dim: int
    block_size: int = BLOCK_SIZE
    dtype: torch.dtype = torch.float16

    @property
    def elem_bytes(self) -> int:
        return torch.tensor([], dtype=self.dtype).element_size()

    @property
    def chunk_elems(self) -> int:
        """X: elements per 16-byte K chunk."""
        return 16 // self.elem_bytes

    @property
    def block_bytes(self) -> int:
        """Bytes of one block of one pool (all kv heads)."""
        return self.num_kv_heads * self.block_size * self.head_dim * self.elem_bytes

    def k_shape(self):
        x = self.chunk_elems
        return (self.num_blocks, self.num_kv_heads, self.head_dim // x, self.block_size, x)

    def v_shape(self):
        return (self.num_blocks, self.num_kv_heads, self.head_dim, self.block_size)


def alloc_pools(geom: PoolGeometry, device="cuda", num_layers: int = 1):
    """Allocate [num_layers] pairs of (K pool, V pool) in the library's layout."""
    if (geom.head_dim * geom.elem_bytes) % 16 != 0:
        raise ValueError("head_dim * element bytes must be a multiple of 16")
    pools = [(torch.empty(geom.k_shape(), dtype=geom.dtype, device=device),
              torch.empty(geom.v_shape(), dtype=geom.dtype, device=device))
             for _ in range(num_layers)]
    return pools


def _pool_geom(k_pool: torch.Tensor, v_pool: torch.Tensor, num_kv_heads: int, head_dim: int,
               block_size: int) -> int:
    _dev(k_pool, "k_pool")
    _dev(v_pool, "v_pool")
    if k_pool.dtype != v_pool.dtype or k_pool.numel() != v_pool.numel():
        raise ValueError("k_pool and v_pool must have one dtype and size")
    per_block = num_kv_heads * head_dim * block_size
    if k_pool.numel() % per_block != 0:
        raise ValueError(f"pool of {k_pool.numel()} elements is not whole blocks of {per_block}")
    return k_pool.numel() // per_block


def kv_append(k_pool, v_pool, k, v, slot_mapping, *, num_kv_heads: int, head_dim: int,
              block_size: int = BLOCK_SIZE, stream=None) -> None:
    """Scatter tokens k, v ([n, Hkv, d]) into their slots (paged KvLayerCache::append)."""
    num_blocks = _pool_geom(k_pool, v_pool, num_kv_heads, head_dim, block_size)
    for t, nm in ((k, "k"), (v, "v")):
        _dev(t, nm)
        if t.dtype != k_pool.dtype:
            raise TypeError(f"{nm} dtype {t.dtype} != pool dtype {k_pool.dtype}")
    _dev(slot_mapping, "slot_mapping")
    if slot_mapping.dtype != torch.int64:
        raise TypeError("slot_mapping must be int64")
    n = slot_mapping.numel()
    if k.numel() != n * num_kv_heads * head_dim or v.numel() != k.numel():
        raise ValueError(f"k/v hold {k.numel()}/{v.numel()} elements, expected "
                         f"{n}x{num_kv_heads}x{head_dim}")
    check(lib().dlmk_kv_append(_stream(stream), k_pool.data_ptr(), v_pool.data_ptr(),
                               k.data_ptr(), v.data_ptr(), slot_mapping.data_ptr(), n,
                               num_kv_heads, head_dim, block_size, num_blocks,
                               dtype_code(k_pool.dtype)))


def attention_workspace_bytes(num_seqs: int, num_q_per_seq: int, num_q_heads: int,
                              head_dim: int, max_blocks_per_seq: int,
                              block_size: int = BLOCK_SIZE) -> int:
    return lib().dlmk_paged_attention_workspace_size(num_seqs, num_q_per_seq, num_q_heads,
                                                     head_dim, block_size, max_blocks_per_seq)


def alloc_workspace(nbytes: int, device="cuda") -> Optional[torch.Tensor]:
    if nbytes == 0:
        return None
    # torch's caching allocator returns >= 256-byte aligned blocks.
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def _attention_call(q, k_pool, v_pool, block_tables, ctx_lens, num_kv_heads, scale, out,
                    out_dtype, workspace, block_size, stream, k_new=None, v_new=None,
                    quant: Optional["QuantKv"] = None):
    _dev(q, "q")
    if q.dim() != 4:
        raise ValueError("q must be [num_seqs, num_q_per_seq, num_q_heads, head_dim]")
    B, nq, Hq, d = q.shape
    if quant is None:
        num_blocks = _pool_geom(k_pool, v_pool, num_kv_heads, d, block_size)
        if q.dtype != k_pool.dtype:
            raise TypeError(f"q dtype {q.dtype} != pool dtype {k_pool.dtype}")
    else:
        num_blocks = quant.check(num_kv_heads, d, block_size)
        if q.dtype != torch.float16:
            raise TypeError(f"q must be float16 for quantized pools (got {q.dtype})")
    _dev(block_tables, "block_tables")
    _dev(ctx_lens, "ctx_lens")
    if block_tables.dtype != torch.int32 or ctx_lens.dtype != torch.int32:
        raise TypeError("block_tables and ctx_lens must be int32")
    if block_tables.dim() != 2 or block_tables.shape[0] != B or ctx_lens.numel() != B:
        raise ValueError("block_tables must be [B, max_blocks] and ctx_lens [B]")
    if k_new is not None:
        for t, nm in ((k_new, "k_new"), (v_new, "v_new")):
            _dev(t, nm)
            if t.dtype != k_pool.dtype:
                raise TypeError(f"{nm} dtype {t.dtype} != pool dtype {k_pool.dtype}")
            if t.numel() != B * nq * num_kv_heads * d:
                raise ValueError(f"{nm} must be [{B}, {nq}, {num_kv_heads}, {d}]")
    max_blocks = block_tables.shape[1]
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if out is None:
        out = torch.empty((B, nq, Hq, d), dtype=out_dtype or q.dtype, device=q.device)
    _dev(out, "out")
    if out.numel() != q.numel():
        raise ValueError("out must have q's shape")
    need = attention_workspace_bytes(B, nq, Hq, d, max_blocks, block_size)
    if workspace is None:
        workspace = alloc_workspace(need, q.device)
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    tail = (block_tables.data_ptr(), ctx_lens.data_ptr(), B, nq, Hq, num_kv_heads, d, block_size,
            max_blocks, num_blocks, float(scale), ws_ptr, ws_bytes)
    if quant is not None:
        check(lib().dlmk_paged_decode_attention_quant(
            _stream(stream), out.data_ptr(), dtype_code(out.dtype), q.data_ptr(),
            quant.k.data_ptr(), quant.v.data_ptr(), quant.k_scales.data_ptr(),
            quant.v_scales.data_ptr(), quant.code, *tail))
        return out
    head = (_stream(stream), out.data_ptr(), dtype_code(out.dtype), q.data_ptr(),
            k_pool.data_ptr(), v_pool.data_ptr(), dtype_code(q.dtype))
    if k_new is None:
        check(lib().dlmk_paged_decode_attention(*head, *tail))
    else:
        check(lib().dlmk_paged_decode_step(*head, k_new.data_ptr(), v_new.data_ptr(), *tail))
    return out


def paged_decode_attention(q, k_pool, v_pool, block_tables, ctx_lens, *, num_kv_heads: int,
                           scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
                           out_dtype: Optional[torch.dtype] = None,
                           workspace: Optional[torch.Tensor] = None,
                           block_size: int = BLOCK_SIZE, stream=None) -> torch.Tensor:
    """Paged GQA decode attention.

    q: [B, nq, Hq, d] (nq > 1 is causal speculative verify); block_tables int32
    [B, max_blocks]; ctx_lens int32 [B].  Returns out [B, nq, Hq, d]."""
    return _attention_call(q, k_pool, v_pool, block_tables, ctx_lens, num_kv_heads, scale, out,
                           out_dtype, workspace, block_size, stream)


def paged_decode_step(q, k_new, v_new, k_pool, v_pool, block_tables, ctx_lens, *,
                      num_kv_heads: int, scale: Optional[float] = None,
                      out: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None,
                      workspace: Optional[torch.Tensor] = None, block_size: int = BLOCK_SIZE,
                      stream=None) -> torch.Tensor:
    """Fused decode step: append each sequence's nq newest tokens (k_new, v_new:
    [B, nq, Hkv, d], at positions ctx - nq .. ctx - 1) and attend, in one launch.
    Equivalent to kv_append followed by paged_decode_attention."""
    return _attention_call(q, k_pool, v_pool, block_tables, ctx_lens, num_kv_heads, scale, out,
                           out_dtype, workspace, block_size, stream, k_new, v_new)


_QUANT = {"int8": (DLMK_I8, 8), "int4": (DLMK_I4, 4)}


@dataclass(frozen=True)
class QuantKv:
    """One layer's quantized KV pools (dlm's --kv-quant int8 / int4).

    k, v: uint8 code pools; k_scales, v_scales: float32 [num_blocks, block_size],
    one scale per token slot over the whole kv_dim."""

    k: torch.Tensor
    v: torch.Tensor
    k_scales: torch.Tensor
    v_scales: torch.Tensor
    quant: str

    @property
    def code(self) -> int:
        return _QUANT[self.quant][0]

    @property
    def bits(self) -> int:
        return _QUANT[self.quant][1]

    @property
    def num_blocks(self) -> int:
        return self.k_scales.shape[0]

    def block_bytes(self) -> int:
        """Bytes of one block of one code pool."""
        return self.k.numel() // self.num_blocks

    def check(self, num_kv_heads: int, head_dim: int, block_size: int) -> int:
        """Validate against (Hkv, d, block_size); return num_blocks."""
        if self.quant not in _QUANT:
            raise ValueError(f"quant must be int8 or int4 (got {self.quant!r})")
        for t, nm in ((self.k, "k"), (self.v, "v"), (self.k_scales, "k_scales"),
                      (self.v_scales, "v_scales")):
            _dev(t, nm)
        if self.k.dtype != torch.uint8 or self.v.dtype != torch.uint8:
            raise TypeError("quantized code pools must be uint8")
        if self.k_scales.dtype != torch.float32 or self.v_scales.dtype != torch.float32:
            raise TypeError("scales must be float32")
        nb = self.num_blocks
        if self.k_scales.shape != (nb, block_size) or self.v_scales.shape != (nb, block_size):
            raise ValueError("scales must be [num_blocks, block_size]")
        per_block = num_kv_heads * head_dim * block_size * self.bits // 8
        if self.k.numel() != nb * per_block or self.v.numel() != nb * per_block:
            raise ValueError(f"code pools must hold {nb} blocks of {per_block} bytes")
        return nb


def alloc_quant_pools(num_blocks: int, num_kv_heads: int, head_dim: int, quant: str,
                      device="cuda", block_size: int = BLOCK_SIZE) -> QuantKv:
    """Allocate one layer's int8 / int4 pools in the library's layout (head_dim
    a multiple of 64; codes offset binary, c + 128 / c + 8, int4 two to a byte):
    K [nb, Hkv, d/KG, 16, KG], V [nb, Hkv, d/(16 VG), 4, 16, 4 VG] with KG, VG =
    16, 4 for int8 and 32, 8 (d % 128 == 0) or 16, 4 for int4; scales [nb, 16]
    float32 (zero)."""
    if quant not in _QUANT:
        raise ValueError(f"quant must be int8 or int4 (got {quant!r})")
    if head_dim % 64 != 0:
        raise ValueError("head_dim must be a multiple of 64")
    nb, H, d, bs = num_blocks, num_kv_heads, head_dim, block_size
    kg, vg = (16, 4) if quant == "int8" or d % 128 else (32, 8)
    per = 1 if quant == "int8" else 2
    ks, vs = (nb, H, d // kg, bs, kg // per), (nb, H, d // (16 * vg), 4, 16, 4 * vg // per)
    return QuantKv(torch.zeros(ks, dtype=torch.uint8, device=device),
                   torch.zeros(vs, dtype=torch.uint8, device=device),
                   torch.zeros((nb, bs), dtype=torch.float32, device=device),
                   torch.zeros((nb, bs), dtype=torch.float32, device=device), quant)


def kv_append_quant(kv: QuantKv, k, v, slot_mapping, *, num_kv_heads: int, head_dim: int,
                    block_size: int = BLOCK_SIZE, stream=None) -> None:
    """Quantize tokens k, v ([n, Hkv, d], f32/f16/bf16) per token and scatter
    codes and scales into their slots (KvLayerCache::append's int8/int4 branch)."""
    nb = kv.check(num_kv_heads, head_dim, block_size)
    for t, nm in ((k, "k"), (v, "v")):
        _dev(t, nm)
    if k.dtype != v.dtype:
        raise TypeError("k and v must share a dtype")
    _dev(slot_mapping, "slot_mapping")
    if slot_mapping.dtype != torch.int64:
        raise TypeError("slot_mapping must be int64")
    n = slot_mapping.numel()
    if k.numel() != n * num_kv_heads * head_dim or v.numel() != k.numel():
        raise ValueError(f"k/v hold {k.numel()}/{v.numel()} elements, expected "
                         f"{n}x{num_kv_heads}x{head_dim}")
    check(lib().dlmk_kv_append_quant(_stream(stream), kv.k.data_ptr(), kv.v.data_ptr(),
                                     kv.k_scales.data_ptr(), kv.v_scales.data_ptr(),
                                     k.data_ptr(), v.data_ptr(), dtype_code(k.dtype),
                                     slot_mapping.data_ptr(), n, num_kv_heads, head_dim,
                                     block_size, nb, kv.code))


def paged_decode_attention_quant(q, kv: QuantKv, block_tables, ctx_lens, *, num_kv_heads: int,
                                 scale: Optional[float] = None,
                                 out: Optional[torch.Tensor] = None,
                                 out_dtype: Optional[torch.dtype] = None,
                                 workspace: Optional[torch.Tensor] = None,
                                 block_size: int = BLOCK_SIZE, stream=None) -> torch.Tensor:
    """Paged GQA decode attention over int8 / int4 pools; q float16 [B, nq, Hq, d]."""
    return _attention_call(q, None, None, block_tables, ctx_lens, num_kv_heads, scale, out,
                           out_dtype, workspace, block_size, stream, quant=kv)


def copy_blocks_quant(kv: QuantKv, pairs, stream=None) -> None:
    """Fork / copy-on-write for quantized pools: codes and scales of each pair."""
    copy_blocks(kv.k, kv.v, pairs, kv.block_bytes(), stream)
    copy_blocks(kv.k_scales, kv.v_scales, pairs, kv.k_scales.shape[1] * 4, stream)


def _ids(t: torch.Tensor, name: str, cols: int) -> int:
    _dev(t, name)
    if t.dtype != torch.int32:
        raise TypeError(f"{name} must be int32")
    if cols == 2 and (t.dim() != 2 or t.shape[1] != 2):
        raise ValueError(f"{name} must be [n, 2]")
    return t.shape[0] if cols == 2 else t.numel()


def _block_bytes(k_pool, v_pool, block_bytes: int) -> int:
    _dev(k_pool, "k_pool")
    _dev(v_pool, "v_pool")
    nbytes = k_pool.numel() * k_pool.element_size()
    if v_pool.numel() * v_pool.element_size() != nbytes or nbytes % block_bytes:
        raise ValueError("pools must be equal-sized and whole blocks")
    return nbytes // block_bytes


def copy_blocks(k_pool, v_pool, pairs, block_bytes: int, stream=None) -> None:
    """Copy block src -> dst in both pools for each (src, dst) row of pairs."""
    n = _ids(pairs, "pairs", 2)
    nb = _block_bytes(k_pool, v_pool, block_bytes)
    check(lib().dlmk_copy_blocks(_stream(stream), k_pool.data_ptr(), v_pool.data_ptr(),
                                 pairs.data_ptr(), n, block_bytes, nb))


def gather_blocks(k_pool, v_pool, block_ids, block_bytes: int, staging=None,
                  stream=None) -> torch.Tensor:
    """Device staging [n, 2, block_bytes] of the given blocks (K then V)."""
    n = _ids(block_ids, "block_ids", 1)
    nb = _block_bytes(k_pool, v_pool, block_bytes)
    if staging is None:
        staging = torch.empty((n, 2, block_bytes), dtype=torch.uint8, device=k_pool.device)
    _dev(staging, "staging")
    if staging.numel() * staging.element_size() < 2 * n * block_bytes:
        raise ValueError("staging too small")
    check(lib().dlmk_gather_blocks(_stream(stream), staging.data_ptr(), k_pool.data_ptr(),
                                   v_pool.data_ptr(), block_ids.data_ptr(), n, block_bytes, nb))
    return staging


def scatter_blocks(k_pool, v_pool, staging, block_ids, block_bytes: int, stream=None) -> None:
    n = _ids(block_ids, "block_ids", 1)
    nb = _block_bytes(k_pool, v_pool, block_bytes)
    _dev(staging, "staging")
    if staging.numel() * staging.element_size() < 2 * n * block_bytes:
        raise ValueError("staging too small")
    check(lib().dlmk_scatter_blocks(_stream(stream), k_pool.data_ptr(), v_pool.data_ptr(),
                                    staging.data_ptr(), block_ids.data_ptr(), n, block_bytes,
                                    nb))


class PinnedBuffer:
    """Page-locked host staging from dlmk_alloc_pinned (dlm's PinnedBuffer,
    src/memory/pinned.rs:38-112): at least `nbytes` bytes, rounded up to whole
    pages and zero-initialised; a zero-byte request raises (DlmError::HostAlloc
    there).  Freed with dlmk_free_pinned by free(), on context exit or when
    the object is collected."""

    PAGE = 4096

    def __init__(self, nbytes: int):
        import ctypes
        p = ctypes.c_void_p()
        check(lib().dlmk_alloc_pinned(ctypes.byref(p), int(nbytes)))
        self._ptr = p.value
        self.len = int(nbytes)
        self.capacity = -(-self.len // self.PAGE) * self.PAGE

    def data_ptr(self) -> int:
        if not self._ptr:
            raise ValueError("pinned buffer already freed")
        return self._ptr

    def numpy(self):
        """A uint8 NumPy view of the first `len` bytes (valid until free())."""
        import ctypes
        import numpy as np
        return np.ctypeslib.as_array((ctypes.c_uint8 * self.len).from_address(self.data_ptr()))

    def free(self) -> None:
        if self._ptr:
            ptr, self._ptr = self._ptr, None
            check(lib().dlmk_free_pinned(ptr))

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.free()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _pinned(host, n: int, block_bytes: int) -> None:
    if isinstance(host, PinnedBuffer):
        nbytes = host.len
    else:
        if host.device.type != "cpu" or not host.is_pinned() or not host.is_contiguous():
            raise ValueError("host buffer must be contiguous pinned CPU memory")
        nbytes = host.numel() * host.element_size()
    if nbytes < 2 * n * block_bytes:
        raise ValueError("host buffer too small")


def swap_out(host, k_pool, v_pool, block_ids, block_bytes: int, staging, stream=None) -> None:
    """Gather blocks into device staging, then one async D2H copy into pinned host."""
    n = _ids(block_ids, "block_ids", 1)
    nb = _block_bytes(k_pool, v_pool, block_bytes)
    _pinned(host, n, block_bytes)
    _dev(staging, "staging")
    check(lib().dlmk_swap_out(_stream(stream), host.data_ptr(), k_pool.data_ptr(),
                              v_pool.data_ptr(), block_ids.data_ptr(), n, block_bytes, nb,
                              staging.data_ptr(), staging.numel() * staging.element_size()))


def swap_in(k_pool, v_pool, host, block_ids, block_bytes: int, staging, stream=None) -> None:
    """One async H2D copy into device staging, then scatter into the blocks."""
    n = _ids(block_ids, "block_ids", 1)
    nb = _block_bytes(k_pool, v_pool, block_bytes)
    _pinned(host, n, block_bytes)
    _dev(staging, "staging")
    check(lib().dlmk_swap_in(_stream(stream), k_pool.data_ptr(), v_pool.data_ptr(),
                             host.data_ptr(), block_ids.data_ptr(), n, block_bytes, nb,
                             staging.data_ptr(), staging.numel() * staging.element_size()))
