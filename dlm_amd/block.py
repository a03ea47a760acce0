"""One decode block on the GPU over the paged KV cache: the host mirror of
dlm's GPU compute kernel with its per-kernel contiguous KV replaced by paged
pools (``dlmk_decode_block_paged``).

Mirrors, by name and argument meaning:
  * ``BlockConfig`` (src/forward/cpu.rs:48-92): hidden_size, num_heads,
    num_kv_heads, head_dim, intermediate_size, rope_theta, rms_eps,
    rope_scaling; ``q_dim``, ``kv_dim``, ``group_size``.
  * ``rope_inv_freqs`` (src/forward/cpu.rs:1057-1092): the host-side RoPE
    frequencies the device reads (the reference uploads them once too).
  * ``PagedGpuKernel`` -- ``ComputeKernel`` (src/forward/kernel.rs:22-48) as
    ``GpuKernel`` implements it (src/forward/gpu.rs): per-layer weights resident
    on the device in their checkpoint dtype, ``run_block(layer, hidden, kv,
    position)`` running one token through one layer.  ``kv`` is the layer's
    paged pools plus the sequence's device block table instead of a
    ``KvLayerCache``.
  * ``decode_token`` -- ``ForwardOrchestrator::decode_token``
    (src/forward/orchestrator.rs:107-128): reserve the token in the
    ``PagedKvCache`` books (append_tokens, the budget check), then run every
    layer at that position.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import numpy as np
import torch

from ._lib import check, lib
from .ops import BLOCK_SIZE, _dev, _stream

W_F32, W_BF16, W_F16, W_INT4, W_INT8 = 0, 1, 2, 3, 4  # DLM_W_* (src/gpu/kernels.cu:61-65)
QUANT_GROUP_SIZE = 128  # src/forward/cpu.rs:161


@dataclass(frozen=True)
class BlockConfig:
    hidden_size: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    intermediate_size: int
    rope_theta: float = 10000.0
    rms_eps: float = 1e-5
    # None, ("linear", factor) or ("llama3", factor, low_freq_factor,
    # high_freq_factor, original_max_position)  (RopeScaling, cpu.rs:33-46)
    rope_scaling: Optional[Tuple] = None

    @property
    def q_dim(self) -> int:
        return self.num_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.num_kv_heads * self.head_dim

    @property
    def group_size(self) -> int:
        return self.num_heads // self.num_kv_heads


def rope_inv_freqs(head_dim: int, theta: float, scaling: Optional[Tuple] = None) -> np.ndarray:
    """head_dim / 2 inverse frequencies, scaling folded in, in f32 arithmetic."""
    f32 = np.float32
    out = np.empty(head_dim // 2, f32)
    for i in range(head_dim // 2):
        base = f32(np.power(f32(theta), f32(-2.0) * f32(i) / f32(head_dim), dtype=f32))
        f = base
        if scaling is not None and scaling[0] == "linear":
            f = f32(base / f32(scaling[1]))
        elif scaling is not None:
            factor, low, high, orig = (f32(v) for v in scaling[1:5])
            wavelen = f32(f32(2.0) * f32(math.pi) / base)
            if wavelen > orig / low:
                f = f32(base / factor)
            elif wavelen < orig / high:
                f = base
            else:
                smooth = f32((orig / wavelen - low) / (high - low))
                f = f32((f32(1.0) - smooth) * base / factor + smooth * base)
        out[i] = f
    return out


@dataclass
class LayerWeights:
    """One layer's tensors on the device.  Matrices are raw byte tensors in the
    checkpoint dtype (row-major [out, in]); int4/int8 are dlm's group-affine
    blobs.  Norms and biases are f32; biases may be None."""

    q_proj: torch.Tensor
    k_proj: torch.Tensor
    v_proj: torch.Tensor
    o_proj: torch.Tensor
    gate_proj: torch.Tensor
    up_proj: torch.Tensor
    down_proj: torch.Tensor
    input_layernorm: torch.Tensor
    post_attention_layernorm: torch.Tensor
    q_bias: Optional[torch.Tensor] = None
    k_bias: Optional[torch.Tensor] = None
    v_bias: Optional[torch.Tensor] = None


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def weight_bytes(w_dtype: int, n: int, group_size: int = QUANT_GROUP_SIZE) -> int:
    """Bytes of an n-element matrix in this dtype (QuantLayout for int4/int8,
    src/forward/cpu.rs:132-159)."""
    if w_dtype == W_F32:
        return 4 * n
    if w_dtype in (W_BF16, W_F16):
        return 2 * n
    if w_dtype not in (W_INT4, W_INT8) or group_size <= 0:
        raise ValueError(f"bad weight dtype {w_dtype} / group size {group_size}")
    code = (n + 1) // 2 if w_dtype == W_INT4 else n
    groups = -(-n // group_size)
    return (code + 3) // 4 * 4 + 8 * groups


def _check_layer(cfg: BlockConfig, w: LayerWeights, w_dtype: int, group_size: int) -> None:
    """Every operand the kernels read has exactly the size they assume."""
    H, qd, kvd, I = cfg.hidden_size, cfg.q_dim, cfg.kv_dim, cfg.intermediate_size
    mats = {"q_proj": qd * H, "k_proj": kvd * H, "v_proj": kvd * H, "o_proj": H * qd,
            "gate_proj": I * H, "up_proj": I * H, "down_proj": H * I}
    for name, n in mats.items():
        t = getattr(w, name)
        _dev(t, name)
        want = weight_bytes(w_dtype, n, group_size)
        if t.numel() * t.element_size() != want:
            raise ValueError(f"{name}: {t.numel() * t.element_size()} bytes, expected {want}")
    vecs = {"input_layernorm": H, "post_attention_layernorm": H, "q_bias": qd, "k_bias": kvd,
            "v_bias": kvd}
    for name, n in vecs.items():
        t = getattr(w, name)
        if t is None and name.endswith("bias"):
            continue
        _dev(t, name)
        if t.dtype != torch.float32 or t.numel() != n:
            raise ValueError(f"{name} must be float32 [{n}]")


class PagedGpuKernel:
    """``ComputeKernel`` over paged KV: weights resident, one launch sequence
    (rmsnorm, GEMVs, RoPE + append, attention, residuals, SwiGLU) per
    ``run_block``, all on the caller's stream, never synchronising."""

    def __init__(self, cfg: BlockConfig, layers: Sequence[LayerWeights], w_dtype: int,
                 w_group_size: int = 0, max_blocks_per_seq: int = 256, device="cuda"):
        self.cfg = cfg
        self.layers = list(layers)
        self.w_dtype = w_dtype
        self.w_group_size = w_group_size if w_dtype in (W_INT4, W_INT8) else 0
        for w in self.layers:
            _check_layer(cfg, w, w_dtype, self.w_group_size)
        self.max_blocks = max_blocks_per_seq
        self.device = device
        self.inv_freq = torch.from_numpy(
            rope_inv_freqs(cfg.head_dim, cfg.rope_theta, cfg.rope_scaling)).to(device)
        nbytes = lib().dlmk_decode_block_workspace_size(
            cfg.hidden_size, cfg.q_dim, cfg.kv_dim, cfg.num_heads, cfg.head_dim,
            cfg.intermediate_size, max_blocks_per_seq)
        self.workspace = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        self._verify_ws = {}  # num_tokens -> workspace of dlmk_verify_block_paged

    # ComputeKernel surface (src/forward/kernel.rs:22-48)
    def num_layers(self) -> int:
        return len(self.layers)

    def hidden_size(self) -> int:
        return self.cfg.hidden_size

    def kv_dim(self) -> int:
        return self.cfg.kv_dim

    def _check_kv(self, hidden: torch.Tensor, n: int, kv, block_table: torch.Tensor) -> None:
        c = self.cfg
        k_pool, v_pool = kv
        for t, nm in ((hidden, "hidden"), (k_pool, "k_pool"), (v_pool, "v_pool"),
                      (block_table, "block_table")):
            _dev(t, nm)
        if hidden.dtype != torch.float32 or hidden.numel() != n * c.hidden_size:
            raise ValueError(f"hidden must be float32 [{n} x {c.hidden_size}]")
        if k_pool.dtype != torch.float32 or v_pool.dtype != torch.float32:
            raise TypeError("the decode block's pools are float32 (dlm's KV history is f32)")
        tile = c.kv_dim * BLOCK_SIZE
        if k_pool.numel() % tile or v_pool.numel() != k_pool.numel():
            raise ValueError("pools must be [num_blocks, num_kv_heads, head_dim * 16] float32")
        if block_table.dtype != torch.int32 or block_table.numel() != self.max_blocks:
            raise ValueError(f"block_table must be int32 [{self.max_blocks}]")

    def _weights(self, layer: int):
        c, w = self.cfg, self.layers[layer]
        return (c.hidden_size, c.q_dim, c.kv_dim, c.num_heads, c.num_kv_heads, c.head_dim,
                c.intermediate_size, c.rms_eps, self.w_dtype, self.w_group_size,
                _ptr(w.q_proj), _ptr(w.k_proj), _ptr(w.v_proj), _ptr(w.o_proj),
                _ptr(w.gate_proj), _ptr(w.up_proj), _ptr(w.down_proj), _ptr(w.input_layernorm),
                _ptr(w.post_attention_layernorm), _ptr(w.q_bias), _ptr(w.k_bias),
                _ptr(w.v_bias), _ptr(self.inv_freq))

    def run_block(self, layer: int, hidden: torch.Tensor, kv: Tuple[torch.Tensor, torch.Tensor],
                  block_table: torch.Tensor, num_positions: int, position: int,
                  stream=None) -> None:
        """hidden: f32 [hidden_size] on the device, updated in place.  kv: this
        layer's f32 pools; block_table: int32 [max_blocks] of the sequence."""
        self._check_kv(hidden, 1, kv, block_table)
        k_pool, v_pool = kv
        tile = self.cfg.kv_dim * BLOCK_SIZE
        check(lib().dlmk_decode_block_paged(
            _stream(stream), *self._weights(layer), _ptr(hidden), _ptr(k_pool), _ptr(v_pool),
            k_pool.numel() // tile, _ptr(block_table), self.max_blocks, num_positions, position,
            _ptr(self.workspace), self.workspace.numel()))

    def verify_workspace(self, n: int) -> torch.Tensor:
        """The workspace of dlmk_verify_block_paged over n tokens (allocated on
        first use, then reused)."""
        ws = self._verify_ws.get(n)
        if ws is None:
            c = self.cfg
            nbytes = lib().dlmk_verify_block_workspace_size(
                c.hidden_size, c.q_dim, c.kv_dim, c.num_heads, c.head_dim, c.intermediate_size,
                self.max_blocks, n)
            ws = self._verify_ws[n] = torch.empty(max(nbytes, 256), dtype=torch.uint8,
                                                  device=self.device)
        return ws

    def run_tokens(self, layer: int, hidden: torch.Tensor, kv: Tuple[torch.Tensor, torch.Tensor],
                   block_table: torch.Tensor, num_positions: int, position: int,
                   stream=None) -> None:
        """run_block over n consecutive tokens in one pass (the batched verify
        of a speculative round): hidden f32 [n, hidden_size], token j at
        position num_positions + j, attending causally."""
        n = hidden.shape[0] if hidden.dim() == 2 else 1
        self._check_kv(hidden, n, kv, block_table)
        ws = self.verify_workspace(n)
        k_pool, v_pool = kv
        tile = self.cfg.kv_dim * BLOCK_SIZE
        check(lib().dlmk_verify_block_paged(
            _stream(stream), *self._weights(layer), _ptr(hidden), _ptr(k_pool), _ptr(v_pool),
            k_pool.numel() // tile, _ptr(block_table), self.max_blocks, num_positions, position,
            n, _ptr(ws), ws.numel()))


def decode_token(kernel: PagedGpuKernel, cache, seq_id: int, hidden: torch.Tensor,
                 pools: List[Tuple[torch.Tensor, torch.Tensor]], stream=None) -> int:
    """ForwardOrchestrator::decode_token over the paged path: reserve one token
    for ``seq_id`` in the books (raises KvCacheExhausted first, as dlm does),
    upload its block table, run every layer.  Returns the token's position."""
    position = cache.sequence_len(seq_id)
    cache.append_tokens(seq_id, 1)
    tables, _ = cache.block_tables([seq_id], kernel.max_blocks)
    table = torch.from_numpy(np.ascontiguousarray(tables[0], np.int32)).to(hidden.device)
    for layer in range(kernel.num_layers()):
        kernel.run_block(layer, hidden, pools[layer], table, position, position, stream)
    return position
