"""Benchmark: paged KV append + paged GQA decode attention, Llama-3-8B shape, 1 GPU.

Workload: one layer, 32 query heads, 8 KV heads,
head_dim 128, f16 K/V/Q ~ N(0,1)*0.5, block_size 16; 64 sequences with
contexts uniform in [128, 4096] (seeded) on non-contiguous blocks of a shuffled
20k-block pool.  One step = append 1 token per sequence + paged decode
attention over the whole context.  Two disjoint batches alternate step by step
so the bytes read per step come from HBM, not the 256 MB Infinity Cache.

Prints one JSON line (see `result` below).  `value` is the whole step's
algorithmic HBM bytes (attention + append) per second.  The roofline object
covers the dominant kernel, the attention partition kernel; its duration is
measured with HIP events on the stream the kernels run on.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E
HQ, HKV, D, BS = 32, 8, 128, 16
BATCH, CTX_LO, CTX_HI, POOL_BLOCKS, SEED = 64, 128, 4096, 20000, 2


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200, help="timed steps (a multiple of 20)")
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="bound on the CPU baseline sample's work")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run dlmk_copy_blocks over 4096 pairs of 32-KiB blocks in each of 2 pools (256 MiB read + "
                        "256 MiB written per launch), to scale FETCH_SIZE/WRITE_SIZE counters")
    return p.parse_args()


def copy_calibration(torch, ops, steps):
    """A plain copy of known size: 4096 pairs of 32 KiB blocks in each of the K and V pools."""
    dev = torch.device("cuda:0")
    nb, bb = 8192, HKV * BS * D * 2
    k = torch.zeros(nb * bb, dtype=torch.uint8, device=dev)
    v = torch.zeros_like(k)
    pairs = torch.stack([torch.arange(0, 4096), torch.arange(4096, 8192)], 1).int().to(dev)
    for _ in range(steps):
        ops.copy_blocks(k, v, pairs, bb)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration": {"launches": steps, "bytes_read_per_launch": 2 * 4096 * bb,
                                           "bytes_written_per_launch": 2 * 4096 * bb}}))


def attn_bytes(ctx, nq=1, out_bytes=2):
    """Algorithmic bytes of one attention launch: K+V read, Q read, out write,
    block table and context lengths."""
    ctx = np.asarray(ctx, np.int64)
    kv = int(ctx.sum()) * 2 * HKV * D * 2
    qo = len(ctx) * nq * HQ * D * (2 + out_bytes)
    meta = int(((ctx + BS - 1) // BS).sum()) * 4 + len(ctx) * 4
    return kv + qo + meta


def append_bytes(n_tok):
    """Per appended token: K+V read (4096 B), written (4096 B), 8-byte slot."""
    return n_tok * (2 * (2 * HKV * D * 2) + 8)


def cpu_baseline(budget_s):
    """dlm's CPU attention path (the oracle restatement, 1 thread) on a bounded
    sample of the same workload: as many config-2 sequences as fit budget_s."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import oracle as orc
    orc.build()
    rng = np.random.default_rng(SEED + 1000)
    ctx_all = rng.integers(CTX_LO, CTX_HI + 1, BATCH)
    done_tok, done_seq, elapsed, nbytes = 0, 0, 0.0, 0
    for c in ctx_all:
        c = int(c)
        nb = -(-c // BS)
        kp = (rng.standard_normal((nb, HKV, D // 8, BS, 8)) * 0.5).astype(np.float16)
        vp = (rng.standard_normal((nb, HKV, D, BS)) * 0.5).astype(np.float16)
        table = rng.permutation(nb).astype(np.int32)[None]
        q = (rng.standard_normal((1, 1, HQ, D)) * 0.5).astype(np.float16)
        t0 = time.perf_counter()
        orc.paged_attention(q, kp, vp, table, np.array([c], np.int32), 1, HQ, HKV, D, BS,
                            1.0 / np.sqrt(D))
        elapsed += time.perf_counter() - t0
        done_tok += c
        done_seq += 1
        nbytes += attn_bytes([c])
        if elapsed >= budget_s:
            break
    return {
        "value": round(nbytes / elapsed / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": (f"oracle/oracle.c paged attention (f32 restatement of dlm attention(), "
                   f"1 thread) over {done_seq} config-2 sequences, {done_tok} context tokens, "
                   f"{elapsed:.1f} s; same algorithmic-bytes formula"),
        "context_tokens_per_s": round(done_tok / elapsed, 1),
        "cpu_model": _cpu_model(), "host_nproc": os.cpu_count(),
    }


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


class Batch:
    """One set of 64 sequences: books, device block tables, slots and inputs."""

    def __init__(self, torch, cache, seq_base, ctx, dev, gen):
        self.seqs = [seq_base + i for i in range(len(ctx))]
        for s, c in zip(self.seqs, ctx):
            cache.append_tokens(s, int(c))  # prefill + the token this step appends
        max_blocks = -(-CTX_HI // BS)
        tables, lens = cache.block_tables(self.seqs, max_blocks)
        slots = np.array([cache.slot_mapping(s, int(c) - 1, 1)[0] for s, c in zip(self.seqs, ctx)],
                         np.int64)
        self.tables = torch.from_numpy(tables).to(dev)
        self.lens = torch.from_numpy(lens).to(dev)
        self.slots = torch.from_numpy(slots).to(dev)
        self.ctx = ctx
        n = len(ctx)
        self.q = (torch.randn((n, 1, HQ, D), generator=gen, device=dev) * 0.5).half()
        self.k_new = (torch.randn((n, HKV, D), generator=gen, device=dev) * 0.5).half()
        self.v_new = (torch.randn((n, HKV, D), generator=gen, device=dev) * 0.5).half()
        self.out = torch.empty((n, 1, HQ, D), dtype=torch.float16, device=dev)


def main():
    args = parse()
    args.steps = max(20, args.steps // 20 * 20)
    if args.gpus != 1:
        print(json.dumps({"error": "bench.py measures one GPU only; every GPU box here has one "
                                   "GPU and multi-GPU runs are out of scope for this path",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    import torch
    from dlm_amd import KvCacheConfig, PagedKvCache, ops

    if args.copy_calibration:
        copy_calibration(torch, ops, args.steps)
        return
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED)

    cfg = KvCacheConfig(num_layers=1, num_kv_heads=HKV, head_dim=D, block_size=BS)
    cache = PagedKvCache.with_seeded_shuffle(cfg, POOL_BLOCKS, seed=SEED)
    geom = ops.PoolGeometry(POOL_BLOCKS, HKV, D, BS, torch.float16)
    (k_pool, v_pool), = ops.alloc_pools(geom, dev)
    k_pool.normal_(0.0, 0.5, generator=gen)
    v_pool.normal_(0.0, 0.5, generator=gen)

    rng = np.random.default_rng(SEED)
    batches = []
    t_books = time.perf_counter()
    for b in range(2):
        ctx = rng.integers(CTX_LO, CTX_HI + 1, BATCH).astype(np.int32)
        batches.append(Batch(torch, cache, b * 1000, ctx, dev, gen))
    books_s = time.perf_counter() - t_books
    ws = ops.alloc_workspace(ops.attention_workspace_bytes(BATCH, 1, HQ, D, -(-CTX_HI // BS)), dev)

    def append(bt):
        ops.kv_append(k_pool, v_pool, bt.k_new, bt.v_new, bt.slots, num_kv_heads=HKV,
                      head_dim=D)

    def attend(bt):
        ops.paged_decode_attention(bt.q, k_pool, v_pool, bt.tables, bt.lens, num_kv_heads=HKV,
                                   out=bt.out, workspace=ws)

    def step(i):
        bt = batches[i & 1]
        append(bt)
        attend(bt)

    stream = torch.cuda.current_stream()
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # The timed work runs as HIP graphs (one per batch and per phase), the way
    # a serving loop replays a fixed decode step: no host launch overhead in
    # the measurement, only the kernels.  Every launch inside is a libdlmk
    # kernel; nothing is captured that writes memory by memset.
    def capture(fn, reps):
        """One graph holding `reps` launches of fn, alternating the two batches
        (amortises the graph launch itself over many kernels)."""
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for r in range(reps):
                fn(batches[r & 1])
        torch.cuda.synchronize()
        return g

    REPS = 20
    g_step = capture(lambda bt: (append(bt), attend(bt)), REPS)
    g_attn = capture(attend, REPS)
    g_app = capture(append, 5 * REPS)
    stream = torch.cuda.current_stream()

    def timed(graph, reps, n):
        for _ in range(max(1, args.warmup // reps)):
            graph.replay()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        for _ in range(n // reps):
            graph.replay()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / (reps * (n // reps))

    # Whole steps.
    t0 = time.perf_counter()
    step_ms = timed(g_step, REPS, args.steps)
    wall_s = time.perf_counter() - t0
    # Attention alone (the dominant kernel pair) and append alone.
    attn_ms = timed(g_attn, REPS, args.steps)
    append_ms = timed(g_app, 5 * REPS, 5 * args.steps)

    mean_attn_bytes = (attn_bytes(batches[0].ctx) + attn_bytes(batches[1].ctx)) / 2
    step_bytes = mean_attn_bytes + append_bytes(BATCH)
    value = step_bytes / (step_ms * 1e-3) / 1e9
    attn_gbps = mean_attn_bytes / (attn_ms * 1e-3) / 1e9
    ctx_tok = (batches[0].ctx.sum() + batches[1].ctx.sum()) / 2

    result = {
        "metric": "paged decode-attn HBM GB/s (% of peak) + KV-append tokens/s, 8B shape, 1 GPU",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1)*0.5 K/V/Q, seeded contexts and shuffled pool)",
        "config": {
            "workload": "configs[1]: Llama-3-8B single layer, paged KV append + GQA decode attention",
            "num_q_heads": HQ, "num_kv_heads": HKV, "head_dim": D, "block_size": BS,
            "batch": BATCH, "ctx": f"U[{CTX_LO},{CTX_HI}] seed {SEED}",
            "pool_blocks": POOL_BLOCKS, "rotating_batches": 2,
            "mean_context_tokens": float(ctx_tok),
            "parallelism": "single GPU",
        },
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBPS, 2),
        "attention": {
            "GBps": round(attn_gbps, 1), "pct_of_hbm_peak": round(100 * attn_gbps / HBM_PEAK_GBPS, 2),
            "us_per_launch": round(attn_ms * 1e3, 2),
            "algorithmic_bytes_per_launch": int(mean_attn_bytes),
            "context_tokens_per_s": round(ctx_tok / (attn_ms * 1e-3), 1),
            "query_tokens_per_s": round(BATCH / (attn_ms * 1e-3), 1),
        },
        "kv_append": {
            "tokens_per_s": round(BATCH / (append_ms * 1e-3), 1),
            "us_per_launch": round(append_ms * 1e3, 2),
            "GBps": round(append_bytes(BATCH) / (append_ms * 1e-3) / 1e9, 2),
        },
        "host_books_s_for_128_seqs": round(books_s, 4),
        "wall_s_timed_region": round(wall_s, 4),
        "timing": "HIP events around replays of HIP graphs of 20 steps each (100 appends for the append-only line), alternating the two batches",
        "roofline": {
            "bound": "hbm", "achieved": round(attn_gbps, 1), "peak": HBM_PEAK_GBPS,
            "unit": "GB/s", "frac": round(attn_gbps / HBM_PEAK_GBPS, 4), "traffic": None,
            "kernel": "paged_attn_mfma_kernel + paged_attn_combine_kernel (one launch pair)",
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
