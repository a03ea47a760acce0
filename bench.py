"""Benchmark: paged KV append + paged GQA decode attention on one MI355X.

Default workload (the metric's configuration):
one Llama-3-8B layer -- 32 query heads, 8 KV heads, head_dim 128, f16 K/V/Q ~
N(0,1)*0.5, block_size 16; 64 sequences with contexts uniform in [128, 4096]
(seeded) on non-contiguous blocks of a shuffled 20k-block pool.  One step =
append 1 token per sequence + paged decode attention over the whole context.
Two disjoint batches alternate step by step so the bytes a step reads come
from HBM, not the 256 MB Infinity Cache.

`--workload config1|config3|config4|config5` runs the other BASELINE.json
configurations the same way (they are parity-test cases for the driver, and
bench lines for the design notes).

Prints one JSON line.  `value` is the whole step's algorithmic HBM bytes
(attention + append) per second; `roofline` covers the dominant kernel
(attention); timing is HIP events around replays of HIP graphs on the stream
the kernels run on.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--workload config2]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from dataclasses import dataclass, field, replace

import numpy as np

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E
BS = 16
SEED = 2
METRIC = "paged decode-attn HBM GB/s (% of peak) + KV-append tokens/s, 8B shape, 1 GPU"


@dataclass
class Workload:
    name: str
    about: str
    hq: int
    hkv: int
    d: int
    dtype: str  # "f16" | "f32"
    batch: int
    ctx: tuple  # uniform [lo, hi]
    nq: int = 1  # tokens appended and queried per sequence per step
    layers: int = 1
    prefill_seqs: int = 0  # chunked-prefill sequences appending alongside
    prefill_chunk: int = 0
    extras: list = field(default_factory=list)  # "fork", "swap"
    quant: str = "none"  # KV storage: "none" (dtype above), "int8", "int4" (dlm's --kv-quant)


WORKLOADS = {
    "config1": Workload("config1", "configs[0]: Llama-3.2-1B KV (16 layers, 32/8 heads, d 64, f32), "
                        "one sequence at 512 + 32 tokens, 1 token appended per layer per step",
                        32, 8, 64, "f32", 1, (544, 544), layers=16),
    "config2": Workload("config2", "configs[1]: Llama-3-8B single layer, paged KV append + GQA decode "
                        "attention, B=64, ctx U[128,4096]", 32, 8, 128, "f16", 64, (128, 4096)),
    "config3": Workload("config3", "configs[2]: continuous batching, 8B shape: 48 decode sequences at "
                        "U[256,8192] + 4 chunked-prefill sequences appending 512 tokens each per step",
                        32, 8, 128, "f16", 48, (256, 8192), prefill_seqs=4, prefill_chunk=512),
    "config4": Workload("config4", "configs[3]: Llama-3-70B single layer (64/8 heads), B=8 x 32768 "
                        "tokens, split-K + LSE merge", 64, 8, 128, "f16", 8, (32768, 32768)),
    "config5": Workload("config5", "configs[4]: speculative verify on the 8B shape, B=32, ctx "
                        "U[1024,8192], 4 drafts appended + 4-query causal attention per step; "
                        "fork of 8 sequences and 25% swap measured separately",
                        32, 8, 128, "f16", 32, (1024, 8192), nq=4, extras=["fork", "swap"]),
}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200, help="timed steps (rounded to a multiple of 20)")
    p.add_argument("--warmup", type=int, default=500,
                   help="untimed steps run before each timed region (lets clocks settle)")
    p.add_argument("--workload", default="config2",
                   choices=sorted(WORKLOADS) + ["block8b", "blockmoves"],
                   help="block8b: dlmk_decode_block_paged on Llama-3-8B layers (the caller "
                        "of the paged path; a design-notes line, not the headline metric); "
                        "blockmoves: block copy / gather / scatter at several sizes with a "
                        "fixed-cost fit")
    p.add_argument("--kv-quant", default="none", choices=["none", "int8", "int4"],
                   help="store K/V as per-token-scaled int8/int4 codes (dlm's --kv-quant); "
                        "queries and new tokens stay f16")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--only", choices=["step", "unfused", "attention", "append"],
                   help="time one phase only (for profiling runs)")
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="bound on the CPU baseline sample's work")
    p.add_argument("--traffic", default="pmc", choices=["pmc", "off"],
                   help="pmc: measure the attention launch's HBM bytes with rocprofv3 --pmc "
                        "(FETCH_SIZE and WRITE_SIZE passes over this script, scaled by the "
                        "same counters on --copy-calibration) before the timed run")
    p.add_argument("--verify-tokens", type=int, default=5,
                   help="block8b: also time dlmk_verify_block_paged over this many tokens "
                        "(a speculative round's gamma + 1; 0 skips it)")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run dlmk_copy_blocks over 4096 pairs of 32-KiB blocks in each of 2 "
                        "pools (256 MiB read + 256 MiB written per launch), to scale "
                        "FETCH_SIZE/WRITE_SIZE counters")
    return p.parse_args()


def elem_bytes(w):
    """Bytes of one query / new-token / output element."""
    return 4 if w.dtype == "f32" else 2


def kv_token_bytes(w):
    """Stored bytes of one token of one pool (all kv heads): elements, or codes
    plus the token's f32 scale."""
    if w.quant == "none":
        return w.hkv * w.d * elem_bytes(w)
    return w.hkv * w.d * (1 if w.quant == "int8" else 0.5) + 4


def attn_bytes(w, ctx, out_bytes):
    """Algorithmic bytes of one attention launch: K+V read (with scales when
    quantized), Q read, out write, block table and context lengths."""
    ctx = np.asarray(ctx, np.int64)
    eb = elem_bytes(w)
    kv = int(int(ctx.sum()) * 2 * kv_token_bytes(w))
    qo = len(ctx) * w.nq * w.hq * w.d * (eb + out_bytes)
    meta = int(((ctx + BS - 1) // BS).sum()) * 4 + len(ctx) * 4
    return kv + qo + meta


def append_bytes(w, n_tok):
    """Per appended token: K+V read, K+V stored (codes and scale when
    quantized), and an 8-byte slot."""
    return n_tok * (2 * (w.hkv * w.d * elem_bytes(w) + kv_token_bytes(w)) + 8)


def _pmc_pass(counter, script_args, timeout_s=120):
    """One rocprofv3 --pmc pass (a single counter, no tracing domains) over this
    script as a child process; returns {kernel name: mean counter value per
    dispatch}.  The child runs alone: this process has not touched the GPU."""
    import csv
    import shutil
    import subprocess
    import tempfile
    prof = shutil.which("rocprofv3")
    if prof is None:
        raise RuntimeError("rocprofv3 not on PATH")
    out = tempfile.mkdtemp(prefix="dlmk_pmc_")
    cmd = ["timeout", "-s", "KILL", str(timeout_s), prof, "--pmc", counter, "--output-format", "csv",
           "-d", out, "-o", "run", "--", sys.executable, os.path.abspath(__file__), *script_args]
    res = subprocess.run(cmd, capture_output=True, text=True, cwd=tempfile.gettempdir())
    if res.returncode != 0:
        raise RuntimeError(f"rocprofv3 --pmc {counter} exited {res.returncode}: {res.stderr[-300:]}")
    sums, counts = {}, {}
    for root, _, files in os.walk(out):
        for f in files:
            if not f.endswith("counter_collection.csv"):
                continue
            with open(os.path.join(root, f)) as fh:
                for row in csv.DictReader(fh):
                    if row.get("Counter_Name") != counter:
                        continue
                    k = row["Kernel_Name"]
                    sums[k] = sums.get(k, 0.0) + float(row["Counter_Value"])
                    counts[k] = counts.get(k, 0) + 1
    shutil.rmtree(out, ignore_errors=True)
    if not sums:
        raise RuntimeError(f"no {counter} rows in rocprofv3 output")
    return {k: sums[k] / counts[k] for k in sums}


def measure_traffic(args):
    """HBM bytes per attention launch (partition + combine kernels): FETCH_SIZE
    and WRITE_SIZE (KiB per dispatch) from their own --pmc passes over
    `--only attention`, each scaled by what the same counter reads for the copy
    calibration kernel, whose bytes are known.  Returns (bytes, detail)."""
    base = ["--workload", args.workload, "--kv-quant", args.kv_quant, "--only", "attention",
            "--steps", "20", "--warmup", "20", "--no-cpu-baseline", "--traffic", "off"]
    cal = ["--copy-calibration", "--steps", "20", "--traffic", "off"]
    known = 2 * 4096 * 8 * BS * 128 * 2  # bytes read (and written) per copy launch
    detail = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        print(f"[bench] rocprofv3 --pmc {counter} passes", file=sys.stderr, flush=True)
        attn = _pmc_pass(counter, base)
        copy = _pmc_pass(counter, cal)
        kib = sum(v for k, v in attn.items() if "paged_attn" in k)
        ckib = sum(v for k, v in copy.items() if "copy_blocks" in k)
        scale = known / (ckib * 1024)
        detail[counter] = {"kib_per_launch": round(kib, 1), "copy_kib_per_launch": round(ckib, 1),
                           "scale": round(scale, 4), "bytes_per_launch": int(kib * 1024 * scale)}
    total = detail["FETCH_SIZE"]["bytes_per_launch"] + detail["WRITE_SIZE"]["bytes_per_launch"]
    return total, detail


def bench_block(args):
    """One decode token through two Llama-3-8B layers (hidden 4096, 32/8 heads,
    head_dim 128, inter 14336) with bf16 weights, f32 paged KV (dlm's KV dtype)
    and a 2048-token history on shuffled blocks, via dlmk_decode_block_paged.
    Two layers with distinct weights (2 x 436 MB, above the 256 MB Infinity
    Cache) so every token streams its weights from HBM.  Timed as HIP-graph
    replays of 10 tokens.  Bytes per token: weights + the KV the attention
    reads + the appended K/V."""
    import torch
    from dlm_amd.block import BlockConfig, LayerWeights, PagedGpuKernel

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED)
    H, Hq, Hkv, d, I, L, ctx = 4096, 32, 8, 128, 14336, 2, 2048
    cfg = BlockConfig(H, Hq, Hkv, d, I, rope_theta=500000.0, rms_eps=1e-5,
                      rope_scaling=("llama3", 8.0, 1.0, 4.0, 8192.0))

    def mat(o, i):
        w = torch.empty((o, i), dtype=torch.bfloat16, device=dev)
        w.uniform_(-0.02, 0.02, generator=gen)
        return w.view(torch.uint8).reshape(-1)

    layers = [LayerWeights(mat(cfg.q_dim, H), mat(cfg.kv_dim, H), mat(cfg.kv_dim, H),
                           mat(H, cfg.q_dim), mat(I, H), mat(I, H), mat(H, I),
                           torch.ones(H, device=dev), torch.ones(H, device=dev))
              for _ in range(L)]
    nblk = -(-(ctx + 1) // BS)
    max_blocks = 256
    kern = PagedGpuKernel(cfg, layers, 1, max_blocks_per_seq=max_blocks, device=dev)
    num_pool = 4 * nblk
    pools = [(torch.randn((num_pool, Hkv, d * BS), generator=gen, device=dev) * 0.5,
              torch.randn((num_pool, Hkv, d * BS), generator=gen, device=dev) * 0.5)
             for _ in range(L)]
    rng = np.random.default_rng(SEED)
    table = np.zeros(max_blocks, np.int32)
    table[:nblk] = rng.permutation(num_pool)[:nblk]
    table_d = torch.from_numpy(table).to(dev)
    x = torch.randn(H, generator=gen, device=dev)

    def token():
        for layer in range(L):
            kern.run_block(layer, x, pools[layer], table_d, ctx, ctx)
            x.mul_(0.5)  # keep the residual stream bounded across replays

    for _ in range(3):
        token()
    torch.cuda.synchronize()
    reps = 10
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            token()
    for _ in range(max(1, args.warmup // 50)):
        g.replay()
    torch.cuda.synchronize()
    n = max(2, args.steps // reps)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(n):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    ms_token = a.elapsed_time(b) / (n * reps)

    verify = None
    nv = args.verify_tokens
    if nv > 0:
        # gamma + 1 tokens at positions ctx .. ctx + nv - 1 through both layers
        # in one pass (the batched target verify of a speculative round).
        xv = torch.randn((nv, H), generator=gen, device=dev)

        def verify_round():
            for layer in range(L):
                kern.run_tokens(layer, xv, pools[layer], table_d, ctx, ctx)
                xv.mul_(0.5)

        for _ in range(3):
            verify_round()
        torch.cuda.synchronize()
        gv = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gv):
            for _ in range(reps):
                verify_round()
        for _ in range(max(1, args.warmup // 50)):
            gv.replay()
        torch.cuda.synchronize()
        a.record()
        for _ in range(n):
            gv.replay()
        b.record()
        torch.cuda.synchronize()
        ms_v = a.elapsed_time(b) / (n * reps)
        verify = {"tokens": nv, "ms_per_round": round(ms_v, 5),
                  "us_per_layer": round(ms_v * 1e3 / L, 2),
                  "sequential_decode_ms": round(nv * ms_token, 5),
                  "speedup_vs_sequential": round(nv * ms_token / ms_v, 2)}
    wbytes = 2 * (cfg.q_dim * H + 2 * cfg.kv_dim * H + H * cfg.q_dim + 3 * I * H)
    kvbytes = (ctx + 1) * 2 * cfg.kv_dim * 4
    tok_bytes = L * (wbytes + kvbytes + 2 * cfg.kv_dim * 4)
    gbps = tok_bytes / (ms_token * 1e-3) / 1e9
    print(json.dumps({
        "metric": "paged decode block HBM GB/s (Llama-3-8B layers, bf16 weights, f32 paged KV)",
        "value": round(gbps, 1), "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
        "ms_per_token": round(ms_token, 5), "us_per_layer": round(ms_token * 1e3 / L, 2),
        "tokens_per_s": round(1e3 / ms_token, 1), "dtype": "bf16 weights, f32 KV and math",
        "data": "synthetic (uniform(-0.02, 0.02) weights, N(0,1)*0.5 KV, seeded)",
        "config": {"workload": "dlmk_decode_block_paged, 2 Llama-3-8B layers, ctx 2048",
                   "hidden": H, "heads": Hq, "kv_heads": Hkv, "head_dim": d, "inter": I,
                   "layers": L, "context": ctx},
        "algorithmic_bytes_per_token": tok_bytes,
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4)},
        "verify": verify,
        "timing": f"HIP events around replays of a HIP graph of {reps} tokens",
    }), flush=True)


def bench_block_moves(args):
    """dlmk_copy_blocks / dlmk_gather_blocks / dlmk_scatter_blocks on 8B-shaped
    f16 blocks (8 kv heads x 16 tokens x 128 dims: 32 KiB per pool) at 128 ..
    8192 blocks drawn at random from a 40,000-block pool, each size timed as
    HIP-graph replays of 10 launches.  Bytes per launch: every block read and
    written once in each of the K and V pools (4 x blocks x 32 KiB).  A
    least-squares fit t = a + bytes / BW over the sizes separates a fixed
    per-launch cost a from the streaming rate BW."""
    import torch
    from dlm_amd import ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    nb, bb = 40000, 8 * BS * 128 * 2
    k = torch.zeros(nb * bb, dtype=torch.uint8, device=dev)
    v = torch.zeros_like(k)
    rng = np.random.default_rng(SEED)
    sizes = [128, 512, 2048, 8192]
    reps = 10
    out = {}
    for n in sizes:
        perm = rng.permutation(nb).astype(np.int32)
        pairs = torch.from_numpy(np.stack([perm[:n], perm[n:2 * n]], 1).copy()).to(dev)
        ids = torch.from_numpy(perm[:n].copy()).to(dev)
        staging = torch.empty(2 * n * bb, dtype=torch.uint8, device=dev)
        fns = {"copy": lambda: ops.copy_blocks(k, v, pairs, bb),
               "gather": lambda: ops.gather_blocks(k, v, ids, bb, staging),
               "scatter": lambda: ops.scatter_blocks(k, v, staging, ids, bb)}
        for name, fn in fns.items():
            fn()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(reps):
                    fn()
            torch.cuda.synchronize()
            for _ in range(3):
                g.replay()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            a.record()
            for _ in range(max(1, args.steps // reps)):
                g.replay()
            b.record()
            torch.cuda.synchronize()
            us = a.elapsed_time(b) * 1e3 / (reps * max(1, args.steps // reps))
            nbytes = 4 * n * bb
            out.setdefault(name, []).append({"blocks": n, "bytes": nbytes, "us": round(us, 2),
                                             "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)})
    fits = {}
    for name, rows in out.items():
        x = np.array([r["bytes"] for r in rows], np.float64)
        t = np.array([r["us"] for r in rows], np.float64)
        slope, icpt = np.polyfit(x, t, 1)
        resid = t - (icpt + slope * x)
        fits[name] = {"fixed_us": round(float(icpt), 2),
                      "stream_GBps": round(float(1e-3 / slope), 1) if slope > 0 else None,
                      "max_resid_us": round(float(np.abs(resid).max()), 2)}
    print(json.dumps({"metric": "block move HBM GB/s by size (8B-shaped f16 blocks)",
                      "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
                      "data": "synthetic (zero pools, random block ids, seeded)",
                      "config": {"workload": "blockmoves", "block_bytes_per_pool": bb,
                                 "pool_blocks": nb, "sizes": sizes},
                      "moves": out, "fit": fits,
                      "timing": f"HIP events around replays of a HIP graph of {reps} launches"}),
          flush=True)


def copy_calibration(torch, ops, steps):
    """A plain copy of known size: 4096 pairs of 32 KiB blocks in each of the K and V pools."""
    dev = torch.device("cuda:0")
    nb, bb = 8192, 8 * BS * 128 * 2
    k = torch.zeros(nb * bb, dtype=torch.uint8, device=dev)
    v = torch.zeros_like(k)
    pairs = torch.stack([torch.arange(0, 4096), torch.arange(4096, 8192)], 1).int().to(dev)
    for _ in range(steps):
        ops.copy_blocks(k, v, pairs, bb)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration": {"launches": steps, "bytes_read_per_launch": 2 * 4096 * bb,
                                           "bytes_written_per_launch": 2 * 4096 * bb}}))


def cpu_baseline(w, budget_s, max_threads=16):
    """dlm's CPU attention path (the oracle restatement, 1 thread) on a bounded
    sample of the same workload: as many sequences as fit budget_s.  The same
    sample is then run again over up to max_threads host threads, one sequence
    each at a time (an extension: dlm steps sessions serially), reported
    beside the 1-thread figure."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import oracle as orc
    orc.build()
    rng = np.random.default_rng(SEED + 1000)
    npdt = np.float32 if w.dtype == "f32" else np.float16
    X = 16 // np.dtype(npdt).itemsize
    done_tok, done_seq, elapsed, nbytes = 0, 0, 0.0, 0
    qcode = {"int8": orc.I8, "int4": orc.I4}.get(w.quant)
    jobs = []  # the sample's calls, replayed over threads below
    while elapsed < budget_s and done_seq < 4096:
        c = int(rng.integers(w.ctx[0], w.ctx[1] + 1))
        nb = -(-c // BS)
        table = rng.permutation(nb).astype(np.int32)[None]
        q = (rng.standard_normal((1, w.nq, w.hq, w.d)) * 0.5).astype(npdt)
        if qcode is None:
            kp = (rng.standard_normal((nb, w.hkv, w.d // X, BS, X)) * 0.5).astype(npdt)
            vp = (rng.standard_normal((nb, w.hkv, w.d, BS)) * 0.5).astype(npdt)
            job = (lambda q=q, kp=kp, vp=vp, table=table, c=c:
                   orc.paged_attention(q, kp, vp, table, np.array([c], np.int32), w.nq, w.hq,
                                       w.hkv, w.d, BS, 1.0 / np.sqrt(w.d)))
            t0 = time.perf_counter()
            job()
        else:
            ks, vs = orc.quant_pool_shapes(nb, w.hkv, w.d, qcode)
            kp = rng.integers(0, 256, ks, dtype=np.uint8)
            vp = rng.integers(0, 256, vs, dtype=np.uint8)
            ksc = rng.random((nb, BS), dtype=np.float32) * 0.02
            vsc = rng.random((nb, BS), dtype=np.float32) * 0.02
            qf = q.astype(np.float32)
            job = (lambda qf=qf, kp=kp, vp=vp, ksc=ksc, vsc=vsc, table=table, c=c:
                   orc.paged_attention_quant(qf, kp, vp, ksc, vsc, qcode, table,
                                             np.array([c], np.int32), w.nq, w.hq, w.hkv, w.d,
                                             1.0 / np.sqrt(w.d)))
            t0 = time.perf_counter()
            job()
        elapsed += time.perf_counter() - t0
        jobs.append(job)
        done_tok += c
        done_seq += 1
        nbytes += attn_bytes(w, [c], elem_bytes(w))
    # The same calls over threads (the C oracle releases the GIL in ctypes
    # calls and keeps no shared state).
    from concurrent.futures import ThreadPoolExecutor
    threads = max(1, min(max_threads, os.cpu_count() or 1))
    t0 = time.perf_counter()
    with ThreadPoolExecutor(max_workers=threads) as ex:
        list(ex.map(lambda f: f(), jobs))
    par_s = time.perf_counter() - t0
    del jobs
    return {
        "value": round(nbytes / elapsed / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": (f"oracle/oracle.c paged attention{'' if qcode is None else ' over ' + w.quant + ' pools'} "
                   f"(f32 restatement of dlm attention(), "
                   f"1 thread) over {done_seq} {w.name} sequences, {done_tok} context tokens, "
                   f"{elapsed:.1f} s; same algorithmic-bytes formula"),
        "context_tokens_per_s": round(done_tok / elapsed, 1),
        "cpu_model": _cpu_model(), "host_nproc": os.cpu_count(),
        "extension_threads": {"threads": threads, "value": round(nbytes / par_s / 1e9, 4),
                              "unit": "GB/s", "seconds": round(par_s, 2),
                              "note": "same sample, one sequence per thread at a time; "
                                      "dlm itself steps sessions serially"},
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
    """One set of sequences: books, device block tables, slots and inputs."""

    def __init__(self, torch, w, cache, seq_base, ctx, dev, gen, tdt):
        self.seqs = [seq_base + i for i in range(len(ctx))]
        # Each sequence holds its context, the last nq tokens being this step's drafts.
        for s, c in zip(self.seqs, ctx):
            cache.append_tokens(s, int(c))
        max_blocks = -(-w.ctx[1] // BS)
        tables, lens = cache.block_tables(self.seqs, max_blocks)
        slots = [cache.slot_mapping(s, int(c) - w.nq, w.nq) for s, c in zip(self.seqs, ctx)]
        # Chunked-prefill sequences: their chunk of this step is appended alongside.
        self.prefill = [seq_base + 500 + i for i in range(w.prefill_seqs)]
        for s in self.prefill:
            cache.append_tokens(s, w.prefill_chunk)
            slots.append(cache.slot_mapping(s, 0, w.prefill_chunk))
        slots = np.concatenate(slots).astype(np.int64)
        self.n_append = len(slots)
        self.tables = torch.from_numpy(tables).to(dev)
        self.lens = torch.from_numpy(lens).to(dev)
        self.slots = torch.from_numpy(slots).to(dev)
        self.ctx = ctx
        n = len(ctx)
        self.q = (torch.randn((n, w.nq, w.hq, w.d), generator=gen, device=dev) * 0.5).to(tdt)
        self.k_new = (torch.randn((self.n_append, w.hkv, w.d), generator=gen, device=dev) * 0.5).to(tdt)
        self.v_new = (torch.randn((self.n_append, w.hkv, w.d), generator=gen, device=dev) * 0.5).to(tdt)
        self.out = torch.empty((n, w.nq, w.hq, w.d), dtype=tdt, device=dev)
        # The decode sequences' tokens come first: [B][nq][Hkv][d] for the fused
        # step; the prefill chunks (if any) follow and are appended on their own.
        nd = n * w.nq
        self.k_dec, self.v_dec = self.k_new[:nd], self.v_new[:nd]
        self.k_pre, self.v_pre, self.slots_pre = self.k_new[nd:], self.v_new[nd:], self.slots[nd:]


def main():
    args = parse()
    args.steps = max(20, args.steps // 20 * 20)
    if args.gpus != 1:
        print(json.dumps({"error": "bench.py measures one GPU only; every GPU box here has one "
                                   "GPU and multi-GPU runs are out of scope for this path",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    if args.workload == "block8b":
        bench_block(args)
        return
    if args.workload == "blockmoves":
        bench_block_moves(args)
        return
    traffic, traffic_note = None, None
    if args.traffic == "pmc" and not args.copy_calibration and args.only is None:
        # Before this process touches the GPU: the counter passes run as children.
        try:
            traffic, traffic_note = measure_traffic(args)
        except Exception as e:  # the timed line stands without it
            traffic_note = f"not measured: {e}"

    import torch
    from dlm_amd import KvCacheConfig, PagedKvCache, ops

    if args.copy_calibration:
        copy_calibration(torch, ops, args.steps)
        return
    w = WORKLOADS[args.workload]
    if args.kv_quant != "none":
        if w.dtype != "f16":
            sys.exit(f"--kv-quant needs an f16 workload ({w.name} is {w.dtype})")
        w = replace(w, quant=args.kv_quant, extras=[])
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED)
    tdt = torch.float32 if w.dtype == "f32" else torch.float16

    # Pool: both batches (plus prefill chunks and fork room) with slack, shuffled.
    rng = np.random.default_rng(SEED)
    ctxs = [rng.integers(w.ctx[0], w.ctx[1] + 1, w.batch).astype(np.int32) for _ in range(2)]
    need = sum(int(((c + BS - 1) // BS).sum()) for c in ctxs)
    need += 2 * w.prefill_seqs * (-(-w.prefill_chunk // BS))
    floor = 20000 if w.layers == 1 else 0  # configs[1] quotes a 20k-block pool
    pool_blocks = max(floor, int(need * (1.6 if "fork" in w.extras else 1.2)) + 64)
    cfg = KvCacheConfig(num_layers=w.layers, num_kv_heads=w.hkv, head_dim=w.d, block_size=BS)
    cache = PagedKvCache.with_seeded_shuffle(cfg, pool_blocks, seed=SEED)
    quant = w.quant != "none"
    if quant:
        # Quantized pools: every slot filled by the quantizing append itself.
        layers = [ops.alloc_quant_pools(pool_blocks, w.hkv, w.d, w.quant, dev)
                  for _ in range(w.layers)]
        fill = torch.arange(pool_blocks * BS, dtype=torch.int64, device=dev)
        for kv in layers:
            for lo in range(0, fill.numel(), 65536):
                sl = fill[lo:lo + 65536]
                src = torch.randn((sl.numel(), w.hkv, w.d), generator=gen, device=dev,
                                  dtype=tdt) * 0.5
                ops.kv_append_quant(kv, src, src.flip(0), sl, num_kv_heads=w.hkv, head_dim=w.d)
        del fill
    else:
        geom = ops.PoolGeometry(pool_blocks, w.hkv, w.d, BS, tdt)
        layers = ops.alloc_pools(geom, dev, num_layers=w.layers)
        for kp, vp in layers:
            kp.normal_(0.0, 0.5, generator=gen)
            vp.normal_(0.0, 0.5, generator=gen)

    t_books = time.perf_counter()
    batches = [Batch(torch, w, cache, b * 1000, ctxs[b], dev, gen, tdt) for b in range(2)]
    books_s = time.perf_counter() - t_books
    max_blocks = -(-w.ctx[1] // BS)
    ws = ops.alloc_workspace(ops.attention_workspace_bytes(w.batch, w.nq, w.hq, w.d, max_blocks), dev)

    def append_quant(bt):
        for kv in layers:
            ops.kv_append_quant(kv, bt.k_new, bt.v_new, bt.slots, num_kv_heads=w.hkv, head_dim=w.d)

    def attend_quant(bt):
        for kv in layers:
            ops.paged_decode_attention_quant(bt.q, kv, bt.tables, bt.lens, num_kv_heads=w.hkv,
                                             out=bt.out, workspace=ws)

    def step_quant(bt):
        # No fused append into quantized pools: quantizing append, then attention.
        for kv in layers:
            ops.kv_append_quant(kv, bt.k_new, bt.v_new, bt.slots, num_kv_heads=w.hkv, head_dim=w.d)
            ops.paged_decode_attention_quant(bt.q, kv, bt.tables, bt.lens, num_kv_heads=w.hkv,
                                             out=bt.out, workspace=ws)

    def append(bt):
        for kp, vp in layers:
            ops.kv_append(kp, vp, bt.k_new, bt.v_new, bt.slots, num_kv_heads=w.hkv, head_dim=w.d)

    def attend(bt):
        for kp, vp in layers:
            ops.paged_decode_attention(bt.q, kp, vp, bt.tables, bt.lens, num_kv_heads=w.hkv,
                                       out=bt.out, workspace=ws)

    def step_unfused(bt):
        # Per layer: append this step's tokens, then attend (dlm's per-layer order).
        for kp, vp in layers:
            ops.kv_append(kp, vp, bt.k_new, bt.v_new, bt.slots, num_kv_heads=w.hkv, head_dim=w.d)
            ops.paged_decode_attention(bt.q, kp, vp, bt.tables, bt.lens, num_kv_heads=w.hkv,
                                       out=bt.out, workspace=ws)

    def step(bt):
        # Per layer: the fused decode step appends the decode tokens and attends
        # in one launch; chunked-prefill tokens are appended alongside.
        for kp, vp in layers:
            if bt.slots_pre.numel():
                ops.kv_append(kp, vp, bt.k_pre, bt.v_pre, bt.slots_pre, num_kv_heads=w.hkv,
                              head_dim=w.d)
            ops.paged_decode_step(bt.q, bt.k_dec, bt.v_dec, kp, vp, bt.tables, bt.lens,
                                  num_kv_heads=w.hkv, out=bt.out, workspace=ws)

    if quant:
        step, step_unfused, attend, append = step_quant, None, attend_quant, append_quant
    for i in range(args.warmup):
        step(batches[i & 1])
    torch.cuda.synchronize()

    # The timed work runs as HIP graphs, the way a serving loop replays a fixed
    # decode step: no host launch overhead in the measurement, only kernels.
    # Every launch inside is a libdlmk kernel; nothing writes memory by memset.
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
    stream = torch.cuda.current_stream()

    def timed(graph, reps, n):
        for _ in range(max(1, -(-args.warmup // reps))):
            graph.replay()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        for _ in range(n // reps):
            graph.replay()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / (reps * (n // reps))

    def phase(name, fn, reps, n):
        if args.only not in (None, name) or fn is None:
            return float("nan")
        return timed(capture(fn, reps), reps, n)

    t0 = time.perf_counter()
    step_ms = phase("step", step, REPS, args.steps)
    wall_s = time.perf_counter() - t0
    unfused_ms = phase("unfused", step_unfused, REPS, args.steps)
    attn_ms = phase("attention", attend, REPS, args.steps)
    append_ms = phase("append", append, 5 * REPS, 5 * args.steps)

    eb = elem_bytes(w)
    L = w.layers
    mean_attn_bytes = L * (attn_bytes(w, batches[0].ctx, eb) + attn_bytes(w, batches[1].ctx, eb)) / 2
    n_app = (batches[0].n_append + batches[1].n_append) / 2
    step_bytes = mean_attn_bytes + L * append_bytes(w, n_app)
    value = step_bytes / (step_ms * 1e-3) / 1e9
    attn_gbps = mean_attn_bytes / (attn_ms * 1e-3) / 1e9
    # Context tokens one step attends over (summed over the batch, mean of the
    # two rotating batches), and the per-sequence mean.
    ctx_tok = (batches[0].ctx.sum() + batches[1].ctx.sum()) / 2
    ctx_mean = ctx_tok / w.batch

    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "ms_per_step_unfused": None if quant else round(unfused_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w.dtype if not quant else f"{w.quant} KV codes (f16 q, f16 MFMA operands)",
        "data": "synthetic (seeded N(0,1)*0.5 K/V/Q, seeded contexts and shuffled pool)",
        "config": {
            "workload": w.about,
            "num_q_heads": w.hq, "num_kv_heads": w.hkv, "head_dim": w.d, "block_size": BS,
            "layers": w.layers, "batch": w.batch, "queries_per_seq": w.nq,
            "ctx": f"U[{w.ctx[0]},{w.ctx[1]}] seed {SEED}", "pool_blocks": pool_blocks,
            "kv_quant": w.quant, "rotating_batches": 2, "mean_context_tokens": round(float(ctx_mean), 1),
            "context_tokens_per_step": float(ctx_tok),
            "appended_tokens_per_step": n_app, "parallelism": "single GPU",
        },
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBPS, 2),
        "attention": {
            "GBps": round(attn_gbps, 1), "pct_of_hbm_peak": round(100 * attn_gbps / HBM_PEAK_GBPS, 2),
            "us_per_launch": round(attn_ms * 1e3 / L, 2),
            "algorithmic_bytes_per_launch": int(mean_attn_bytes / L),
            "context_tokens_per_s": round(L * ctx_tok / (attn_ms * 1e-3), 1),
            "query_tokens_per_s": round(w.batch * w.nq / (attn_ms * 1e-3), 1),
        },
        "kv_append": {
            "tokens_per_s": round(L * n_app / (append_ms * 1e-3), 1),
            "us_per_launch": round(append_ms * 1e3 / L, 2),
            "GBps": round(L * append_bytes(w, n_app) / (append_ms * 1e-3) / 1e9, 2),
        },
        "host_books_s": round(books_s, 4),
        "wall_s_timed_region": round(wall_s, 4),
        "timing": f"HIP events around replays of HIP graphs of {REPS} steps each ({5 * REPS} "
                  "appends for the append-only line), alternating the two batches; a step is "
                  + ("dlmk_kv_append_quant + dlmk_paged_decode_attention_quant (no fused "
                     "step for quantized pools)" if quant else
                     "dlmk_paged_decode_step (append + attention in one launch), "
                     "ms_per_step_unfused the same step as dlmk_kv_append + "
                     "dlmk_paged_decode_attention"),
        "roofline": {
            "bound": "hbm", "achieved": round(attn_gbps, 1), "peak": HBM_PEAK_GBPS,
            "unit": "GB/s", "frac": round(attn_gbps / HBM_PEAK_GBPS, 4), "traffic": traffic,
            # Quantized pools with GQA groups of up to 4 rows (int4: 8) run the
            # packed kernel (several blocks per score tile); int8 only for rows
            # of up to 4 partitions of 1024 tokens.
            "kernel": ("paged_attn_generic_kernel" if w.dtype == "f32" else
                       "paged_attn_packed_kernel" if (w.quant == "int4" and w.hq // w.hkv * w.nq <= 8)
                       or (w.quant == "int8" and w.hq // w.hkv * w.nq <= 4 and w.ctx[1] <= 4096)
                       else "paged_attn_mfma_kernel"),
            "traffic_detail": traffic_note,
        },
    }
    if "fork" in w.extras:
        result["fork"] = bench_fork(torch, ops, cache, layers[0], batches[0], w)
    if "swap" in w.extras:
        result["swap"] = bench_swap(torch, ops, cache, layers[0], batches[0], w, dev)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds)
    print(json.dumps(_finite(result)), flush=True)


def _finite(x):
    """NaN (a phase skipped by --only) becomes null: the line stays valid JSON."""
    if isinstance(x, dict):
        return {k: _finite(v) for k, v in x.items()}
    if isinstance(x, float) and x != x:
        return None
    return x


def _events(torch, fn, n):
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    fn()
    torch.cuda.synchronize()
    a.record()
    for _ in range(n):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / n


def bench_fork(torch, ops, cache, pools, bt, w):
    """Fork 8 sequences by block copy (dlmk_copy_blocks), K and V pools."""
    pairs = np.concatenate([cache.fork_sequence(s, 10_000 + s) for s in bt.seqs[:8]])
    bb = w.hkv * BS * w.d * elem_bytes(w)
    p = torch.from_numpy(pairs).to(pools[0].device)
    ms = _events(torch, lambda: ops.copy_blocks(pools[0], pools[1], p, bb), 20)
    nbytes = 2 * 2 * len(pairs) * bb
    return {"blocks": int(len(pairs)), "bytes_moved": nbytes, "us": round(ms * 1e3, 2),
            "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1)}


def bench_swap(torch, ops, cache, pools, bt, w, dev):
    """Swap 25% of the batch's blocks out to pinned host memory and back:
    gather/scatter kernels (HBM GB/s) and the PCIe copies (GB/s) separately."""
    rng = np.random.default_rng(SEED + 5)
    owned = np.array([b for s in bt.seqs for b in cache.block_table(s)], np.int32)
    ids_np = rng.choice(owned, len(owned) // 4, replace=False).astype(np.int32)
    ids = torch.from_numpy(ids_np).to(dev)
    bb = w.hkv * BS * w.d * elem_bytes(w)
    nbytes = 2 * len(ids_np) * bb
    staging = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    host = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    g_ms = _events(torch, lambda: ops.gather_blocks(pools[0], pools[1], ids, bb, staging), 10)
    s_ms = _events(torch, lambda: ops.scatter_blocks(pools[0], pools[1], staging, ids, bb), 10)
    out_ms = _events(torch, lambda: ops.swap_out(host, pools[0], pools[1], ids, bb, staging), 5)
    in_ms = _events(torch, lambda: ops.swap_in(pools[0], pools[1], host, ids, bb, staging), 5)
    return {"blocks": int(len(ids_np)), "bytes": nbytes,
            "gather_hbm_GBps": round(2 * nbytes / (g_ms * 1e-3) / 1e9, 1),
            "scatter_hbm_GBps": round(2 * nbytes / (s_ms * 1e-3) / 1e9, 1),
            "swap_out_us": round(out_ms * 1e3, 1), "swap_in_us": round(in_ms * 1e3, 1),
            "swap_out_pcie_GBps": round(nbytes / (out_ms * 1e-3) / 1e9, 1),
            "swap_in_pcie_GBps": round(nbytes / (in_ms * 1e-3) / 1e9, 1)}


if __name__ == "__main__":
    main()
