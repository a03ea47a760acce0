"""HIP-graph capture of the paged path: append + attention, the fused decode
step, quantizing append + attention over int8 / int4 pools, and the decode and
verify blocks.  Every replay must equal the eager result, also with eager work
and synchronisations between replays (no memset nodes are recorded by
libdlmk)."""
import numpy as np
import pytest

from helpers import make_workload, to_dev

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(cuda):
    import torch
    from dlm_amd import ops
    print("[gpu-test] graph replay of append + attention", flush=True)
    rng = np.random.default_rng(40)
    Hq, Hkv, d = 32, 8, 128
    w = make_workload(rng, [700, 1500, 40, 3000], Hq, Hkv, d, np.float16, sigma=0.5)
    kp, vp = to_dev(torch, w.k_pool, cuda), to_dev(torch, w.v_pool, cuda)
    tables, lens = to_dev(torch, w.tables, cuda), to_dev(torch, w.ctx, cuda)
    q = to_dev(torch, w.q, cuda)
    slots = torch.tensor([int(w.tables[s, (c - 1) // 16]) * 16 + (c - 1) % 16
                          for s, c in enumerate(w.ctx)], dtype=torch.int64, device=cuda)
    knew = (torch.randn((4, Hkv, d), device=cuda) * 0.5).half()
    vnew = (torch.randn((4, Hkv, d), device=cuda) * 0.5).half()
    ws = ops.alloc_workspace(ops.attention_workspace_bytes(4, 1, Hq, d, w.tables.shape[1]), cuda)
    out = torch.empty_like(q)

    def step():
        ops.kv_append(kp, vp, knew, vnew, slots, num_kv_heads=Hkv, head_dim=d)
        ops.paged_decode_attention(q, kp, vp, tables, lens, num_kv_heads=Hkv, out=out,
                                   workspace=ws)

    step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    for it in range(4):
        # Eager work between replays changes the inputs the graph reads.
        q.mul_(-1.0 if it % 2 else 0.5)
        knew.add_(0.25)
        step()
        torch.cuda.synchronize()
        eager = out.clone()
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {it} differs from eager"


def test_graph_replays_fused_step(cuda):
    """The fused decode step in a graph: each replay equals the eager call."""
    import torch
    from dlm_amd import ops
    print("[gpu-test] graph replay of the fused decode step", flush=True)
    rng = np.random.default_rng(41)
    Hq, Hkv, d, nq = 32, 8, 128, 4
    w = make_workload(rng, [900, 2500, 7], Hq, Hkv, d, np.float16, nq=nq, sigma=0.5)
    kp, vp = to_dev(torch, w.k_pool, cuda), to_dev(torch, w.v_pool, cuda)
    tables, lens = to_dev(torch, w.tables, cuda), to_dev(torch, w.ctx, cuda)
    q = to_dev(torch, w.q, cuda)
    knew = (torch.randn((3, nq, Hkv, d), device=cuda) * 0.5).half()
    vnew = (torch.randn((3, nq, Hkv, d), device=cuda) * 0.5).half()
    ws = ops.alloc_workspace(ops.attention_workspace_bytes(3, nq, Hq, d, w.tables.shape[1]), cuda)
    out = torch.empty_like(q)

    def step():
        ops.paged_decode_step(q, knew, vnew, kp, vp, tables, lens, num_kv_heads=Hkv, out=out,
                              workspace=ws)

    step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    for it in range(4):
        knew.mul_(-1.0)
        q.add_(0.125)
        step()
        torch.cuda.synchronize()
        eager = out.clone()
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {it} differs from eager"


def _replay_check(torch, g, eager_step, out, mutate, label):
    """Eager work between replays changes the graph's inputs; each replay must
    then equal the eager call on the same inputs, bit for bit."""
    for it in range(4):
        mutate(it)
        eager_step()
        torch.cuda.synchronize()
        eager = out.clone()
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"{label}: replay {it} differs from eager"


@pytest.mark.parametrize("quant", ["int8", "int4"])
def test_graph_replays_quant_append_attention(cuda, quant):
    """Quantizing append (quad kernel, 256+ tokens) + attention over the code
    pools in one graph."""
    import torch
    from dlm_amd import ops
    print(f"[gpu-test] graph replay of quantized append + attention ({quant})", flush=True)
    rng = np.random.default_rng(42)
    Hq, Hkv, d = 32, 8, 128
    w = make_workload(rng, [700, 1500, 40, 3000], Hq, Hkv, d, np.float16, sigma=0.5)
    nb = w.k_pool.shape[0]
    kv = ops.alloc_quant_pools(nb, Hkv, d, quant, cuda)
    tables, lens = to_dev(torch, w.tables, cuda), to_dev(torch, w.ctx, cuda)
    # Every history token, then a 300-token "chunk" re-appended by the step.
    slots_all = np.concatenate([w.tables[s, np.arange(c) // 16].astype(np.int64) * 16
                                + np.arange(c) % 16 for s, c in enumerate(w.ctx)])
    hist = (torch.randn((len(slots_all), Hkv, d), device=cuda) * 0.5).half()
    ops.kv_append_quant(kv, hist, hist.flip(0).contiguous(), torch.from_numpy(slots_all).to(cuda),
                        num_kv_heads=Hkv, head_dim=d)
    step_slots = torch.from_numpy(slots_all[-300:].copy()).to(cuda)
    knew = (torch.randn((300, Hkv, d), device=cuda) * 0.5).half()
    vnew = (torch.randn((300, Hkv, d), device=cuda) * 0.5).half()
    q = to_dev(torch, w.q, cuda)
    ws = ops.alloc_workspace(ops.attention_workspace_bytes(4, 1, Hq, d, w.tables.shape[1]), cuda)
    out = torch.empty_like(q, dtype=torch.float32)

    def step():
        ops.kv_append_quant(kv, knew, vnew, step_slots, num_kv_heads=Hkv, head_dim=d)
        ops.paged_decode_attention_quant(q, kv, tables, lens, num_kv_heads=Hkv, out=out,
                                         workspace=ws)

    step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()

    def mutate(it):
        knew.mul_(-1.0 if it % 2 else 1.5)
        q.add_(0.125)
    _replay_check(torch, g, step, out, mutate, f"quant {quant}")


def _block_kernel(torch, cuda, n_layers=1, H=256, Hq=4, Hkv=2, d=64, inter=512, max_blocks=32):
    from dlm_amd.block import BlockConfig, LayerWeights, PagedGpuKernel
    g = torch.Generator(device="cpu").manual_seed(7)
    mat = lambda r, c: ((torch.rand((r, c), generator=g) * 2 - 1) * 0.05).to(cuda).view(
        torch.uint8).reshape(-1)
    layers = [LayerWeights(
        q_proj=mat(Hq * d, H), k_proj=mat(Hkv * d, H), v_proj=mat(Hkv * d, H),
        o_proj=mat(H, Hq * d), gate_proj=mat(inter, H), up_proj=mat(inter, H),
        down_proj=mat(H, inter), input_layernorm=torch.ones(H, device=cuda),
        post_attention_layernorm=torch.ones(H, device=cuda)) for _ in range(n_layers)]
    cfg = BlockConfig(H, Hq, Hkv, d, inter)
    return PagedGpuKernel(cfg, layers, 0, 0, max_blocks_per_seq=max_blocks, device=cuda)


@pytest.mark.parametrize("n_tokens", [1, 5])
def test_graph_replays_decode_and_verify_block(cuda, n_tokens):
    """dlmk_decode_block_paged (1 token) / dlmk_verify_block_paged (5) in a
    graph at a 300-token history (split-K partitions and the combine launch):
    each replay re-appends the same positions and must equal the eager call."""
    import torch
    print(f"[gpu-test] graph replay of the decode block, {n_tokens} token(s)", flush=True)
    H, Hkv, d, hist = 256, 2, 64, 300
    kern = _block_kernel(torch, cuda)
    nb = 40
    rng = np.random.default_rng(43)
    table = torch.from_numpy(rng.permutation(nb)[:32].astype(np.int32)).to(cuda)
    kp = (torch.randn((nb, Hkv, d * 16), device=cuda) * 0.5)
    vp = (torch.randn((nb, Hkv, d * 16), device=cuda) * 0.5)
    x0 = (torch.randn((n_tokens, H), device=cuda) * 0.5)
    x = torch.empty_like(x0)

    def step():
        x.copy_(x0)
        if n_tokens == 1:
            kern.run_block(0, x[0], (kp, vp), table, hist, hist)
        else:
            kern.run_tokens(0, x, (kp, vp), table, hist, hist)

    step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()

    def mutate(it):
        x0.mul_(-1.0 if it % 2 else 0.75)
    _replay_check(torch, g, step, x, mutate, f"block n={n_tokens}")
