"""HIP-graph capture of a decode step (append + paged attention): every replay
must equal the eager result, also with eager work and synchronisations between
replays (no memset nodes are recorded by libdlmk)."""
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
