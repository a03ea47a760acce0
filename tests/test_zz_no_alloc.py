"""dlmk_paged_decode_attention_noalloc against dlmk_paged_decode_attention,
both called through the C ABI: bitwise-equal outputs on two calls in a row
(the second smaller, so stale partials of the first are in the shared scratch
array), the f32 and f16 kernels, and a clear error for partials beyond the
scratch array's size.  The allocation-free entry point has no counterpart in
the reference; its result is pinned to the workspace entry point, which the
other GPU tests pin to the oracle."""
import ctypes as C

import numpy as np
import pytest

from helpers import F16_ATOL, F16_RTOL, F32_ATOL, F32_RTOL, assert_close, make_workload, to_dev

pytestmark = pytest.mark.gpu


def _call_both(torch, cuda, lib, oracle, w, dtype_code, torch_dt):
    from dlm_amd import _lib, ops
    dv = lambda a: to_dev(torch, a, cuda)
    B, nq, Hq, Hkv, d = len(w.ctx), w.nq, w.Hq, w.Hkv, w.d
    kp, vp, q, t, lens = dv(w.k_pool), dv(w.v_pool), dv(w.q), dv(w.tables), dv(w.ctx)
    max_blocks = w.tables.shape[1]
    ws = ops.alloc_workspace(ops.attention_workspace_bytes(B, nq, Hq, d, max_blocks), cuda)
    out_ref = torch.full((B, nq, Hq, d), float("nan"), dtype=torch.float32, device=cuda)
    out_new = torch.full((B, nq, Hq, d), float("nan"), dtype=torch.float32, device=cuda)
    stream = torch.cuda.current_stream().cuda_stream
    scale = float(w.scale)
    _lib.check(lib.dlmk_paged_decode_attention(
        stream, out_ref.data_ptr(), _lib.DLMK_F32, q.data_ptr(), kp.data_ptr(), vp.data_ptr(),
        dtype_code, t.data_ptr(), lens.data_ptr(), B, nq, Hq, Hkv, d, 16, max_blocks,
        w.k_pool.shape[0], scale, ws.data_ptr() if ws is not None else None,
        ws.numel() if ws is not None else 0))
    _lib.check(lib.dlmk_paged_decode_attention_noalloc(
        stream, out_new.data_ptr(), _lib.DLMK_F32, q.data_ptr(), kp.data_ptr(), vp.data_ptr(),
        dtype_code, t.data_ptr(), lens.data_ptr(), B, nq, Hq, Hkv, d, 16, max_blocks,
        w.k_pool.shape[0], scale))
    torch.cuda.synchronize()
    assert torch.equal(out_ref, out_new), "allocation-free output differs from the workspace one"
    ref = oracle.paged_attention(w.q, w.k_pool, w.v_pool, w.tables, w.ctx, nq, Hq, Hkv, d, 16,
                                 w.scale)
    atol, rtol = (F32_ATOL, F32_RTOL) if torch_dt == torch.float32 else (F16_ATOL, F16_RTOL)
    assert_close(out_new.cpu().numpy(), ref, atol, rtol, "allocation-free attention vs oracle")


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_noalloc_matches_workspace_entry_point_twice(oracle, cuda, dtype):
    import torch
    from dlm_amd import _lib
    lib = _lib.lib()
    name = np.dtype(dtype).name
    code, tdt = ((_lib.DLMK_F16, torch.float16) if dtype is np.float16
                 else (_lib.DLMK_F32, torch.float32))
    rng = np.random.default_rng(77)
    Hq, Hkv, d = (32, 8, 128) if dtype is np.float16 else (32, 8, 64)
    sigma = 0.5 if dtype is np.float16 else 1.0
    # First call: many multi-partition rows; second: fewer, shorter rows
    # (the scratch array still holds the first call's partials).
    for ctx, nq in (([4096, 3000, 128, 2049, 1025, 5000, 7, 4000], 1), ([1500, 33, 700], 2)):
        print(f"[gpu-test] noalloc {name} ctx={ctx} nq={nq}", flush=True)
        w = make_workload(rng, ctx, Hq, Hkv, d, dtype, nq=nq, sigma=sigma)
        _call_both(torch, cuda, lib, oracle, w, code, tdt)


def test_noalloc_rejects_partials_beyond_scratch(cuda):
    """rows x partitions x (d + 2) floats above DLMK_NOALLOC_SCRATCH_BYTES: an
    error before any launch (the pointers are never dereferenced)."""
    import torch
    from dlm_amd import _lib
    lib = _lib.lib()
    print("[gpu-test] noalloc size limit", flush=True)
    buf = torch.zeros(1024, dtype=torch.float16, device=cuda)
    lens = torch.zeros(64, dtype=torch.int32, device=cuda)
    p = buf.data_ptr()
    # 64 sequences x 4 queries x 32 heads, 2048-block tables: 32 partitions of
    # 1024 tokens -> 8192 rows x 32 x 520 bytes = 136 MB of partials.
    rc = lib.dlmk_paged_decode_attention_noalloc(
        torch.cuda.current_stream().cuda_stream, p, _lib.DLMK_F32, p, p, p, _lib.DLMK_F16, p,
        lens.data_ptr(), 64, 4, 32, 8, 128, 16, 2048, 64, 0.1)
    assert rc == _lib.DLMK_ERR_WORKSPACE
    msg = _lib.last_error()
    assert "split-K partials need" in msg and str(32 << 20) in msg, msg
