"""Host side of the decode-block path (no GPU): the RoPE frequencies the host
computes for the device agree with the oracle's restatement of
rope_inv_freqs (src/forward/cpu.rs:1057-1092) to the reference tests' own
1e-6 (its f32 powf and NumPy's float32 power may differ in the last bit), and
the workspace-size entry point is consistent."""
import numpy as np
import pytest

from dlm_amd.block import BlockConfig, rope_inv_freqs


@pytest.mark.parametrize("d,theta,scaling", [
    (64, 10000.0, None), (128, 500000.0, None), (64, 10000.0, ("linear", 4.0)),
    (128, 500000.0, ("llama3", 8.0, 1.0, 4.0, 8192.0)), (64, 1_000_000.0, None)])
def test_rope_inv_freqs_match_oracle(oracle, d, theta, scaling):
    np.testing.assert_allclose(rope_inv_freqs(d, theta, scaling),
                               oracle.rope_inv_freqs(d, theta, scaling), rtol=1e-6)


def test_block_config_geometry():
    c = BlockConfig(4096, 32, 8, 128, 14336)
    assert (c.q_dim, c.kv_dim, c.group_size) == (4096, 1024, 4)


def test_decode_block_workspace_size(dlmk):
    # regions: q, k, v, ctx, act, ctx_len, then the attention workspace, each
    # on a 256-byte boundary
    up = lambda x: (x + 255) // 256 * 256
    H, qd, kvd, Hq, d, I = 4096, 4096, 1024, 32, 128, 14336
    attn = dlmk.dlmk_paged_attention_workspace_size(1, 1, Hq, d, 16, 256)
    off = 0
    for n in (qd, kvd, kvd, qd, I, 1):
        off = up(off + 4 * n)
    assert dlmk.dlmk_decode_block_workspace_size(H, qd, kvd, Hq, d, I, 256) == off + attn
    assert dlmk.dlmk_decode_block_workspace_size(0, qd, kvd, Hq, d, I, 256) == 0


@pytest.mark.parametrize("w_dtype", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("n", [1, 7, 128, 1000, 4096 * 1024])
def test_weight_bytes_match_the_blob_layout(oracle, w_dtype, n):
    from dlm_amd.block import weight_bytes
    want = {0: 4 * n, 1: 2 * n, 2: 2 * n}.get(w_dtype)
    if want is None:
        want = oracle.quant_blob_bytes(w_dtype, n, 128)
    assert weight_bytes(w_dtype, n, 128) == want
