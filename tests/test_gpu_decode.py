"""GPU checks of incremental decoding (ssa_amd.decode.SSADecodeCache, the block
entry points ssa_select_block / ssa_sparse_attention_block).

A step that leaves n tokens in the cache must equal the last rows of the
whole-sequence forward over those n tokens (same keys, codes and index; the
filler of a row with fewer than k candidates comes from the same n keys):
selected index sets bit for bit, attention outputs bit for bit (same kernels
on the same inputs).
The prefix forward is itself pinned to the oracle by the other GPU tests; here
one step is also checked against the oracle directly.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.helpers import clustered_qk, f32

pytestmark = pytest.mark.gpu


def _setup(dev, n, h_q, h_kv, d, n_c, top_k, dtype, seed):
    from ssa_amd import CodebookRouter

    q, k = clustered_qk(n, h_q, h_kv, d, 16, 0.3, seed, dtype)
    v = torch.randn(n, h_kv, d, generator=torch.Generator().manual_seed(seed + 1)).to(dtype)
    torch.manual_seed(seed + 2)
    router = CodebookRouter(head_dim=d, route_dim=32, num_kv_heads=h_kv, num_codebook=n_c,
                            codes_per_key=4, codes_per_query=8, top_k=top_k).to(dev)
    return q[None].to(dev), k[None].to(dev), v[None].to(dev), router


def _prefix_forward(router, q, k, v, n):
    """Whole-sequence forward over tokens 0..n-1."""
    from ssa_amd import kernels

    qp, kp, vp = q[:, :n], k[:, :n], v[:, :n]
    qc, kc = kernels.route_codes(qp, kp, router.W_qr.weight, router.W_kr.weight, router.codebook,
                                 router.codes_per_query, router.codes_per_key, router.temperature)
    off, post = kernels.build_index(kc, router.num_codebook)
    idx = kernels.select(qp, kp, qc, off, post, router.codes_per_key, router.top_k, sorted=False,
                         index_dtype=torch.int32)
    out = kernels.sparse_attention(qp, kp, vp, idx, None, True)
    return idx, out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_decode_steps_match_prefix_forward(dev, dtype):
    from ssa_amd.decode import SSADecodeCache

    n, h_q, h_kv, d = 160, 8, 2, 128
    q, k, v, router = _setup(dev, n, h_q, h_kv, d, 64, 24, dtype, seed=3)
    cache = SSADecodeCache(router, 1, 256, d, dtype=dtype)
    pos = 0
    for m in (96, 1, 1, 3, 1, 7, 1):  # a prefill chunk, then single tokens and small chunks
        out, idx = cache.step(q[:, pos:pos + m], k[:, pos:pos + m], v[:, pos:pos + m], return_indices=True)
        ref_idx, ref_out = _prefix_forward(router, q, k, v, pos + m)
        assert torch.equal(idx, ref_idx[:, pos:]), f"indices differ in the step at {pos}"
        assert torch.equal(out, ref_out[:, pos:]), f"outputs differ in the step at {pos}"
        pos += m
    assert cache.len == pos


def test_decode_step_matches_oracle(dev, orc):
    from ssa_amd.decode import SSADecodeCache

    n, h_q, h_kv, d = 200, 8, 2, 64
    q, k, v, router = _setup(dev, n, h_q, h_kv, d, 32, 16, torch.float32, seed=8)
    cache = SSADecodeCache(router, 1, n, d, dtype=torch.float32)
    cache.step(q[:, :199], k[:, :199], v[:, :199])
    out, idx = cache.step(q[:, 199:], k[:, 199:], v[:, 199:], return_indices=True)
    qf, kf, vf = f32(q[0]), f32(k[0]), f32(v[0])
    ref_idx, _ = orc.router_forward(qf, kf, f32(router.W_qr.weight), f32(router.W_kr.weight),
                                    f32(router.codebook), 8, 4, 16, orc.MASK_CAUSAL)
    got = np.sort(idx[0, 0].cpu().numpy().astype(np.int64), axis=-1)
    assert np.array_equal(got, np.sort(ref_idx[199], axis=-1))
    ref_out = orc.sparse_attention(qf, kf, vf, ref_idx[199:200], causal=True, rows=np.array([199]))
    np.testing.assert_allclose(out[0].cpu().numpy(), ref_out, rtol=2e-5, atol=2e-5)


def test_block_rejects_rows_past_the_keys(dev):
    from ssa_amd import kernels

    q, k, v, router = _setup(dev, 32, 4, 2, 64, 16, 8, torch.float32, seed=1)
    idx = torch.zeros(1, 4, 2, 8, dtype=torch.int32, device=dev)
    with pytest.raises(Exception, match="outside"):
        kernels.sparse_attention(q[:, :4], k, v, idx, None, True, q_pos0=30)
