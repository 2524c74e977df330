"""GPU checks of incremental decoding (ssa_amd.decode.SSADecodeCache, the block
entry points ssa_select_block / ssa_sparse_attention_block).

A step that leaves n tokens in the cache must equal the last rows of the
whole-sequence forward over those n tokens (same keys, codes and candidate
sets -- a single-token step reads them from the main index over the keys up to
its last rebuild plus the tail index over the keys appended since; the filler
of a row with fewer than k candidates comes from the same n keys): selected
index sets bit for bit, attention outputs bit for bit (same kernels on the
same inputs).
The prefix forward is itself pinned to the oracle by the other GPU tests; here
one step is also checked against the oracle directly.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.helpers import clustered_qk, f32

pytestmark = pytest.mark.gpu


def _setup(dev, n, h_q, h_kv, d, n_c, top_k, dtype, seed, batch=1):
    from ssa_amd import CodebookRouter

    qs, ks, vs = [], [], []
    for bb in range(batch):
        q, k = clustered_qk(n, h_q, h_kv, d, 16, 0.3, seed + 10 * bb, dtype)
        v = torch.randn(n, h_kv, d, generator=torch.Generator().manual_seed(seed + 10 * bb + 1)).to(dtype)
        qs.append(q), ks.append(k), vs.append(v)
    torch.manual_seed(seed + 2)
    router = CodebookRouter(head_dim=d, route_dim=32, num_kv_heads=h_kv, num_codebook=n_c,
                            codes_per_key=4, codes_per_query=8, top_k=top_k).to(dev)
    return (torch.stack(qs).to(dev), torch.stack(ks).to(dev), torch.stack(vs).to(dev), router)


def _prefix_forward(router, q, k, v, n, causal=True):
    """Whole-sequence forward over tokens 0..n-1."""
    from ssa_amd import kernels

    qp, kp, vp = q[:, :n], k[:, :n], v[:, :n]
    qc, kc = kernels.route_codes(qp, kp, router.W_qr.weight, router.W_kr.weight, router.codebook,
                                 router.codes_per_query, router.codes_per_key, router.temperature)
    off, post = kernels.build_index(kc, router.num_codebook)
    idx = kernels.select(qp, kp, qc, off, post, router.codes_per_key, router.top_k, sorted=False,
                         index_dtype=torch.int32)
    # the row path alone (the dense-prefix pass sums the same terms in another order)
    out = kernels.sparse_attention(qp, kp, vp, idx, None, causal, dense_prefix=False)
    return idx, out


def test_decode_default_attends_every_selected_index(dev):
    """The step's default (causal_attention=False, as SSAAttention's) attends
    every selected index, as the whole-sequence forward without the mask does.
    Steps of 4 tokens with rows below top_k: an earlier row of a step can hold
    filler keys of the step's later tokens, so the setting matters there."""
    from ssa_amd.decode import SSADecodeCache

    n, h_q, h_kv, d, m = 40, 8, 2, 64, 4
    q, k, v, router = _setup(dev, n, h_q, h_kv, d, 32, 24, torch.bfloat16, seed=4)
    cache = SSADecodeCache(router, 1, 64, d, dtype=torch.bfloat16, tail_tokens=16)
    cache.step(q[:, :8], k[:, :8], v[:, :8])
    later = False
    for pos in range(8, 24, m):
        out, idx = cache.step(q[:, pos:pos + m], k[:, pos:pos + m], v[:, pos:pos + m], return_indices=True)
        ref_idx, ref_out = _prefix_forward(router, q, k, v, pos + m, causal=False)
        assert torch.equal(idx, ref_idx[:, pos:]), f"indices differ in the step at {pos}"
        assert torch.equal(out, ref_out[:, pos:]), f"outputs differ in the step at {pos}"
        rowpos = torch.arange(pos, pos + m, device=idx.device)[None, :, None, None]
        later = later or bool((idx.to(torch.int64) > rowpos).any())
    assert later, "some row should hold a filler key past its position"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("tail_tokens,batch", [(512, 1), (6, 1), (6, 2)])
def test_decode_steps_match_prefix_forward(dev, dtype, tail_tokens, batch):
    """A prefill chunk, then single tokens and small chunks: each step's indices
    and outputs equal the last rows of the whole-sequence forward.  With
    tail_tokens = 6 the main index is rebuilt inside the single-token steps
    (the tail outgrows it) as well as by the chunks."""
    from ssa_amd.decode import SSADecodeCache

    print(f"decode dtype={dtype} tail_tokens={tail_tokens} batch={batch}", flush=True)
    n, h_q, h_kv, d = 160, 8, 2, 128
    q, k, v, router = _setup(dev, n, h_q, h_kv, d, 64, 24, dtype, seed=3, batch=batch)
    cache = SSADecodeCache(router, batch, 256, d, dtype=dtype, tail_tokens=tail_tokens)
    pos = 0
    for m in (96, 1, 1, 3, 1, 1, 1, 7, 1, 1):
        out, idx = cache.step(q[:, pos:pos + m], k[:, pos:pos + m], v[:, pos:pos + m],
                              causal_attention=True, return_indices=True)
        ref_idx, ref_out = _prefix_forward(router, q, k, v, pos + m)
        assert torch.equal(idx, ref_idx[:, pos:]), f"indices differ in the step at {pos}"
        assert torch.equal(out, ref_out[:, pos:]), f"outputs differ in the step at {pos}"
        pos += m
    assert cache.len == pos
    if tail_tokens == 6:
        assert cache.rebuilds == 3  # the two chunks and one single step (the tail passed 6 keys)


def test_decode_step_matches_oracle(dev, orc):
    from ssa_amd.decode import SSADecodeCache

    n, h_q, h_kv, d = 200, 8, 2, 64
    q, k, v, router = _setup(dev, n, h_q, h_kv, d, 32, 16, torch.float32, seed=8)
    cache = SSADecodeCache(router, 1, n, d, dtype=torch.float32)
    cache.step(q[:, :199], k[:, :199], v[:, :199])
    out, idx = cache.step(q[:, 199:], k[:, 199:], v[:, 199:], causal_attention=True, return_indices=True)
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


@pytest.mark.parametrize("n_c,a,periodic", [(1000, 32, False), (4096, 8, False), (4096, 32, True),
                                             (16384, 16, False)])
def test_decode_codebook_sizes_and_ties(dev, n_c, a, periodic):
    """Single-token steps route their rows with the decoding top-k (scores per
    256-code chunk, then a per-row select): codebooks that are not a multiple
    of the chunk, a temperature, the largest code count, zero queries and
    keys, whose scores all tie (the lowest codes win), and a codebook whose
    rows repeat every 256 codes (each thread of the select then holds many
    equal best keys, which sends it to its radix select) give the indices and
    outputs of the whole-sequence forward."""
    from ssa_amd import CodebookRouter
    from ssa_amd.decode import SSADecodeCache

    print(f"decode n_c={n_c} a={a} periodic={periodic}", flush=True)
    n, h_q, h_kv, d, batch = 120, 8, 2, 128, 2
    q, k, v, _ = _setup(dev, n, h_q, h_kv, d, 64, 24, torch.bfloat16, seed=5, batch=batch)
    q[0, 110] = 0
    k[1, 112] = 0
    q[1, 115], k[1, 115] = 0, 0
    torch.manual_seed(11)
    router = CodebookRouter(head_dim=d, route_dim=32, num_kv_heads=h_kv, num_codebook=n_c,
                            codes_per_key=4, codes_per_query=a, top_k=24, temperature=0.7).to(dev)
    if periodic:
        with torch.no_grad():
            router.codebook.copy_(router.codebook[:, :256].repeat(1, n_c // 256, 1))
    cache = SSADecodeCache(router, batch, 128, d, dtype=torch.bfloat16, tail_tokens=16)
    cache.step(q[:, :100], k[:, :100], v[:, :100])
    for pos in range(100, n):
        out, idx = cache.step(q[:, pos:pos + 1], k[:, pos:pos + 1], v[:, pos:pos + 1],
                              causal_attention=True, return_indices=True)
        ref_idx, ref_out = _prefix_forward(router, q, k, v, pos + 1)
        assert torch.equal(idx, ref_idx[:, pos:]), f"indices differ at {pos}"
        assert torch.equal(out, ref_out[:, pos:]), f"outputs differ at {pos}"
