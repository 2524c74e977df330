"""Block-granular variant on the GPU: ssa_block_indices (bit-exact with the
oracle) and ssa_block_sparse_attention (against the float64 restatement)."""

import numpy as np
import pytest
import torch

from tests.helpers import f32, randn

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-blocks] {msg}", flush=True)


@pytest.mark.parametrize("B,n,h,k,bs,nkb,i64", [(2, 1000, 2, 64, 64, None, True), (1, 4096, 8, 512, 64, None, False),
                                                 (1, 777, 3, 40, 16, 10, True), (2, 300, 1, 9, 2, 150, False)])
def test_block_indices_bit_exact(dev, orc, B, n, h, k, bs, nkb, i64):
    from ssa_amd import kernels

    _say(f"block_indices B={B} n={n} h={h} k={k} bs={bs} nkb={nkb}")
    g = torch.Generator().manual_seed(n + k)
    idx = torch.randint(0, n, (B, n, h, k), generator=g)
    idx = idx if i64 else idx.to(torch.int32)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    got = kernels.block_indices(idx.to(dev), bs, nkb, error_flag=flag).cpu().numpy()
    assert int(flag.item()) == 0
    for b in range(B):
        np.testing.assert_array_equal(got[b], orc.block_indices(idx[b].numpy(), bs, nkb))


def test_block_indices_flags_out_of_range(dev, orc):
    from ssa_amd import kernels

    idx = torch.zeros(1, 64, 1, 4, dtype=torch.int64)
    idx[0, 5, 0, 2] = 64
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    kernels.block_indices(idx.to(dev), 16, error_flag=flag)
    assert int(flag.item()) == 1


@pytest.mark.parametrize("dtype,d,g,tol", [(torch.float32, 64, 4, 1e-5), (torch.bfloat16, 128, 4, 1e-3),
                                           (torch.bfloat16, 64, 8, 1e-3), (torch.float32, 32, 1, 1e-5)])
@pytest.mark.parametrize("n,bs,nkb", [(512, 64, 3), (333, 32, 4), (200, 16, 13)])
def test_block_sparse_attention_vs_oracle(dev, orc, dtype, d, g, tol, n, bs, nkb):
    from ssa_amd import kernels

    _say(f"block attention dtype={dtype} d={d} g={g} n={n} bs={bs} nkb={nkb}")
    B, h_kv = 2, 2
    h_q = h_kv * g
    q = randn((B, n, h_q, d), 51, dtype)
    k = randn((B, n, h_kv, d), 52, dtype)
    v = randn((B, n, h_kv, d), 53, dtype)
    nb = (n + bs - 1) // bs
    gen = torch.Generator().manual_seed(54)
    blocks = torch.stack([torch.randperm(nb, generator=gen)[:nkb] for _ in range(B * nb * h_kv)])
    blocks = blocks.view(B, nb, h_kv, nkb)
    out = torch.empty(B, n, h_q, d, device=dev, dtype=torch.float32)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    kernels.block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), blocks.to(dev), bs, out=out,
                                   error_flag=flag)
    assert int(flag.item()) == 0
    got = out.cpu().numpy()
    for b in range(B):
        ref = orc.block_sparse_attention64(f32(q[b]), f32(k[b]), f32(v[b]), blocks[b].numpy(), bs)
        np.testing.assert_allclose(got[b], ref, rtol=tol, atol=tol)


def test_block_sparse_attention_flags_bad_block(dev, orc):
    from ssa_amd import kernels

    n, bs = 128, 32
    q, k, v = randn((1, n, 2, 64), 61), randn((1, n, 1, 64), 62), randn((1, n, 1, 64), 63)
    blocks = torch.zeros(1, n // bs, 1, 2, dtype=torch.int64)
    blocks[0, 2, 0, 1] = n // bs
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    kernels.block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), blocks.to(dev), bs, error_flag=flag)
    assert int(flag.item()) == 1


def test_router_blocks_pipeline_all_blocks_is_dense(dev, orc):
    """Router selections -> convert_indices_to_blocks -> block attention.  With
    k >= the number of blocks every block is listed, so the result is causal
    dense attention (fp32, within 1e-5)."""
    from ssa_amd import CodebookRouter
    from ssa_amd.blocks import block_sparse_attention, convert_indices_to_blocks

    n, h_q, h_kv, d, bs = 1000, 8, 2, 64, 64
    q, k, v = randn((n, h_q, d), 71), randn((n, h_kv, d), 72), randn((n, h_kv, d), 73)
    torch.manual_seed(74)
    r = CodebookRouter(head_dim=d, route_dim=16, num_kv_heads=h_kv, num_codebook=64, codes_per_key=4,
                       codes_per_query=8, top_k=32).to(dev)
    idx = r(q.to(dev), k.to(dev), causal_mask=True)
    blocks = convert_indices_to_blocks(idx, bs)
    nb = (n + bs - 1) // bs
    assert tuple(blocks.shape) == (nb, h_kv, min(32, nb))
    np.testing.assert_array_equal(blocks.cpu().numpy(), orc.block_indices(idx.cpu().numpy(), bs))
    got = block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), blocks, bs).cpu().numpy()
    ref = orc.dense_attention(f32(q), f32(k), f32(v), causal=True)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


def test_ssa_triton_attention_name_and_fp16(dev, orc):
    """The reference launcher's name and signature (ssa/triton_kernel.py:141-148)
    with fp16 inputs (the reference kernel's type), widened exactly to fp32: the
    output equals the fp32 call rounded to fp16, and the float64 restatement
    within 1e-3."""
    from ssa_amd.blocks import block_sparse_attention, ssa_triton_attention

    n, h_q, h_kv, d, bs, nkb = 300, 4, 2, 64, 64, 3
    q, k, v = (randn((n, h, d), s).to(torch.float16) for h, s in ((h_q, 81), (h_kv, 82), (h_kv, 83)))
    nb = (n + bs - 1) // bs
    g = torch.Generator().manual_seed(84)
    blocks = torch.randint(0, nb, (nb, h_kv, nkb), generator=g)
    got = ssa_triton_attention(q.to(dev), k.to(dev), v.to(dev), blocks.to(dev), bs)
    assert got.dtype == torch.float16
    ref32 = block_sparse_attention(q.float().to(dev), k.float().to(dev), v.float().to(dev),
                                   blocks.to(dev), bs)
    assert torch.equal(got, ref32.to(torch.float16))
    ref = orc.block_sparse_attention64(f32(q), f32(k), f32(v), blocks.numpy(), bs)
    np.testing.assert_allclose(got.float().cpu().numpy(), ref, rtol=1e-3, atol=1e-3)
