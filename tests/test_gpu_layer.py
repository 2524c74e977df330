"""The SSAAttention layer end to end on the GPU, and the int32 index handoff the
layer uses between stages (c) and (d).

The layer's forward (ssa/ssa_layer.py:68-138) is checked against the CPU oracle
fed with the layer's own projections: candidate indices bit-exact, the
attention output and the output after o_proj within the stated tolerances.
"""

import numpy as np
import pytest
import torch

from tests.helpers import f32, randn

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("causal_attention", [True, False])
def test_layer_forward_matches_oracle(dev, orc, dtype, causal_attention):
    """B=2, n=300, hidden 256, GQA 4/2, d=64, d_s=16, N_c=64, b=2, a=8, k=32, RoPE.

    Indices bit-exact.  fp32: the attention output and the layer output within
    rtol = atol = 1e-5 of the oracle (float64 o_proj of the oracle's attention).
    bf16: the attention output computed in fp32 from the layer's bf16 q/k/v
    within rtol = atol = 1e-3; the layer output (a bf16 o_proj of the bf16
    attention output, two bf16 roundings of 2^-9) within 1e-2 of max|ref|."""
    from ssa_amd import SSAAttention, kernels, precompute_rope_freqs

    _say(f"layer forward dtype={dtype} causal_attention={causal_attention}")
    B, n, hidden, h_q, h_kv, d, d_s, n_c, b, a, k = 2, 300, 256, 4, 2, 64, 16, 64, 2, 8, 32
    torch.manual_seed(5)
    layer = SSAAttention(hidden_size=hidden, num_q_heads=h_q, num_kv_heads=h_kv, head_dim=d,
                         route_dim=d_s, num_codebook=n_c, codes_per_key=b, codes_per_query=a,
                         top_k=k, causal_attention=causal_attention)
    layer = layer.to(dev, dtype).eval()
    x = randn((B, n, hidden), 51, dtype).to(dev)
    freqs = precompute_rope_freqs(d, n, 1e6).to(dev)
    with torch.no_grad():
        got = layer(x, freqs=freqs).float().cpu().numpy()
        q, kk, v = layer.project(x, None, freqs)
        r = layer.router
        idx32 = r.route(q, kk, causal_mask=True, sorted=False, index_dtype=torch.int32).indices
        idx64 = r.route(q, kk, causal_mask=True, sorted=False).indices
        att32 = torch.empty(q.shape, device=dev, dtype=torch.float32)
        kernels.sparse_attention(q, kk, v, idx32, None, causal_attention, out=att32)
    assert idx32.dtype == torch.int32 and idx64.dtype == torch.int64
    assert torch.equal(idx32.to(torch.int64), idx64)
    w_o = f32(layer.o_proj.weight).astype(np.float64)
    att_tol = 1e-5 if dtype == torch.float32 else 1e-3
    for bb in range(B):
        qf, kf, vf = f32(q[bb]), f32(kk[bb]), f32(v[bb])
        ref_idx, _ = orc.router_forward(qf, kf, f32(r.W_qr.weight), f32(r.W_kr.weight),
                                        f32(r.codebook), a, b, k, orc.MASK_CAUSAL, sorted=False)
        np.testing.assert_array_equal(idx64[bb].cpu().numpy(), ref_idx)
        att = orc.sparse_attention(qf, kf, vf, ref_idx, causal=causal_attention)
        np.testing.assert_allclose(att32[bb].cpu().numpy(), att, rtol=att_tol, atol=att_tol)
        if dtype == torch.float32:
            ref = att.reshape(n, h_q * d) @ w_o.T
            np.testing.assert_allclose(got[bb], ref, rtol=1e-5, atol=1e-5)
        else:
            ref = orc.bf16_round(att.astype(np.float32)).reshape(n, h_q * d).astype(np.float64) @ w_o.T
            err = float(np.abs(got[bb] - ref).max())
            assert err <= 1e-2 * float(np.abs(ref).max()), (bb, err)


@pytest.mark.parametrize("dtype,d,g", [(torch.bfloat16, 128, 4), (torch.bfloat16, 64, 8),
                                       (torch.float32, 64, 2), (torch.bfloat16, 96, 2)])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_int32_indices_equal_int64(dev, dtype, d, g, causal):
    """Both attention kernels read int32 and int64 indices to bit-identical outputs."""
    from ssa_amd import kernels

    _say(f"attention int32 vs int64 dtype={dtype} d={d} g={g} causal={causal}")
    B, n, h_kv, top_k = 2, 400, 2, 96
    q = randn((B, n, h_kv * g, d), 61, dtype).to(dev)
    k = randn((B, n, h_kv, d), 62, dtype).to(dev)
    v = randn((B, n, h_kv, d), 63, dtype).to(dev)
    gi = torch.Generator().manual_seed(64)
    idx = torch.randint(0, n, (B, n, h_kv, top_k), generator=gi).to(dev)
    o64 = torch.empty(q.shape, device=dev, dtype=torch.float32)
    o32 = torch.empty_like(o64)
    kernels.sparse_attention(q, k, v, idx, None, causal, out=o64)
    kernels.sparse_attention(q, k, v, idx.to(torch.int32), None, causal, out=o32)
    assert torch.equal(o64, o32)


@pytest.mark.parametrize("d,g", [(128, 4), (64, 8)])
def test_attention_k_v_with_different_row_strides(dev, orc, d, g):
    """K and V as views with different row strides (K sliced out of a wider
    tensor), and a top_k that leaves a partial last chunk: the same output as
    contiguous copies, and the oracle's within the bf16 tolerance."""
    from ssa_amd import kernels

    _say(f"attention strided K/V d={d} g={g}")
    B, n, h_kv, top_k = 2, 333, 2, 77
    q = randn((B, n, h_kv * g, d), 71, torch.bfloat16).to(dev)
    kw = randn((B, n, 3 * h_kv, d), 72, torch.bfloat16).to(dev)
    k = kw[:, :, h_kv:2 * h_kv]                      # row stride 3*h_kv*d
    v = randn((B, n, h_kv, d), 73, torch.bfloat16).to(dev)
    gi = torch.Generator().manual_seed(74)
    idx = torch.randint(0, n, (B, n, h_kv, top_k), generator=gi).to(dev)
    assert k.stride(1) != v.stride(1)
    for causal in (False, True):
        o = torch.empty(q.shape, device=dev, dtype=torch.float32)
        oc = torch.empty_like(o)
        kernels.sparse_attention(q, k, v, idx, None, causal, out=o)
        kernels.sparse_attention(q, k.contiguous(), v, idx, None, causal, out=oc)
        assert torch.equal(o, oc)
        got = o.cpu().numpy()
        for bb in range(B):
            ref = orc.sparse_attention(f32(q[bb]), f32(k[bb]), f32(v[bb]), idx[bb].cpu().numpy(),
                                       causal=causal)
            np.testing.assert_allclose(got[bb], ref, rtol=1e-3, atol=1e-3)
