"""GPU checks of ``reference_flat_gather``: stage (d) reading K and V the way the
reference's code does (ssa/attention.py:76-96: index j of KV head h is row
j + h*n of K flattened to [n*h_kv, d]) through strided views, with no copy.

Forward outputs against the float64 oracle fed with that layout (which
tests/test_oracle.py pins to a float64 restatement of the reference's code),
gradients against float64 autograd of the same code, and the layer with the
option against the router's own indices attended through that layout.
"""

import numpy as np
import pytest
import torch

from tests.helpers import f32, randn

pytestmark = pytest.mark.gpu


def _flat64(t):
    """Contiguous float64-ready copy of the flat-gather layout (host side)."""
    from ssa_amd.attention import flat_gather_view

    return np.ascontiguousarray(flat_gather_view(t.detach().float().cpu()).numpy())


@pytest.mark.parametrize("dtype,d,g,h_kv", [(torch.bfloat16, 128, 4, 2), (torch.float32, 64, 2, 3),
                                            (torch.bfloat16, 64, 8, 2)])
@pytest.mark.parametrize("causal", [False, True])
def test_flat_gather_forward_matches_oracle(dev, orc, dtype, d, g, h_kv, causal):
    from ssa_amd import sparse_exact_attention

    print(f"flat gather forward dtype={dtype} d={d} g={g} h_kv={h_kv} causal={causal}", flush=True)
    n, kk = 700, 96
    q = randn((n, h_kv * g, d), 11, dtype).to(dev)
    k = randn((n, h_kv, d), 12, dtype).to(dev)
    v = randn((n, h_kv, d), 13, dtype).to(dev)
    idx = torch.from_numpy(np.random.default_rng(5).integers(0, n, size=(n, h_kv, kk))).to(dev)
    with torch.no_grad():
        got = sparse_exact_attention(q, k, v, idx, causal=causal, reference_flat_gather=True)
        plain = sparse_exact_attention(q, k, v, idx, causal=causal)
    ref = orc.sparse_attention(f32(q), _flat64(k), _flat64(v), idx.cpu().numpy(), causal=causal)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    # bf16 output: one rounding of 2^-9 on |out| <~ 3
    np.testing.assert_allclose(got.float().cpu().numpy(), ref, rtol=tol, atol=tol)
    assert float((got.float() - plain.float()).abs().max()) > 1e-2, "h_kv > 1: the layouts differ"


def test_flat_gather_gradients_match_float64_autograd(dev):
    """fp32 inputs: dq, dk, dv through the strided view equal float64 autograd
    of the reference's flat gather / softmax / weighted sum within 1e-5."""
    from ssa_amd import sparse_exact_attention

    print("flat gather gradients", flush=True)
    n, h_q, h_kv, d, kk = 300, 8, 2, 64, 48
    q = randn((n, h_q, d), 21).to(dev).requires_grad_(True)
    k = randn((n, h_kv, d), 22).to(dev).requires_grad_(True)
    v = randn((n, h_kv, d), 23).to(dev).requires_grad_(True)
    idx = torch.from_numpy(np.random.default_rng(6).integers(0, n, size=(n, h_kv, kk))).to(dev)
    go = randn((n, h_q, d), 24).to(dev)
    out = sparse_exact_attention(q, k, v, idx, reference_flat_gather=True)
    (out * go).sum().backward()

    q64, k64, v64 = (t.detach().double().cpu().requires_grad_(True) for t in (q, k, v))
    flat = idx.cpu().reshape(-1)
    offs = (torch.arange(h_kv) * n)[None, :, None].expand(n, h_kv, kk).reshape(-1)
    kg = k64.reshape(n * h_kv, d)[flat + offs].reshape(n, h_kv, kk, d)
    vg = v64.reshape(n * h_kv, d)[flat + offs].reshape(n, h_kv, kk, d)
    logit = torch.matmul(q64.reshape(n, h_kv, h_q // h_kv, d), kg.transpose(-1, -2)) / d ** 0.5
    ref = torch.matmul(torch.softmax(logit, -1), vg).reshape(n, h_q, d)
    (ref * go.double().cpu()).sum().backward()
    torch.testing.assert_close(out.detach().double().cpu(), ref.detach(), rtol=1e-5, atol=1e-5)
    for name, got, want in (("dq", q.grad, q64.grad), ("dk", k.grad, k64.grad), ("dv", v.grad, v64.grad)):
        err = float((got.double().cpu() - want).abs().max())
        assert err <= 1e-5 * max(1.0, float(want.abs().max())), f"{name}: {err:.3e}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_layer_flat_gather_attends_the_router_indices_in_that_layout(dev, orc, dtype):
    """SSAAttention(reference_flat_gather=True): the router's indices (unchanged:
    it scores K[j, h] as the reference's router does) attended through the flat
    layout, with the layer's dense prefix and query order."""
    from ssa_amd import SSAAttention, kernels
    from ssa_amd.attention import flat_gather_view

    print(f"layer flat gather dtype={dtype}", flush=True)
    n, hidden, h_q, h_kv, d = 640, 512, 8, 2, 128
    torch.manual_seed(9)
    layer = SSAAttention(hidden_size=hidden, num_q_heads=h_q, num_kv_heads=h_kv, head_dim=d,
                         route_dim=32, num_codebook=64, codes_per_key=4, codes_per_query=8,
                         top_k=96, reference_flat_gather=True).to(dev, dtype).eval()
    x = randn((1, n, hidden), 31, dtype).to(dev)
    with torch.no_grad():
        q, k, v = layer.project(x)
        res = layer.router.route(q, k, causal_mask=True, sorted=False, index_dtype=torch.int32,
                                 with_order=True, with_prefix=True)
        got = layer(x)
        att = torch.empty(q.shape, device=dev, dtype=torch.float32)
        kernels.sparse_attention(q, flat_gather_view(k), flat_gather_view(v), res.indices, None, False,
                                 out=att, row_order=res.order, row_prefix=res.prefix)
    ref = orc.sparse_attention(f32(q[0]), _flat64(k[0]), _flat64(v[0]),
                               res.indices[0].cpu().numpy().astype(np.int64))
    tol = 1e-5 if dtype == torch.float32 else 1e-3
    np.testing.assert_allclose(att[0].cpu().numpy(), ref, rtol=tol, atol=tol)
    with torch.no_grad():
        want = layer.o_proj(att.to(dtype).reshape(1, n, -1)).float()
    err = float((got.float() - want).abs().max())
    assert err <= (1e-5 if dtype == torch.float32 else 1e-2) * float(want.abs().max()), err
