"""GPU checks of the stage-(d) backward (ssa_sparse_attention_backward) against the
float64 oracle, through the C ABI wrapper and through autograd
(sparse_exact_attention, SSAAttention).

Tolerances: gradients are compared with max|HIP - oracle| <= tol * max|oracle|
per tensor.  With the forward output passed in fp32, tol = 2e-5 for fp32 and
bf16 inputs alike (the oracle sees the same input values; the HIP path works in
fp32, atomics in any order).  A bf16 forward output carries a relative rounding
of 2^-9 into D = dO . o, so that path is checked at 1e-2; the autograd path keeps
an fp32 copy of the output for the backward.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.helpers import f32

pytestmark = pytest.mark.gpu


def _case(B, n, h_q, h_kv, d, kk, seed, dtype, dup=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, n, h_q, d, generator=g).to(dtype)
    k = torch.randn(B, n, h_kv, d, generator=g).to(dtype)
    v = torch.randn(B, n, h_kv, d, generator=g).to(dtype)
    idx = torch.randint(0, n, (B, n, h_kv, kk), generator=g)
    idx[..., 0] = 0
    if dup and kk > 2:
        idx[..., 1] = idx[..., 2]
    dout = torch.randn(B, n, h_q, d, generator=g)
    return q, k, v, idx, dout


def _oracle(orc, q, k, v, idx, dout, causal, scale=None):
    outs = [orc.sparse_attention_backward(f32(q[b]), f32(k[b]), f32(v[b]), idx[b].numpy(),
                                          dout[b].double().numpy(), scale=scale, causal=causal)
            for b in range(q.shape[0])]
    return [np.stack([o[i] for o in outs]) for i in range(3)]


def _close(got, ref, tol, what):
    err = float(np.abs(got - ref).max())
    scale = float(np.abs(ref).max())
    assert err <= tol * scale, f"{what}: max|err| {err:.3e} > {tol} * {scale:.3e}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("h_q,h_kv,d", [(4, 4, 64), (8, 2, 128), (16, 2, 64), (16, 1, 256), (6, 2, 40)])
@pytest.mark.parametrize("causal", [False, True])
def test_backward_matches_oracle(dev, orc, dtype, h_q, h_kv, d, causal):
    from ssa_amd import kernels

    q, k, v, idx, dout = _case(2, 96, h_q, h_kv, d, 24, seed=h_q * 31 + d + int(causal), dtype=dtype,
                               dup=True)
    qd, kd, vd, idd = q.to(dev), k.to(dev), v.to(dev), idx.to(dev)
    out32 = torch.empty(q.shape, device=dev, dtype=torch.float32)
    kernels.sparse_attention(qd, kd, vd, idd, None, causal, out=out32)
    # the oracle takes dout as given to the kernel (rounded to the input dtype)
    rq, rk, rv = _oracle(orc, q, k, v, idx, dout.to(dtype).float(), causal)
    dq, dk, dv = kernels.sparse_attention_backward(qd, kd, vd, idd, out32, dout.to(dev, dtype), None, causal)
    _close(dq.cpu().numpy(), rq, 2e-5, "dq")
    _close(dk.cpu().numpy(), rk, 2e-5, "dk")
    _close(dv.cpu().numpy(), rv, 2e-5, "dv")
    if dtype == torch.bfloat16:  # forward output stored in bf16
        out16 = kernels.sparse_attention(qd, kd, vd, idd, None, causal)
        dq, dk, dv = kernels.sparse_attention_backward(qd, kd, vd, idd, out16, dout.to(dev, dtype), None,
                                                       causal)
        _close(dq.cpu().numpy(), rq, 1e-2, "dq (bf16 output)")
        _close(dk.cpu().numpy(), rk, 1e-2, "dk (bf16 output)")
        _close(dv.cpu().numpy(), rv, 1e-2, "dv (bf16 output)")


def test_backward_int32_indices_row_order_and_scale(dev, orc):
    from ssa_amd import kernels

    B, n, h_q, h_kv, d, kk = 1, 128, 8, 2, 128, 32
    q, k, v, idx, dout = _case(B, n, h_q, h_kv, d, kk, seed=5, dtype=torch.float32)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    order = torch.stack([torch.randperm(n, generator=torch.Generator().manual_seed(h)) for h in range(h_kv)])
    order = order.to(torch.int32)[None].to(dev)
    out = kernels.sparse_attention(qd, kd, vd, idx.to(dev), 3.0, True)
    a = kernels.sparse_attention_backward(qd, kd, vd, idx.to(dev), out, dout.to(dev), 3.0, True)
    b = kernels.sparse_attention_backward(qd, kd, vd, idx.to(dev, torch.int32), out, dout.to(dev), 3.0,
                                          True, row_order=order)
    ref = _oracle(orc, q, k, v, idx, dout, True, scale=3.0)
    for x, y, r, name in zip(a, b, ref, ("dq", "dk", "dv")):
        _close(x.cpu().numpy(), r, 2e-5, name)
        _close(y.cpu().numpy(), r, 2e-5, name + " (int32, row order)")


def test_backward_flags_out_of_range(dev):
    from ssa_amd import kernels

    q, k, v, idx, dout = _case(1, 32, 4, 2, 64, 8, seed=9, dtype=torch.float32)
    idx[0, 3, 1, 2] = 32  # past n
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    out = kernels.sparse_attention(q.to(dev), k.to(dev), v.to(dev), idx.to(dev), None, False,
                                   error_flag=flag)
    flag.zero_()
    kernels.sparse_attention_backward(q.to(dev), k.to(dev), v.to(dev), idx.to(dev), out, dout.to(dev),
                                      None, False, error_flag=flag)
    assert int(flag.item()) == 1


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_autograd_through_sparse_exact_attention(dev, orc, dtype):
    from ssa_amd import sparse_exact_attention

    n, h_q, h_kv, d, kk = 64, 8, 2, 64, 16
    q, k, v, idx, dout = _case(1, n, h_q, h_kv, d, kk, seed=21, dtype=dtype)
    qd = q[0].to(dev).requires_grad_()
    kd = k[0].to(dev).requires_grad_()
    vd = v[0].to(dev).requires_grad_()
    out = sparse_exact_attention(qd, kd, vd, idx[0].to(dev), causal=True)
    out.backward(dout[0].to(dev, dtype))
    rq, rk, rv = _oracle(orc, q, k, v, idx, dout.to(dtype).float(), True)
    tol = 2e-5 if dtype == torch.float32 else 1e-2  # bf16 gradients are rounded to bf16
    _close(qd.grad.float().cpu().numpy(), rq[0], tol, "q.grad")
    _close(kd.grad.float().cpu().numpy(), rk[0], tol, "k.grad")
    _close(vd.grad.float().cpu().numpy(), rv[0], tol, "v.grad")


@pytest.mark.parametrize("causal_attention,rope", [(False, False), (False, True), (True, True)])
def test_layer_gradient_flow_matches_reference_formula(dev, causal_attention, rope):
    """tests/test_integration.py:32-49 of the reference (gradients reach q/k/v/o_proj
    and the input), and the gradients equal those of the reference's op sequence
    (apply_rope on [n, h, d], gather, einsum, / scale, softmax, einsum) run under
    float64 autograd on the CPU with the layer's own indices.  With rope the
    layer's HIP RoPE kernel and its transpose are on the gradient path."""
    from ssa_amd import SSAAttention, precompute_rope_freqs
    from ssa_amd.utils import apply_rope

    print(f"layer gradients causal_attention={causal_attention} rope={rope}", flush=True)
    torch.manual_seed(0)
    kw = dict(hidden_size=256, num_q_heads=4, num_kv_heads=1, head_dim=64, route_dim=16,
              num_codebook=128, codes_per_key=4, codes_per_query=8, top_k=16,
              causal_attention=causal_attention)
    layer = SSAAttention(**kw)
    x = torch.randn(2, 32, 256)
    ref_layer = SSAAttention(**kw)
    ref_layer.load_state_dict(layer.state_dict())
    layer = layer.to(dev)
    freqs = precompute_rope_freqs(64, 32, 1e4) if rope else None
    xd = x.to(dev).requires_grad_()
    out = layer(xd, freqs=freqs.to(dev) if rope else None)
    out.sum().backward()
    for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
        gr = getattr(layer, name).weight.grad
        assert gr is not None and torch.isfinite(gr).all(), name
    assert xd.grad is not None and torch.isfinite(xd.grad).all()

    # reference op sequence in float64 on the CPU, same indices as the layer routed
    with torch.no_grad():
        q, k, _ = layer.project(x.to(dev), freqs=freqs.to(dev) if rope else None)
        idx = torch.stack([layer.router(q[b], k[b], causal_mask=True) for b in range(2)]).cpu()
    ref_layer = ref_layer.double()
    xr = x.double().requires_grad_()
    B, n = 2, 32
    h_q, d = 4, 64
    q = ref_layer.q_proj(xr).view(B, n, h_q, d)
    k = ref_layer.k_proj(xr).view(B, n, 1, d)
    v = ref_layer.v_proj(xr).view(B, n, 1, d)
    heads = torch.arange(1)[None, :, None]
    outs = []
    for b in range(B):
        qb, kb = q[b], k[b]
        if rope:  # ssa/ssa_layer.py:115-117: apply_rope on [n, heads, d]
            qb, kb = apply_rope(qb, freqs.double()), apply_rope(kb, freqs.double())
        kg, vg = kb[idx[b], heads], v[b][idx[b], heads]
        lg = torch.einsum("nhgd,nhkd->nhgk", qb.reshape(n, 1, h_q, d), kg) / d ** 0.5
        if causal_attention:  # drops selected keys past the query
            fut = idx[b][:, :, None, :] > torch.arange(n)[:, None, None, None]
            lg = lg.masked_fill(fut, float("-inf"))
        p = torch.softmax(lg, dim=-1)
        outs.append(torch.einsum("nhgk,nhkd->nhgd", p, vg).reshape(n, h_q * d))
    ref_out = ref_layer.o_proj(torch.stack(outs))
    ref_out.sum().backward()
    np.testing.assert_allclose(out.detach().cpu().double().numpy(), ref_out.detach().numpy(), rtol=1e-4, atol=1e-4)
    for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
        got = getattr(layer, name).weight.grad.cpu().double()
        ref = getattr(ref_layer, name).weight.grad
        err = float((got - ref).abs().max())
        assert err <= 1e-4 * float(ref.abs().max()) + 1e-6, f"{name}: {err:.3e}"
    err = float((xd.grad.cpu().double() - xr.grad).abs().max())
    assert err <= 1e-4 * float(xr.grad.abs().max()) + 1e-6
