"""CPU checks of oracle.sparse_attention_backward (the float64 restatement of the
autograd backward of ssa/attention.py:64-113).

Two independent pins: torch float64 autograd through the reference's own op
sequence (gather, einsum, / scale, masked softmax, einsum), and central finite
differences of the float64 numpy forward.  Planted mistakes in the oracle's call
(k and v swapped, the scale used as a multiplier, the causal mask dropped) must
fail the finite-difference check.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle


def _inputs(n, h_q, h_kv, d, kk, seed, dup=False):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((n, h_q, d)).astype(np.float32)
    k = rng.standard_normal((n, h_kv, d)).astype(np.float32)
    v = rng.standard_normal((n, h_kv, d)).astype(np.float32)
    idx = rng.integers(0, n, (n, h_kv, kk)).astype(np.int64)
    idx[:, :, 0] = 0  # every causal row keeps at least one slot
    if dup:
        idx[:, :, 1] = idx[:, :, 2]
    dout = rng.standard_normal((n, h_q, d))
    return q, k, v, idx, dout


def _torch_grads(q, k, v, idx, dout, scale, causal):
    """Reference op order (ssa/attention.py:70-113) under torch float64 autograd."""
    n, h_q, d = q.shape
    h_kv = k.shape[1]
    g = h_q // h_kv
    Q = torch.tensor(q, dtype=torch.float64, requires_grad=True)
    K = torch.tensor(k, dtype=torch.float64, requires_grad=True)
    V = torch.tensor(v, dtype=torch.float64, requires_grad=True)
    I = torch.tensor(idx)
    heads = torch.arange(h_kv)[None, :, None]
    kg, vg = K[I, heads], V[I, heads]
    lg = torch.einsum("nhgd,nhkd->nhgk", Q.view(n, h_kv, g, d), kg) / scale
    if causal:
        lg = lg.masked_fill(I[:, :, None, :] > torch.arange(n)[:, None, None, None], float("-inf"))
    p = torch.softmax(lg, dim=-1)
    o = torch.einsum("nhgk,nhkd->nhgd", p, vg).reshape(n, h_q, d)
    (o * torch.tensor(dout)).sum().backward()
    return Q.grad.numpy(), K.grad.numpy(), V.grad.numpy()


@pytest.mark.parametrize("h_q,h_kv", [(2, 2), (4, 2), (8, 1)])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dup", [False, True])
def test_backward_matches_torch_autograd(h_q, h_kv, causal, dup):
    q, k, v, idx, dout = _inputs(24, h_q, h_kv, 16, 6, seed=h_q * 10 + h_kv + int(causal) + 7 * dup, dup=dup)
    scale = 16 ** 0.5
    dq, dk, dv = oracle.sparse_attention_backward(q, k, v, idx, dout, causal=causal)
    tq, tk, tv = _torch_grads(q, k, v, idx, dout, scale, causal)
    for a, b in ((dq, tq), (dk, tk), (dv, tv)):
        np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-12)


def _loss(q, k, v, idx, dout, scale, causal):
    return float((oracle.np_sparse_attention64(q, k, v, idx, scale=scale, causal=causal) * dout).sum())


def _fd_grads(q, k, v, idx, dout, scale, causal, eps=1e-6):
    q, k, v = (np.asarray(t, np.float64).copy() for t in (q, k, v))
    out = []
    for t in (q, k, v):
        gr = np.zeros_like(t)
        for pos in np.ndindex(*t.shape):
            keep = t[pos]
            t[pos] = keep + eps
            up = _loss(q, k, v, idx, dout, scale, causal)
            t[pos] = keep - eps
            dn = _loss(q, k, v, idx, dout, scale, causal)
            t[pos] = keep
            gr[pos] = (up - dn) / (2 * eps)
        out.append(gr)
    return out


def _fd_agrees(grads, fd):
    return all(np.allclose(a, b, rtol=1e-5, atol=1e-6) for a, b in zip(grads, fd))


@pytest.mark.parametrize("causal", [False, True])
def test_backward_matches_finite_differences(causal):
    q, k, v, idx, dout = _inputs(6, 2, 1, 4, 3, seed=3 + int(causal), dup=True)
    scale = 2.0
    fd = _fd_grads(q, k, v, idx, dout, scale, causal)
    assert _fd_agrees(oracle.sparse_attention_backward(q, k, v, idx, dout, scale=scale, causal=causal), fd)


def test_finite_differences_catch_planted_mistakes():
    q, k, v, idx, dout = _inputs(6, 2, 1, 4, 3, seed=11)
    scale = 2.0
    fd = _fd_grads(q, k, v, idx, dout, scale, True)
    good = oracle.sparse_attention_backward(q, k, v, idx, dout, scale=scale, causal=True)
    assert _fd_agrees(good, fd)
    swapped = oracle.sparse_attention_backward(q, v, k, idx, dout, scale=scale, causal=True)
    assert not _fd_agrees(swapped, fd)
    as_multiplier = oracle.sparse_attention_backward(q, k, v, idx, dout, scale=1.0 / scale, causal=True)
    assert not _fd_agrees(as_multiplier, fd)
    no_mask = oracle.sparse_attention_backward(q, k, v, idx, dout, scale=scale, causal=False)
    assert not _fd_agrees(no_mask, fd)


def test_empty_causal_row_has_zero_gradients():
    q, k, v, idx, dout = _inputs(8, 2, 1, 4, 3, seed=5)
    idx[0] = 5  # row 0 keeps no slot under the causal cut
    dq, dk, dv = oracle.sparse_attention_backward(q, k, v, idx, dout, causal=True)
    assert np.all(dq[0] == 0.0)
    # the other rows are unaffected: same gradients as with row 0's dout zeroed
    dout0 = dout.copy()
    dout0[0] = 0.0
    dq0, dk0, dv0 = oracle.sparse_attention_backward(q, k, v, idx, dout0, causal=True)
    np.testing.assert_array_equal(dq[1:], dq0[1:])
    np.testing.assert_allclose(dk, dk0, rtol=0, atol=0)
    np.testing.assert_allclose(dv, dv0, rtol=0, atol=0)
