"""GPU checks of the bucket-mode backward (ssa_sparse_attention_backward_routed).

The indices come from the real routing pipeline on clustered data, so rows
with filler (fewer candidates than top_k) and rows with more candidates than
top_k both occur.  The routed gradients must equal the plain backward's (the
row kernel with one atomic per slot: the same sums in another order, within
2e-5 of max|ref| per tensor) and the float64 oracle's.  Cases: causal and
unmasked routing, causal and unmasked attention, g in {1, 3, 4, 8}, d 64 and
128, int32 and int64 indices in index and score order, a batch of 2, a = 32
codes per query with b = 8 per key, and a bitmap capacity so small that most
rows without filler keep the row kernel's atomics.
"""

import numpy as np
import pytest
import torch

from tests.helpers import clustered_qk, f32, randn, router_params

pytestmark = pytest.mark.gpu


def _pipeline(dev, B, n, h_q, h_kv, d, n_c, a, b, top_k, router_causal, sorted_, index_dtype, seed):
    from ssa_amd import _lib, kernels

    qs, ks = [], []
    for bi in range(B):
        q, k = clustered_qk(n, h_q, h_kv, d, 12, 0.3, seed=seed + bi)
        qs.append(q)
        ks.append(k)
    q = torch.stack(qs).to(torch.bfloat16).to(dev)
    k = torch.stack(ks).to(torch.bfloat16).to(dev)
    v = randn((B, n, h_kv, d), seed + 50, torch.bfloat16).to(dev)
    w_qr, w_kr, cb = router_params(d, 32, h_kv, n_c, seed + 60)
    qc, kc = kernels.route_codes(q, k, w_qr.to(dev), w_kr.to(dev), cb.to(dev), a, b)
    off, post = kernels.build_index(kc, n_c)
    pfx = torch.empty((B, h_kv, n), device=dev, dtype=torch.int32)
    mode = _lib.MASK_CAUSAL if router_causal else _lib.MASK_NONE
    idx, st = kernels.select(q, k, qc, off, post, b, top_k, mode, with_stats=True, sorted=sorted_,
                             index_dtype=index_dtype, row_prefix=pfx)
    return q, k, v, idx, st, pfx, kernels.Routing(qc, kc, off, post, router_causal)


def _grads(dev, q, k, v, idx, pfx, routing, att_causal, seed, bitmap_rows=-1):
    from ssa_amd import kernels

    dout = randn(tuple(q.shape), seed, torch.float32).to(torch.bfloat16).to(dev)
    out32 = torch.empty(q.shape, device=dev, dtype=torch.float32)
    kernels.sparse_attention(q, k, v, idx, None, att_causal, out=out32, row_prefix=pfx)
    plain = kernels.sparse_attention_backward(q, k, v, idx, out32, dout, None, att_causal)
    routed = kernels.sparse_attention_backward(q, k, v, idx, out32, dout, None, att_causal, row_prefix=pfx,
                                               routing=routing, bitmap_rows=bitmap_rows)
    return dout, plain, routed


def _close(name, got, ref, rel=2e-5):
    scale = float(ref.abs().max())
    err = float((got.double() - ref.double()).abs().max())
    assert err <= rel * scale, f"{name}: {err:.3e} > {rel} * {scale:.3e}"


@pytest.mark.parametrize("d,g,router_causal,att_causal,sorted_,i64,B", [
    (128, 4, True, True, False, False, 1),
    (128, 4, True, False, False, True, 1),
    (64, 8, False, False, True, False, 1),
    (128, 1, True, True, True, True, 1),
    (128, 3, False, True, False, False, 2),
])
def test_routed_backward_matches(dev, orc, d, g, router_causal, att_causal, sorted_, i64, B):
    print(f"routed backward d={d} g={g} router_causal={router_causal} att_causal={att_causal} "
          f"sorted={sorted_} i64={i64} B={B}", flush=True)
    n, h_kv, n_c, a, b, top_k = 1500, 2, 256, 8, 4, 128
    q, k, v, idx, st, pfx, routing = _pipeline(dev, B, n, h_kv * g, h_kv, d, n_c, a, b, top_k, router_causal,
                                               sorted_, torch.int64 if i64 else torch.int32, 700 + g)
    C = st[..., 0]
    assert int((C < top_k).sum()) > 0 and int((C > top_k).sum()) > 0, "light and heavy rows"
    dout, plain, routed = _grads(dev, q, k, v, idx, pfx, routing, att_causal, 710 + g)
    for name, got, ref in zip(("dq", "dk", "dv"), routed, plain):
        _close(name, got, ref)
    rq, rk, rv = orc.sparse_attention_backward(f32(q[0]), f32(k[0]), f32(v[0]), idx[0].cpu().numpy().astype(np.int64),
                                               dout[0].double().cpu().numpy(), causal=att_causal)
    for name, got, ref in zip(("dq", "dk", "dv"), routed, (rq, rk, rv)):
        _close(name + " vs oracle", got[0].cpu(), torch.from_numpy(ref))


def test_routed_backward_bitmap_capacity(dev):
    """Rows without filler past the bitmap capacity keep the row kernel's
    atomics; the gradients do not change."""
    print("routed backward, bitmap capacity 3 rows", flush=True)
    n, h_q, h_kv, d, n_c, a, b, top_k = 1200, 8, 2, 128, 128, 8, 4, 96
    q, k, v, idx, st, pfx, routing = _pipeline(dev, 1, n, h_q, h_kv, d, n_c, a, b, top_k, True, False,
                                               torch.int32, 720)
    assert int((pfx == 0).sum()) > 20, "rows without filler"
    _, plain, routed = _grads(dev, q, k, v, idx, pfx, routing, True, 721, bitmap_rows=3)
    for name, got, ref in zip(("dq", "dk", "dv"), routed, plain):
        _close(name, got, ref)
    _, _, routed0 = _grads(dev, q, k, v, idx, pfx, routing, True, 721, bitmap_rows=0)
    for name, got, ref in zip(("dq", "dk", "dv"), routed0, plain):
        _close(name + " (no bitmaps)", got, ref)


def test_routed_backward_wide_codes(dev):
    """a = 32 query codes, b = 8 key codes (pairs sharing several codes are
    common), N_c 1024, top_k 512."""
    print("routed backward a=32 b=8 n_c=1024 top_k=512", flush=True)
    n, h_q, h_kv, d, n_c, a, b, top_k = 2500, 8, 2, 128, 1024, 32, 8, 512
    q, k, v, idx, st, pfx, routing = _pipeline(dev, 1, n, h_q, h_kv, d, n_c, a, b, top_k, True, False,
                                               torch.int32, 730)
    _, plain, routed = _grads(dev, q, k, v, idx, pfx, routing, False, 731)
    for name, got, ref in zip(("dq", "dk", "dv"), routed, plain):
        _close(name, got, ref)


def test_sparse_exact_attention_routing_autograd(dev):
    """sparse_exact_attention(routing=...) carries the routing into its
    backward: the autograd gradients equal those without it."""
    from ssa_amd import sparse_exact_attention

    print("sparse_exact_attention autograd with routing", flush=True)
    n, h_q, h_kv, d, n_c, a, b, top_k = 1000, 8, 2, 64, 128, 8, 4, 64
    q, k, v, idx, st, pfx, routing = _pipeline(dev, 1, n, h_q, h_kv, d, n_c, a, b, top_k, True, False,
                                               torch.int32, 740)
    go = randn((1, n, h_q, d), 741, torch.float32).to(dev)
    grads = []
    for r in (routing, None):
        qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
        out = sparse_exact_attention(qq, kk, vv, idx, causal=True, check_indices=False, row_prefix=pfx, routing=r)
        (out.float() * go).sum().backward()
        grads.append((qq.grad.float(), kk.grad.float(), vv.grad.float()))
    for name, got, ref in zip(("dq", "dk", "dv"), grads[0], grads[1]):
        # bf16 gradients: the two fp32 sums round to bf16 independently
        _close(name, got, ref, rel=1e-2)


@pytest.mark.parametrize("causal,routed", [(True, True), (False, False), (True, False)])
def test_backward_with_forward_row_stats(dev, causal, routed):
    """The forward's row stats (softmax reference in log2 units and 1 / sum per
    row and head) match a float64 recomputation from the selected slots; the
    backward given them (its first pass skipped, NaN rows recomputed) equals the
    backward without them."""
    from ssa_amd import kernels

    print(f"row stats causal={causal} routed={routed}", flush=True)
    n, h_q, h_kv, d, n_c, a, b, top_k = 1200, 8, 2, 128, 128, 8, 4, 96
    q, k, v, idx, st, pfx, routing = _pipeline(dev, 1, n, h_q, h_kv, d, n_c, a, b, top_k, True, False,
                                               torch.int32, 750)
    stats = kernels.row_stats_buffer(q, h_kv)
    out32 = torch.empty(q.shape, device=dev, dtype=torch.float32)
    kernels.sparse_attention(q, k, v, idx, None, causal, out=out32, row_prefix=pfx, row_stats=stats)
    assert not bool(torch.isnan(stats).any()), "the matrix-core forward writes every row"
    # float64 recomputation on sampled rows
    g = h_q // h_kv
    rows = torch.tensor([0, 1, 5, 97, 400, 777, n - 1])
    scale_log2 = 1.4426950408889634 / (d ** 0.5)
    qd, kd, idc = q[0].double().cpu(), k[0].double().cpu(), idx[0].cpu().long()
    for i in rows.tolist():
        for h in range(h_kv):
            keys = idc[i, h]
            if causal:
                keys = keys[keys <= i]
            s = (qd[i, h * g:(h + 1) * g] @ kd[keys, h].T) * scale_log2  # [g, slots]
            m = s.max(-1).values
            inv = 1.0 / torch.exp2(s - m[:, None]).sum(-1)
            got = stats[0, h, i].double().cpu()
            torch.testing.assert_close(got[:, 0], m, rtol=1e-5, atol=1e-5)
            torch.testing.assert_close(got[:, 1], inv, rtol=1e-5, atol=1e-9)
    dout = randn(tuple(q.shape), 751, torch.float32).to(torch.bfloat16).to(dev)
    kw = dict(row_prefix=pfx, routing=routing if routed else None)
    ref = kernels.sparse_attention_backward(q, k, v, idx, out32, dout, None, causal, **kw)
    got = kernels.sparse_attention_backward(q, k, v, idx, out32, dout, None, causal, row_stats=stats, **kw)
    for name, x, y in zip(("dq", "dk", "dv"), got, ref):
        _close(name + " with stats", x, y)
    stats[0, 1, 300:700] = float("nan")  # these rows take the first pass again
    got2 = kernels.sparse_attention_backward(q, k, v, idx, out32, dout, None, causal, row_stats=stats, **kw)
    for name, x, y in zip(("dq", "dk", "dv"), got2, ref):
        _close(name + " with NaN rows", x, y)
