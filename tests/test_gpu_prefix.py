"""GPU checks of stage (d)'s dense-prefix pass (bf16, d 64 / 128, g <= 8).

A row whose indices hold the keys [0, X) exactly once (the lowest-key filler
of a row with fewer candidates than top_k) has those keys attended by
prefix_attention_kernel, one block per run of neighbouring rows, and the row
kernel then skips them.  The result is the same attention in another
summation order: within 1e-5 (fp32 output) of the row path alone, within
1e-3 of the float64 oracle, independent of the processing order.  Rows cover
empty prefixes, prefixes past the causal cut, prefixes longer than the
1024-key bitmap, duplicates inside and outside the prefix, and int32 and int64
indices.
"""

import numpy as np
import pytest
import torch

from tests.helpers import f32, randn

pytestmark = pytest.mark.gpu


def _prefix_rows(n, h_kv, top_k, seed):
    """idx [1, n, h_kv, top_k]: row i of head h holds [0, X) plus top_k - X
    distinct keys >= X, in a shuffled order; X varies along the rows (long for
    early rows, as for rows with few causal candidates) with random jumps."""
    gen = torch.Generator().manual_seed(seed)
    idx = torch.empty(n, h_kv, top_k, dtype=torch.int64)
    xs = torch.empty(n, h_kv, dtype=torch.int64)
    for h in range(h_kv):
        for i in range(n):
            base = max(0, top_k - (i * top_k) // max(1, n // 2))
            jitter = int(torch.randint(0, max(1, top_k // 8), (1,), generator=gen))
            x = min(top_k, n, max(0, base - jitter))
            if int(torch.randint(0, 10, (1,), generator=gen)) == 0:
                x = 0
            rest = torch.randperm(n - x, generator=gen)[: top_k - x] + x
            row = torch.cat([torch.arange(x), rest])
            row = row[torch.randperm(top_k, generator=gen)]
            idx[i, h] = row
            xs[i, h] = x
    return idx.unsqueeze(0), xs


@pytest.mark.parametrize("d,g,top_k,causal,n,i64", [
    (128, 4, 512, True, 1500, False),
    (128, 8, 256, False, 700, True),
    (64, 2, 128, True, 900, False),
    (128, 3, 1536, False, 1700, False),
    (128, 1, 512, True, 600, True),
])
def test_dense_prefix_matches_row_path(dev, orc, d, g, top_k, causal, n, i64):
    from ssa_amd import kernels

    print(f"dense prefix d={d} g={g} top_k={top_k} causal={causal} n={n} i64={i64}", flush=True)
    h_kv = 2
    q = randn((1, n, h_kv * g, d), 301, torch.bfloat16).to(dev)
    k = randn((1, n, h_kv, d), 302, torch.bfloat16).to(dev)
    v = randn((1, n, h_kv, d), 303, torch.bfloat16).to(dev)
    idx, xs = _prefix_rows(n, h_kv, top_k, 304)
    # duplicates: one inside a prefix (the prefix must stop there), one outside
    idx[0, 40, 0, :] = torch.cat([torch.arange(top_k - 1), torch.tensor([5])])
    idx[0, 41, 1, :] = torch.cat([torch.arange(top_k - 1), torch.tensor([top_k - 2])])
    idx = idx.to(torch.int64 if i64 else torch.int32).to(dev)
    assert (xs > 0).float().mean() > 0.3, "the rows must exercise the prefix pass"
    ws = kernels._lib.load().ssa_sparse_attention_workspace_bytes(
        kernels._lib.DTYPE_BF16, 1, n, h_kv * g, h_kv, d, top_k)
    assert ws > 0, "the dense-prefix pass must run for this shape"

    out_p = torch.empty((1, n, h_kv * g, d), device=dev, dtype=torch.float32)
    kernels.sparse_attention(q, k, v, idx, None, causal, out=out_p, dense_prefix=True)
    out_r = torch.empty_like(out_p)
    kernels.sparse_attention(q, k, v, idx, None, causal, out=out_r, dense_prefix=False)
    torch.testing.assert_close(out_p, out_r, rtol=1e-5, atol=1e-5)

    gen = torch.Generator().manual_seed(305)
    order = torch.stack([torch.randperm(n, generator=gen) for _ in range(h_kv)]).to(torch.int32)
    out_o = torch.empty_like(out_p)
    kernels.sparse_attention(q, k, v, idx, None, causal, out=out_o, row_order=order.unsqueeze(0).to(dev))
    assert torch.equal(out_o, out_p), "the processing order must not change any row"

    bf = kernels.sparse_attention(q, k, v, idx, None, causal)  # bf16 output
    torch.testing.assert_close(bf.float(), out_p, rtol=1e-2, atol=1e-2)
    # the bf16 store rounds the same fp32 values to nearest even, as torch does
    assert torch.equal(bf, out_p.to(torch.bfloat16)), "bf16 output must be the fp32 output rounded"

    rows = np.unique(np.concatenate([np.arange(0, 8), [40, 41], np.arange(n // 2 - 4, n // 2 + 4),
                                     np.arange(n - 8, n)]))
    ref = orc.sparse_attention(f32(q[0]), f32(k[0]), f32(v[0]), idx[0].cpu().numpy().astype(np.int64)[rows],
                               causal=causal, rows=rows)
    np.testing.assert_allclose(out_p[0].cpu().numpy()[rows], ref, rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("sorted_,use_ws", [(False, True), (True, True), (False, False)])
def test_select_row_prefix(dev, sorted_, use_ws):
    """ssa_select's row_prefix: for a row with fewer candidates than top_k, X
    is its last filler key + 1 (the filler is the lowest keys it does not
    hold, so it holds [0, X) once), else 0 -- in both output orders, with and
    without the workspace path; attention given X equals the row path."""
    from ssa_amd import kernels
    from tests.helpers import clustered_qk, router_params

    print(f"select row_prefix sorted={sorted_} workspace={use_ws}", flush=True)
    n, h_q, h_kv, d, n_c, a, b, top_k = 3000, 8, 2, 128, 256, 8, 4, 256
    q, k = clustered_qk(n, h_q, h_kv, d, 8, 0.3, seed=11)
    w_qr, w_kr, cb = router_params(d, 32, h_kv, n_c, seed=12)
    q = q.to(torch.bfloat16).unsqueeze(0).to(dev)
    k = k.to(torch.bfloat16).unsqueeze(0).to(dev)
    v = randn((1, n, h_kv, d), 13, torch.bfloat16).to(dev)
    qc, kc = kernels.route_codes(q, k, w_qr.to(dev), w_kr.to(dev), cb.to(dev), a, b)
    off, post = kernels.build_index(kc, n_c)
    pfx = torch.full((1, h_kv, n), -5, device=dev, dtype=torch.int32)
    idx, st = kernels.select(q, k, qc, off, post, b, top_k, with_stats=True, sorted=sorted_,
                             use_workspace=use_ws, index_dtype=torch.int32, row_prefix=pfx)
    rows = idx.permute(0, 2, 1, 3)                        # [1, h_kv, n, top_k]
    C = st[..., 0]
    want = torch.where(C < top_k, rows[..., top_k - 1] + 1, torch.zeros_like(C))
    assert torch.equal(pfx, want)
    assert int((want > 0).sum()) > n // 4 and int((C > top_k).sum()) > 0, "light and heavy rows"
    # every row holds [0, X) exactly once
    srt = rows.sort(-1).values.cpu()
    x = pfx.cpu()
    ar = torch.arange(top_k)
    assert bool(((srt == ar) | (ar >= x[..., None])).all())

    out_p = torch.empty((1, n, h_q, d), device=dev, dtype=torch.float32)
    kernels.sparse_attention(q, k, v, idx, None, True, out=out_p, row_prefix=pfx)
    out_r = torch.empty_like(out_p)
    kernels.sparse_attention(q, k, v, idx, None, True, out=out_r, dense_prefix=False)
    torch.testing.assert_close(out_p, out_r, rtol=1e-5, atol=1e-5)
    out_i = torch.empty_like(out_p)
    kernels.sparse_attention(q, k, v, idx, None, True, out=out_i)  # X found from the indices
    torch.testing.assert_close(out_i, out_r, rtol=1e-5, atol=1e-5)


def _first_free(idx_row, cap):
    """X of one index row: the first key in [0, cap) it does not hold, lowered
    to the smallest key it holds twice (as the dense pass finds it)."""
    vals, counts = np.unique(idx_row, return_counts=True)
    x = 0
    held = set(vals.tolist())
    while x < cap and x in held:
        x += 1
    dups = vals[counts > 1]
    return int(min(x, dups.min())) if dups.size else x


@pytest.mark.parametrize("d,g,causal,n", [(128, 4, True, 700), (64, 8, False, 500), (128, 3, True, 333)])
def test_backward_dense_prefix(dev, orc, d, g, causal, n):
    """Gradients with the dense-prefix pass (row_prefix given: the row kernel
    skips [0, X), blocks of 8 rows take it) equal the row path's and the
    float64 oracle's (max|err| <= 2e-5 max|ref| per tensor, fp32 forward
    output)."""
    from ssa_amd import kernels

    print(f"backward dense prefix d={d} g={g} causal={causal} n={n}", flush=True)
    h_kv, top_k = 2, 128
    q = randn((1, n, h_kv * g, d), 401, torch.bfloat16)
    k = randn((1, n, h_kv, d), 402, torch.bfloat16)
    v = randn((1, n, h_kv, d), 403, torch.bfloat16)
    dout = randn((1, n, h_kv * g, d), 404, torch.float32).to(torch.bfloat16)
    idx, _ = _prefix_rows(n, h_kv, top_k, 405)
    idx[0, 40, 0, :] = torch.cat([torch.arange(top_k - 1), torch.tensor([5])])  # a duplicate in a prefix
    xs = np.array([[_first_free(idx[0, i, h].numpy(), top_k) for i in range(n)] for h in range(h_kv)],
                  dtype=np.int32)
    assert (xs > 0).mean() > 0.3
    pfx = torch.from_numpy(xs).unsqueeze(0).contiguous().to(dev)
    qd, kd, vd, idd, dod = q.to(dev), k.to(dev), v.to(dev), idx.to(torch.int32).to(dev), dout.to(dev)
    out32 = torch.empty(qd.shape, device=dev, dtype=torch.float32)
    kernels.sparse_attention(qd, kd, vd, idd, None, causal, out=out32, row_prefix=pfx)
    got = kernels.sparse_attention_backward(qd, kd, vd, idd, out32, dod, None, causal, row_prefix=pfx)
    ref_row = kernels.sparse_attention_backward(qd, kd, vd, idd, out32, dod, None, causal)
    rq, rk, rv = [np.stack([o]) for o in orc.sparse_attention_backward(
        f32(q[0]), f32(k[0]), f32(v[0]), idx[0].numpy(), dout[0].double().numpy(), causal=causal)]
    for name, a, b, r in zip(("dq", "dk", "dv"), got, ref_row, (rq, rk, rv)):
        scale = float(np.abs(r).max())
        err_o = float((a.cpu().double() - torch.from_numpy(r)).abs().max())
        err_r = float((a - b).abs().max())
        assert err_o <= 2e-5 * scale, f"{name} vs oracle: {err_o:.3e} > 2e-5 * {scale:.3e}"
        assert err_r <= 2e-5 * scale, f"{name} vs row path: {err_r:.3e} > 2e-5 * {scale:.3e}"


def test_nan_query_propagates_to_its_head_only(dev):
    """A NaN in one query head's vector makes that head's output row NaN in the
    fp32 and the bf16 output (the bf16 store keeps NaN a NaN), and leaves every
    other (row, head) finite and the bf16 output the fp32 output rounded."""
    from ssa_amd import kernels

    print("nan query", flush=True)
    n, h_kv, g, d, top_k = 300, 2, 4, 128, 64
    q = randn((1, n, h_kv * g, d), 501, torch.bfloat16)
    q[0, 10, 5, 7] = float("nan")
    q = q.to(dev)
    k = randn((1, n, h_kv, d), 502, torch.bfloat16).to(dev)
    v = randn((1, n, h_kv, d), 503, torch.bfloat16).to(dev)
    gen = torch.Generator().manual_seed(504)
    idx = torch.stack([torch.randperm(n, generator=gen)[:top_k] for _ in range(n * h_kv)])
    idx = idx.reshape(1, n, h_kv, top_k).to(torch.int32).to(dev)
    out32 = torch.empty((1, n, h_kv * g, d), device=dev, dtype=torch.float32)
    kernels.sparse_attention(q, k, v, idx, None, False, out=out32)
    bf = kernels.sparse_attention(q, k, v, idx, None, False)
    bad = torch.zeros((1, n, h_kv * g), dtype=torch.bool)
    bad[0, 10, 5] = True
    for o in (out32, bf):
        nan_rows = torch.isnan(o.float()).all(-1).cpu()
        assert torch.equal(nan_rows, bad), "only the NaN query's head may be NaN"
        assert bool(torch.isfinite(o.float()[~bad.to(dev)]).all())
    assert torch.equal(bf[~bad.to(dev)], out32.to(torch.bfloat16)[~bad.to(dev)])
