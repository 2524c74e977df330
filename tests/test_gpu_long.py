"""Full-size parity at the long-context workloads: config 3 (n=32768, bf16,
GQA 32/8, d 128, d_s 32, N_c 4096, a 16, b 4, k 512, 64-cluster inputs) and
config 5 (n=131072, GQA 16/2, N_c 8192, a 32, k 1024, 256-cluster inputs),
both causal.

The oracle is too slow for every row at these sizes, so each stage is checked
on sampled rows against the oracle fed with the previous stage's (already
verified) GPU output, and the whole output is checked through size-independent
properties.  Sampled rows always include the rows with the most candidates,
which exercise the streaming top-k with several rescoring batches.
"""

import numpy as np
import pytest
import torch

import bench

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", params=["c3", "c5"])
def lc(dev, request):
    from ssa_amd import kernels
    from ssa_amd.router import query_order

    print(f"{request.param}: generating workload", flush=True)
    cfg = dict(bench.CONFIGS[request.param])
    q, k, v, router = bench.make_workload(cfg, 0, dev)
    qc, kc = kernels.route_codes(q, k, router.W_qr.weight, router.W_kr.weight, router.codebook,
                                 cfg["a"], cfg["b"])
    off, post = kernels.build_index(kc, cfg["n_c"])
    idx_s, st = kernels.select(q, k, qc, off, post, cfg["b"], cfg["k"], with_stats=True, sorted=True)
    idx_u = kernels.select(q, k, qc, off, post, cfg["b"], cfg["k"], sorted=False)
    idx_u2 = kernels.select(q, k, qc, off, post, cfg["b"], cfg["k"], sorted=False)
    idx_ub, st_ub = kernels.select(q, k, qc, off, post, cfg["b"], cfg["k"], sorted=False,
                                   with_stats=True, use_workspace=False)
    _, st_u = kernels.select(q, k, qc, off, post, cfg["b"], cfg["k"], sorted=False, with_stats=True)
    idx_s2 = kernels.select(q, k, qc, off, post, cfg["b"], cfg["k"], sorted=True)
    out = torch.empty(q.shape, device=dev, dtype=torch.float32)
    kernels.sparse_attention(q, k, v, idx_u, None, True, out=out)
    order = query_order(qc, cfg["n_c"])
    out_ord = torch.empty_like(out)
    kernels.sparse_attention(q, k, v, idx_u, None, True, out=out_ord, row_order=order)
    # the headline call, as bench.py times it and SSAAttention makes it: int32
    # indices, the query order, the selection's dense prefix, bf16 output; and
    # its fp32 twin
    pfx = torch.empty(order.shape, device=dev, dtype=torch.int32)
    idx_h = kernels.select(q, k, qc, off, post, cfg["b"], cfg["k"], sorted=False,
                           index_dtype=torch.int32, row_order=order, row_prefix=pfx)
    out_h = kernels.sparse_attention(q, k, v, idx_h, None, True, row_order=order, row_prefix=pfx)
    out_h32 = torch.empty_like(out)
    kernels.sparse_attention(q, k, v, idx_h, None, True, out=out_h32, row_order=order, row_prefix=pfx)
    torch.cuda.synchronize()
    print(f"{request.param}: GPU pipeline done", flush=True)
    return dict(cfg=cfg, q=q, k=k, v=v, router=router, qc=qc, kc=kc, off=off, post=post,
                idx_s=idx_s, idx_u=idx_u, idx_s2=idx_s2, idx_u2=idx_u2, idx_ub=idx_ub, st_u=st_u,
                st_ub=st_ub, stats=st, out=out,
                order=order, out_ord=out_ord, pfx=pfx, idx_h=idx_h, out_h=out_h, out_h32=out_h32)


def test_long_row_order_changes_nothing(lc):
    """Processing rows grouped by code gives bit-identical outputs; the order is
    a permutation of the positions of every (batch, kv head)."""
    order = lc["order"][0].to(torch.int64)
    n = lc["cfg"]["n"]
    assert torch.equal(order.sort(-1).values, torch.arange(n, device=order.device).expand_as(order))
    first = lc["qc"][0].min(-1).values.gather(1, order)  # smallest code along the order
    assert bool((first[:, 1:] >= first[:, :-1]).all()), "order groups rows by ascending code"
    assert torch.equal(lc["out"], lc["out_ord"])


def test_long_select_light_heavy_equals_block_path(lc):
    """Index order through the wave-per-row pass plus the listed heavy rows gives
    the same indices and stats as one block per row."""
    assert torch.equal(lc["idx_u"], lc["idx_ub"])
    assert torch.equal(lc["st_u"], lc["st_ub"])
    assert torch.equal(lc["st_u"], lc["stats"])  # sorted order counts the same


def test_long_select_deterministic(lc):
    assert torch.equal(lc["idx_u"], lc["idx_u2"]), "unsorted selection differs between runs"
    assert torch.equal(lc["idx_s"], lc["idx_s2"]), "sorted selection differs between runs"


def _sample_rows(n, extra, seed=0, count=48):
    rng = np.random.default_rng(seed)
    rows = set(rng.choice(n, count, replace=False).tolist()) | {0, 1, n - 1} | set(extra)
    return np.array(sorted(rows), dtype=np.int64)


def test_long_stage_a_codes(lc, orc):
    cfg, r = lc["cfg"], lc["router"]
    n, g = cfg["n"], cfg["h_q"] // cfg["h_kv"]
    rows = _sample_rows(n, [], seed=1, count=256)
    qf, kf = orc.to_f32(lc["q"][0][rows]), orc.to_f32(lc["k"][0][rows])
    chat = orc.normalize(orc.to_f32(r.codebook))
    qcs = orc.code_topk(orc.route_vectors(qf, orc.to_f32(r.W_qr.weight), g), chat, cfg["a"])
    kcs = orc.code_topk(orc.route_vectors(kf, orc.to_f32(r.W_kr.weight), 1), chat, cfg["b"])
    np.testing.assert_array_equal(lc["qc"][0][:, rows].cpu().numpy(), qcs)
    np.testing.assert_array_equal(lc["kc"][0][:, rows].cpu().numpy(), kcs)


def test_long_stage_b_index(lc, orc):
    off, post = orc.build_index(lc["kc"][0].cpu().numpy(), lc["cfg"]["n_c"])
    np.testing.assert_array_equal(lc["off"][0].cpu().numpy(), off)
    np.testing.assert_array_equal(lc["post"][0].cpu().numpy(), post)


@pytest.mark.parametrize("sorted_", [True, False])
def test_long_stage_c_rows_vs_oracle(lc, orc, sorted_):
    cfg = lc["cfg"]
    n = cfg["n"]
    cand = lc["stats"][0, :, :, 0].cpu().numpy()           # [h, n]
    heavy = np.argsort(-cand.max(0))[:16].tolist()          # rows with the most candidates
    rows = _sample_rows(n, heavy, seed=2)
    idx = (lc["idx_s"] if sorted_ else lc["idx_u"])[0].cpu().numpy()
    ref, ncand, nraw = orc.select(orc.to_f32(lc["q"][0]), orc.to_f32(lc["k"][0]),
                                  lc["qc"][0].cpu().numpy(), lc["off"][0].cpu().numpy(),
                                  lc["post"][0].cpu().numpy(), cfg["b"], cfg["k"],
                                  orc.MASK_CAUSAL, rows=rows, with_stats=True, sorted=sorted_)
    assert cand.max() > 2 * cfg["k"], "workload should contain rows needing several rescoring batches"
    for t, i in enumerate(rows):
        np.testing.assert_array_equal(idx[i], ref[t], err_msg=f"row {i} (sorted={sorted_})")
    st = lc["stats"][0].cpu().numpy()
    np.testing.assert_array_equal(st[:, rows, 0].T, ncand)
    np.testing.assert_array_equal(st[:, rows, 1].T, nraw)


def test_long_stage_c_properties(lc):
    """Whole-output invariants: same set in both orders, candidates causal and
    distinct, filler ascending, bounds."""
    cfg = lc["cfg"]
    n, k = cfg["n"], cfg["k"]
    idx_s = lc["idx_s"][0]
    idx_u = lc["idx_u"][0]
    assert int(idx_s.min()) >= 0 and int(idx_s.max()) < n
    assert torch.equal(idx_s.sort(-1).values, idx_u.sort(-1).values)
    ncand = lc["stats"][0, :, :, 0].T.to(torch.int64)           # [n, h]
    sel = torch.minimum(ncand, torch.tensor(k))
    pos = torch.arange(k, device=idx_s.device)
    is_cand = pos[None, None, :] < sel[..., None]
    i = torch.arange(n, device=idx_s.device)[:, None, None]
    assert bool((idx_s <= i)[is_cand].all()), "selected candidates must be causal"
    srt = idx_s.sort(-1).values
    assert bool((srt[..., 1:] != srt[..., :-1]).all()), "indices within a row must be distinct"
    filler = torch.where(is_cand, torch.full_like(idx_u, -1), idx_u)
    d = filler[..., 1:] - filler[..., :-1]
    valid = ~is_cand[..., 1:]
    assert bool((d[valid] > 0).all()), "filler must ascend"


def test_long_stage_d_rows_vs_oracle(lc, orc):
    n = lc["cfg"]["n"]
    rows = _sample_rows(n, [], seed=3, count=64)
    idx = lc["idx_u"][0].cpu().numpy()[rows]
    ref = orc.sparse_attention(orc.to_f32(lc["q"][0]), orc.to_f32(lc["k"][0]),
                               orc.to_f32(lc["v"][0]), idx, causal=True, rows=rows)
    got = lc["out"][0].cpu().numpy()[rows]
    np.testing.assert_allclose(got, ref, rtol=1e-3, atol=1e-3)


def test_long_headline_call_selection(lc):
    """The headline selection (int32, query order, prefix written) lists the
    index-order selection's indices, and each row's X names a key prefix
    [0, X) that its indices hold exactly once."""
    assert lc["idx_h"].dtype == torch.int32
    assert torch.equal(lc["idx_h"].to(torch.int64), lc["idx_u"])
    k = lc["cfg"]["k"]
    pfx = lc["pfx"][0].to(torch.int64)                       # [h, n]
    assert int(pfx.min()) >= 0 and int(pfx.max()) <= k
    assert int((pfx > 0).sum()) > 0, "clustered rows with filler have a dense prefix"
    n = lc["cfg"]["n"]
    rows = torch.from_numpy(_sample_rows(n, [], seed=4, count=512)).to(pfx.device)
    idx = lc["idx_u"][0][rows]                                 # [r, h, k]
    x = pfx[:, rows].T                                         # [r, h]
    in_pfx = idx < x[..., None]
    assert torch.equal(in_pfx.sum(-1), x), "each key of [0, X) appears exactly once"


def test_long_headline_call_outputs(lc, orc):
    """Stage (d) as timed: the bf16 output is the fp32 twin rounded once; the
    twin equals the no-prefix path within 1e-5 (the dense-prefix pass sums the
    same terms in another order) and the float64 oracle on sampled rows within
    1e-3."""
    out_h, out_h32, out = lc["out_h"], lc["out_h32"], lc["out"]
    assert out_h.dtype == torch.bfloat16
    diff = (out_h.float() - out_h32).abs()
    assert bool((diff <= out_h32.abs() * 2.0 ** -8 + 1e-30).all()), "bf16 output is the fp32 result rounded"
    torch.testing.assert_close(out_h32, out, rtol=1e-5, atol=1e-5)
    n = lc["cfg"]["n"]
    rows = _sample_rows(n, [], seed=5, count=64)
    idx = lc["idx_u"][0].cpu().numpy()[rows]
    ref = orc.sparse_attention(orc.to_f32(lc["q"][0]), orc.to_f32(lc["k"][0]),
                               orc.to_f32(lc["v"][0]), idx, causal=True, rows=rows)
    np.testing.assert_allclose(out_h32[0].cpu().numpy()[rows], ref, rtol=1e-3, atol=1e-3)


def test_long_routed_backward(lc):
    """The backward as training runs it (bench.py's call: bucket mode with the
    forward's row stats, query order and dense prefix) equals the plain
    backward within 2e-5 of max|ref| per tensor, and its dq equals the float64
    oracle on sampled rows at or above top_k (whose filler keys all precede
    them, so the causal mask drops nothing there)."""
    from ssa_amd import kernels

    cfg = lc["cfg"]
    q, k, v, order, pfx, idx = lc["q"], lc["k"], lc["v"], lc["order"], lc["pfx"], lc["idx_h"]
    print(f"{cfg['n']}: routed backward", flush=True)
    stats = kernels.row_stats_buffer(q, cfg["h_kv"])
    out32 = torch.empty(q.shape, device=q.device, dtype=torch.float32)
    kernels.sparse_attention(q, k, v, idx, None, True, out=out32, row_order=order, row_prefix=pfx,
                             row_stats=stats)
    gen = torch.Generator(device=q.device).manual_seed(7)
    dout = torch.randn(q.shape, generator=gen, device=q.device).to(q.dtype)
    routing = kernels.Routing(lc["qc"], lc["kc"], lc["off"], lc["post"], True)
    routed = kernels.sparse_attention_backward(q, k, v, idx, out32, dout, None, True, row_order=order,
                                               row_prefix=pfx, routing=routing, row_stats=stats)
    plain = kernels.sparse_attention_backward(q, k, v, idx, out32, dout, None, True)
    torch.cuda.synchronize()
    for name, got, ref in zip(("dq", "dk", "dv"), routed, plain):
        scale = float(ref.abs().max())
        err = float((got - ref).abs().max())
        assert err <= 2e-5 * scale, f"{name}: {err:.3e} > 2e-5 * {scale:.3e}"
    del plain
    # dq of sampled rows by float64 autograd through the reference's gather /
    # softmax / weighted sum (ssa/attention.py:64-113) on the CPU
    n, kk, h_kv, d = cfg["n"], cfg["k"], cfg["h_kv"], cfg["d"]
    g = cfg["h_q"] // h_kv
    rows = torch.from_numpy(_sample_rows(n - kk, [], seed=6, count=24) + kk)
    ids = idx[0].cpu().long()[rows]                                   # [r, h_kv, kk]
    qs = q[0].cpu().double()[rows].requires_grad_(True)               # [r, h_q, d]
    kd, vd = k[0].cpu().double(), v[0].cpu().double()
    hh = torch.arange(h_kv)[None, :, None]
    kg, vg = kd[ids, hh], vd[ids, hh]                                 # [r, h_kv, kk, d]
    logit = torch.matmul(qs.view(-1, h_kv, g, d), kg.transpose(-1, -2)) / d ** 0.5
    o = torch.matmul(torch.softmax(logit, -1), vg).reshape(-1, cfg["h_q"], d)
    (o * dout[0].cpu().double()[rows]).sum().backward()
    ref = qs.grad
    got = routed[0][0].cpu().double()[rows]
    err = float((got - ref).abs().max())
    assert err <= 2e-5 * float(ref.abs().max()), f"dq vs float64 autograd: {err:.3e}"
