"""Stage-by-stage parity of the HIP kernels against the CPU oracle.

Selections (codes, index, candidates) must be bit-identical; attention outputs
match within 1e-5 (fp32) / 1e-3 (bf16 inputs, fp32 output).
"""

import numpy as np
import pytest
import torch

from tests.helpers import clustered_qk, f32, randn, router_params

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("h_in,group,d,d_s", [(8, 4, 128, 32), (6, 3, 64, 16), (2, 1, 64, 8),
                                              (16, 8, 128, 32), (8, 1, 128, 32)])
def test_route_vectors_bit_exact(dev, orc, dtype, h_in, group, d, d_s):
    from ssa_amd import kernels

    _say(f"route_vectors dtype={dtype} h_in={h_in} g={group} d={d} d_s={d_s}")
    n = 300
    x = randn((2, n, h_in, d), 1, dtype)
    w = torch.nn.init.uniform_(torch.empty(d_s, d), -0.2, 0.2)
    got = kernels.route_vectors(x.to(dev), w.to(dev), group).cpu().numpy()
    for b in range(2):
        ref = orc.route_vectors(f32(x[b]), f32(w), group)
        np.testing.assert_array_equal(got[b], ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,batch,h_in,group,d,d_s", [
    (1, 1, 32, 4, 128, 32),     # a decoding step: the one-wave-per-row kernel
    (3, 2, 6, 3, 64, 16),
    (17, 1, 8, 1, 128, 48),
    (500, 2, 4, 2, 64, 48),     # route_dim > 32: the general LDS-tiled kernel
    (300, 1, 2, 1, 128, 64),
    (100, 2, 3, 1, 128, 32),    # the keys' kernel (two waves per 64 rows), a partial tile
])
def test_route_vectors_small_and_wide_bit_exact(dev, orc, dtype, n, batch, h_in, group, d, d_s):
    """Few rows (the lane-per-coordinate kernel of decoding steps) and route
    dims above 32 (the general kernel) against the oracle's chains."""
    from ssa_amd import kernels

    _say(f"route_vectors small/wide n={n} B={batch} h_in={h_in} g={group} d={d} d_s={d_s}")
    x = randn((batch, n, h_in, d), 5, dtype)
    w = torch.nn.init.uniform_(torch.empty(d_s, d), -0.2, 0.2)
    got = kernels.route_vectors(x.to(dev), w.to(dev), group).cpu().numpy()
    for b in range(batch):
        np.testing.assert_array_equal(got[b], orc.route_vectors(f32(x[b]), f32(w), group))


@pytest.mark.parametrize("top,n_c,d_s,rows,h", [(16, 4096, 32, 1, 8), (4, 4096, 32, 3, 2),
                                                (32, 8192, 32, 2, 2), (8, 300, 16, 5, 3)])
def test_code_topk_few_rows_bit_exact(dev, orc, top, n_c, d_s, rows, h):
    """A handful of rows (decoding) take the exhaustive one-wave-per-row kernel."""
    from ssa_amd import kernels

    _say(f"code_topk few rows top={top} n_c={n_c} rows={rows} h={h}")
    xhat = torch.from_numpy(orc.normalize(f32(randn((1, h, rows, d_s), 6))))
    chat = torch.from_numpy(orc.normalize(f32(randn((h, n_c, d_s), 7))))
    got = kernels.code_topk(xhat.to(dev), chat.to(dev), top).cpu().numpy()
    np.testing.assert_array_equal(got[0], orc.code_topk(xhat[0].numpy(), chat.numpy(), top))


def test_normalize_rows_bit_exact(dev, orc):
    from ssa_amd import kernels

    x = randn((4, 512, 32), 2)
    x[0, 0] = 0.0  # eps clamp: 0 / 1e-12 = 0
    got = kernels.normalize_rows(x.to(dev)).cpu().numpy()
    np.testing.assert_array_equal(got, orc.normalize(f32(x)))
    # rows at an address 4 bytes past 16-byte alignment (the per-element path)
    buf = torch.empty(x.numel() + 1, device=dev)
    xm = buf[1:].view(x.shape)
    xm.copy_(x.to(dev))
    np.testing.assert_array_equal(kernels.normalize_rows(xm).cpu().numpy(), orc.normalize(f32(x)))


@pytest.mark.parametrize("top,temperature,n_c,d_s", [(16, 1.0, 512, 32), (4, 1.0, 4096, 32),
                                                     (8, 0.7, 130, 16), (64, 1.0, 1000, 8)])
def test_code_topk_bit_exact(dev, orc, top, temperature, n_c, d_s):
    from ssa_amd import kernels

    _say(f"code_topk top={top} T={temperature} n_c={n_c} d_s={d_s}")
    B, h, rows = 2, 3, 200
    xhat = torch.from_numpy(orc.normalize(f32(randn((B, h, rows, d_s), 3))))
    chat = torch.from_numpy(orc.normalize(f32(randn((h, n_c, d_s), 4))))
    got = kernels.code_topk(xhat.to(dev), chat.to(dev), top, temperature).cpu().numpy()
    for b in range(B):
        ref = orc.code_topk(xhat[b].numpy(), chat.numpy(), top, temperature)
        np.testing.assert_array_equal(got[b], ref)


def test_code_topk_ties_lowest_index(dev, orc):
    """Duplicated codebook rows tie exactly; the lower code id must come first."""
    from ssa_amd import kernels

    d_s, n_c = 16, 96
    base = orc.normalize(f32(randn((1, 32, d_s), 5)))
    chat = np.concatenate([base, base, base], axis=1)  # codes c, c+32, c+64 identical
    xhat = orc.normalize(f32(randn((1, 1, 50, d_s), 6)))
    got = kernels.code_topk(torch.from_numpy(xhat).to(dev), torch.from_numpy(chat).to(dev), 9).cpu().numpy()
    ref = orc.code_topk(xhat[0], chat, 9)
    np.testing.assert_array_equal(got[0], ref)
    # every triple appears as c, c+32, c+64 in that order
    assert (ref[0, :, 0] % 32 == ref[0, :, 1] % 32).all() and (ref[0, :, 0] < ref[0, :, 1]).all()


@pytest.mark.parametrize("n,h_kv,b,n_c", [(700, 2, 4, 64), (5000, 3, 4, 4096), (3000, 1, 2, 7)])
def test_build_index_bit_exact(dev, orc, n, h_kv, b, n_c):
    from ssa_amd import kernels

    _say(f"build_index n={n} h_kv={h_kv} b={b} n_c={n_c}")
    g = torch.Generator().manual_seed(7)
    B = 2
    # distinct codes per key, skewed towards low code ids (heavy buckets)
    scores = torch.rand(B, h_kv, n, n_c, generator=g) ** 4 + torch.linspace(1, 0, n_c)
    kc = scores.topk(b, dim=-1).indices.to(torch.int32)
    off, post = kernels.build_index(kc.to(dev), n_c)
    off, post = off.cpu().numpy(), post.cpu().numpy()
    for bb in range(B):
        roff, rpost = orc.build_index(kc[bb].numpy(), n_c)
        np.testing.assert_array_equal(off[bb], roff)
        np.testing.assert_array_equal(post[bb], rpost)


@pytest.mark.parametrize("n,h_kv,a,n_c", [(5000, 2, 16, 256), (70000, 1, 3, 4096), (1, 2, 1, 8)])
def test_query_order_is_stable_sort_by_smallest_code(dev, n, h_kv, a, n_c):
    """The processing order equals numpy's stable argsort of each row's
    smallest code."""
    from ssa_amd import kernels

    _say(f"query_order n={n} h_kv={h_kv} a={a} n_c={n_c}")
    g = torch.Generator().manual_seed(8)
    B = 2
    qc = (torch.rand(B, h_kv, n, a, generator=g) ** 3 * n_c).to(torch.int32)  # skewed buckets
    got = kernels.query_order(qc.to(dev), n_c).cpu().numpy()
    want = np.argsort(qc.numpy().min(-1), axis=-1, kind="stable").astype(np.int32)
    np.testing.assert_array_equal(got, want)


def _route_inputs(n, h_q, h_kv, d, d_s, n_c, seed, dtype, clustered):
    if clustered:
        q, k = clustered_qk(n, h_q, h_kv, d, 8, 0.3, seed, dtype)
    else:
        q, k = randn((n, h_q, d), seed, dtype), randn((n, h_kv, d), seed + 1, dtype)
    w_qr, w_kr, cb = router_params(d, d_s, h_kv, n_c, seed + 2)
    return q, k, w_qr, w_kr, cb


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", ["causal", "none", "dense"])
@pytest.mark.parametrize("clustered", [False, True])
@pytest.mark.parametrize("sorted_", [True, False])
def test_router_pipeline_bit_exact(dev, orc, dtype, mode, clustered, sorted_):
    """Stages (a)-(c) through CodebookRouter vs the oracle, with per-row stats."""
    from ssa_amd import CodebookRouter, build_causal_mask

    _say(f"router pipeline dtype={dtype} mode={mode} clustered={clustered} sorted={sorted_}")
    n, h_q, h_kv, d, d_s, n_c, a, b, k = 777, 8, 2, 128, 32, 128, 16, 4, 64
    q, kk, w_qr, w_kr, cb = _route_inputs(n, h_q, h_kv, d, d_s, n_c, 11, dtype, clustered)
    r = CodebookRouter(head_dim=d, route_dim=d_s, num_kv_heads=h_kv, num_codebook=n_c,
                       codes_per_key=b, codes_per_query=a, top_k=k)
    with torch.no_grad():
        r.W_qr.weight.copy_(w_qr)
        r.W_kr.weight.copy_(w_kr)
        r.codebook.copy_(cb)
    r = r.to(dev)
    if mode == "causal":
        cm, omode, omask = build_causal_mask(n, device=dev), orc.MASK_CAUSAL, None
    elif mode == "none":
        cm, omode, omask = None, orc.MASK_NONE, None
    else:
        gm = torch.Generator().manual_seed(3)
        m = (torch.rand(n, n, generator=gm) < 0.6) | torch.eye(n, dtype=torch.bool)
        cm, omode, omask = m.to(dev), orc.MASK_DENSE, m.numpy().astype(np.uint8)
    res = r.route(q.to(dev), kk.to(dev), causal_mask=cm, with_stats=True, sorted=sorted_)
    (ref, ncand, nraw), ex = orc.router_forward(f32(q), f32(kk), f32(w_qr), f32(w_kr), f32(cb),
                                               a, b, k, omode, omask, with_stats=True,
                                               sorted=sorted_)
    np.testing.assert_array_equal(res.q_codes[0].cpu().numpy(), ex["q_codes"])
    np.testing.assert_array_equal(res.k_codes[0].cpu().numpy(), ex["k_codes"])
    np.testing.assert_array_equal(res.offsets[0].cpu().numpy(), ex["offsets"])
    np.testing.assert_array_equal(res.postings[0].cpu().numpy(), ex["postings"])
    np.testing.assert_array_equal(res.indices[0].cpu().numpy(), ref)
    st = res.stats[0].cpu().numpy()  # [h, n, 2]
    np.testing.assert_array_equal(st[..., 0].T, ncand)
    np.testing.assert_array_equal(st[..., 1].T, nraw)


@pytest.mark.parametrize("top_k", [1, 600, 1000, 4096])
@pytest.mark.parametrize("sorted_", [True, False])
def test_select_k_edges(dev, orc, top_k, sorted_):
    """k > n pads zeros; k = n lists every index; k = 1."""
    from ssa_amd import CodebookRouter

    n = 1000 if top_k != 4096 else 2500
    _say(f"select k edges n={n} top_k={top_k} sorted={sorted_}")
    q, kk, w_qr, w_kr, cb = _route_inputs(n, 4, 1, 64, 16, 64, 21, torch.float32, False)
    r = CodebookRouter(head_dim=64, route_dim=16, num_kv_heads=1, num_codebook=64,
                       codes_per_key=4, codes_per_query=8, top_k=top_k)
    with torch.no_grad():
        r.W_qr.weight.copy_(w_qr)
        r.W_kr.weight.copy_(w_kr)
        r.codebook.copy_(cb)
    got = r.to(dev)(q.to(dev), kk.to(dev), causal_mask=True, sorted=sorted_).cpu().numpy()
    ref, _ = orc.router_forward(f32(q), f32(kk), f32(w_qr), f32(w_kr), f32(cb), 8, 4, top_k,
                                sorted=sorted_)
    np.testing.assert_array_equal(got, ref)
    if top_k >= n:
        assert (np.sort(got[:, :, :n], axis=-1) == np.arange(n)).all()


@pytest.mark.parametrize("dtype,d,g,tol", [(torch.float32, 64, 4, 1e-5), (torch.float32, 128, 3, 1e-5),
                                           (torch.bfloat16, 128, 4, 1e-3), (torch.bfloat16, 64, 8, 1e-3),
                                           (torch.bfloat16, 256, 16, 1e-3), (torch.float32, 256, 1, 1e-5),
                                           # head dims below / between the padded widths
                                           (torch.bfloat16, 8, 1, 1e-3), (torch.float32, 16, 2, 1e-5),
                                           (torch.bfloat16, 32, 4, 1e-3), (torch.bfloat16, 96, 2, 1e-3),
                                           (torch.bfloat16, 136, 4, 1e-3), (torch.float32, 200, 2, 1e-5)])
@pytest.mark.parametrize("causal", [False, True])
def test_sparse_attention_vs_oracle(dev, orc, dtype, d, g, tol, causal):
    from ssa_amd import kernels

    _say(f"sparse_attention dtype={dtype} d={d} g={g} causal={causal}")
    n, h_kv, top_k, B = 300, 2, 100, 2
    h_q = h_kv * g
    q = randn((B, n, h_q, d), 31, dtype)
    k = randn((B, n, h_kv, d), 32, dtype)
    v = randn((B, n, h_kv, d), 33, dtype)
    gi = torch.Generator().manual_seed(34)
    idx = torch.randint(0, n, (B, n, h_kv, top_k), generator=gi)
    idx[..., :3] = 0  # duplicates count twice
    out = torch.empty(B, n, h_q, d, device=dev, dtype=torch.float32)
    kernels.sparse_attention(q.to(dev), k.to(dev), v.to(dev), idx.to(dev), None, causal, out=out)
    got = out.cpu().numpy()
    for b in range(B):
        ref = orc.sparse_attention(f32(q[b]), f32(k[b]), f32(v[b]), idx[b].numpy(), causal=causal)
        np.testing.assert_allclose(got[b], ref, rtol=tol, atol=tol)


@pytest.mark.parametrize("top_k,causal,g", [(512, True, 4), (2048, False, 8), (256, True, 2)])
def test_sparse_attention_few_rows_split(dev, orc, top_k, causal, g):
    """Calls of at most 512 rows (decoding steps) split each row's chunks over
    four waves and combine their states: against the oracle (bf16 inputs, fp32
    output, 1e-3) and against the same rows of a large call (one wave per row)
    within 1e-5; with duplicated and out-of-range slots."""
    from ssa_amd import kernels

    _say(f"attention few rows split top_k={top_k} causal={causal} g={g}")
    n, h_kv, d, m = 3000, 2, 128, 3
    q = randn((1, n, h_kv * g, d), 121, torch.bfloat16).to(dev)
    k = randn((1, n, h_kv, d), 122, torch.bfloat16).to(dev)
    v = randn((1, n, h_kv, d), 123, torch.bfloat16).to(dev)
    gi = torch.Generator().manual_seed(124)
    idx = torch.randint(0, n, (1, n, h_kv, top_k), generator=gi)
    idx[0, -2, 0, 7] = idx[0, -2, 0, 3]                # a duplicate counts twice
    idx = idx.to(torch.int32).to(dev)
    rows = slice(n - m, n)
    few = torch.empty((1, m, h_kv * g, d), device=dev, dtype=torch.float32)
    kernels.sparse_attention(q[:, rows], k, v, idx[:, rows], None, causal, out=few, q_pos0=n - m)
    big = torch.empty((1, n, h_kv * g, d), device=dev, dtype=torch.float32)
    kernels.sparse_attention(q, k, v, idx, None, causal, out=big)
    torch.testing.assert_close(few, big[:, rows], rtol=1e-5, atol=1e-5)
    ref = orc.sparse_attention(f32(q[0]), f32(k[0]), f32(v[0]), idx[0].cpu().numpy()[rows],
                               causal=causal, rows=np.arange(n - m, n))
    np.testing.assert_allclose(few[0].cpu().numpy(), ref, rtol=1e-3, atol=1e-3)
    flag = torch.zeros(1, device=dev, dtype=torch.int32)
    bad = idx[:, rows].clone()
    bad[0, 0, 1, 5] = n + 3
    kernels.sparse_attention(q[:, rows], k, v, bad, None, causal, out=few, q_pos0=n - m, error_flag=flag)
    assert int(flag.item()) == 1


def test_sparse_attention_k_equals_n_is_causal_dense(dev, orc):
    """Config 2 shape: fp32, n=2048, GQA 8/2, d=64, k=n, causal -> dense causal within 1e-5."""
    from ssa_amd import dense_attention, sparse_exact_attention

    n, h_q, h_kv, d = 2048, 8, 2, 64
    q, k, v = randn((n, h_q, d), 41), randn((n, h_kv, d), 42), randn((n, h_kv, d), 43)
    idx = torch.arange(n).view(1, 1, n).expand(n, h_kv, n).contiguous()
    got = sparse_exact_attention(q.to(dev), k.to(dev), v.to(dev), idx.to(dev), causal=True).cpu().numpy()
    ref = orc.dense_attention(f32(q), f32(k), f32(v), causal=True)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)
    mask = torch.ones(n, n, dtype=torch.bool).tril()
    td = dense_attention(q.to(dev), k.to(dev), v.to(dev), causal_mask=mask.to(dev)).cpu().numpy()
    np.testing.assert_allclose(td, ref, rtol=1e-4, atol=1e-4)


def test_sparse_attention_bad_index_raises(dev):
    from ssa_amd import sparse_exact_attention

    n = 64
    q, k, v = randn((n, 4, 64), 1), randn((n, 2, 64), 2), randn((n, 2, 64), 3)
    idx = torch.zeros(n, 2, 8, dtype=torch.int64)
    idx[5, 1, 3] = n
    with pytest.raises(IndexError):
        sparse_exact_attention(q.to(dev), k.to(dev), v.to(dev), idx.to(dev))


@pytest.mark.parametrize("top,n_c,d_s", [(4, 4096, 32), (16, 4096, 32), (32, 1000, 32),
                                         (32, 8192, 32), (24, 2050, 32), (17, 300, 20),
                                         (16, 777, 16), (8, 64, 8), (3, 4099, 32)])
def test_code_topk_screen_equals_exhaustive_and_oracle(dev, orc, top, n_c, d_s):
    """The matrix-core screen + exact rescoring returns the same codes as exhaustive
    fp32 scoring and as the oracle, including ragged N_c."""
    from ssa_amd import kernels

    _say(f"code_topk screen top={top} n_c={n_c} d_s={d_s}")
    B, h, rows = 1, 2, 3000
    xhat = torch.from_numpy(orc.normalize(f32(randn((B, h, rows, d_s), 12))))
    chat = torch.from_numpy(orc.normalize(f32(randn((h, n_c, d_s), 13))))
    got = kernels.code_topk(xhat.to(dev), chat.to(dev), top).cpu().numpy()
    exh = kernels.code_topk(xhat.to(dev), chat.to(dev), top, exhaustive=True).cpu().numpy()
    np.testing.assert_array_equal(got, exh)
    np.testing.assert_array_equal(got[0], orc.code_topk(xhat[0].numpy(), chat.numpy(), top))


def test_code_topk_screen_overflow_falls_back(dev, orc):
    """300 identical codebook rows tie exactly for every query: the screen keeps more
    than its capacity, flags the rows and the exact kernel settles them."""
    from ssa_amd import kernels

    d_s, n_c, top = 32, 1024, 16
    chat = orc.normalize(f32(randn((1, n_c, d_s), 14)))
    chat[0, 100:400] = chat[0, 100]
    xhat = orc.normalize(f32(randn((1, 1, 500, d_s), 15)))
    xhat[0, 0, :250] = chat[0, 100]          # rows pointing at the tied block
    xhat[0, 0, 250] = 0.0                    # a zero routing vector: every score ties at 0
    got = kernels.code_topk(torch.from_numpy(xhat).to(dev), torch.from_numpy(chat).to(dev), top)
    ref = orc.code_topk(xhat[0], chat, top)
    np.testing.assert_array_equal(got.cpu().numpy()[0], ref)
    assert (ref[0, 0] == np.arange(100, 116)).all()
    assert (ref[0, 250] == np.arange(16)).all()


@pytest.mark.parametrize("top,n_c,temperature", [(4, 1024, 1.0), (8, 2000, 0.7), (16, 1024, 1.0),
                                                 (16, 20000, 1.0), (32, 1500, 0.7)])
def test_code_topk_flagged_rows_batched(dev, orc, top, n_c, temperature):
    """Rows the screen cannot settle (exact ties over a block of 300 equal codes in
    head 1 only) are recomputed one wave per row; every (batch, head, row) lands
    in its own output row and matches the oracle."""
    from ssa_amd import kernels

    _say(f"code_topk flagged rows top={top} n_c={n_c} temperature={temperature}")
    B, h, rows, d_s = 2, 2, 700, 32
    chat = orc.normalize(f32(randn((h, n_c, d_s), 16)))
    chat[1, 100:400] = chat[1, 100]
    xhat = orc.normalize(f32(randn((B, h, rows, d_s), 17)))
    xhat[:, 1, 50:120] = chat[1, 100]         # tied rows in head 1 of both batches
    xhat[1, 1, 600] = 0.0                     # every score ties at 0
    got = kernels.code_topk(torch.from_numpy(xhat).to(dev), torch.from_numpy(chat).to(dev), top,
                            temperature).cpu().numpy()
    for bb in range(B):
        ref = orc.code_topk(xhat[bb], chat, top, temperature)
        np.testing.assert_array_equal(got[bb], ref)
    assert (got[:, 1, 50] == np.arange(100, 100 + top)).all()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", ["causal", "none"])
@pytest.mark.parametrize("n_c,a", [(2048, 4), (8192, 8)])
def test_router_long_rows_bit_exact(dev, orc, dtype, mode, n_c, a):
    """n = 70000 keys: a row's key bitmap spans more than one 65536-key chunk,
    so the index-order pass marks and reads its candidates back in two chunks
    (at N_c = 8192 the buckets hold about 17 postings, and a half-wave marks
    each); stats and indices must equal the oracle's."""
    from ssa_amd import CodebookRouter

    _say(f"router long rows dtype={dtype} mode={mode} n_c={n_c} a={a}")
    n, h_q, h_kv, d, d_s, b, k = 70000, 2, 1, 64, 16, 2, 128
    q, kk, w_qr, w_kr, cb = _route_inputs(n, h_q, h_kv, d, d_s, n_c, 23, dtype, False)
    r = CodebookRouter(head_dim=d, route_dim=d_s, num_kv_heads=h_kv, num_codebook=n_c,
                       codes_per_key=b, codes_per_query=a, top_k=k)
    with torch.no_grad():
        r.W_qr.weight.copy_(w_qr)
        r.W_kr.weight.copy_(w_kr)
        r.codebook.copy_(cb)
    r = r.to(dev)
    causal = mode == "causal"
    res = r.route(q.to(dev), kk.to(dev), causal_mask=True if causal else None, with_stats=True,
                  sorted=False)
    (ref, ncand, nraw), _ = orc.router_forward(f32(q), f32(kk), f32(w_qr), f32(w_kr), f32(cb),
                                               a, b, k, orc.MASK_CAUSAL if causal else orc.MASK_NONE,
                                               None, with_stats=True, sorted=False)
    np.testing.assert_array_equal(res.indices[0].cpu().numpy(), ref)
    st = res.stats[0].cpu().numpy()
    np.testing.assert_array_equal(st[..., 0].T, ncand)
    np.testing.assert_array_equal(st[..., 1].T, nraw)
    assert (ncand > k).any()
