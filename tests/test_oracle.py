"""Pins the CPU oracle (oracle/ssa_oracle.c) before it is trusted as the checker.

Each oracle function is checked against something independent of its own
formula: closed forms, the reference's set definitions written as plain loops,
float64 restatements, torch's SDPA, and hand-built cases whose answer is known.
"""

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import f32, randn


def _ulp_close(a, b, ulps=4):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    tol = ulps * np.spacing(np.maximum(np.abs(a), np.abs(b)).astype(np.float32)).astype(np.float64)
    assert (np.abs(a - b) <= tol + 1e-30).all(), float(np.abs(a - b).max())


# ------------------------------------------------------------------ normalize

def test_normalize_closed_forms():
    x = np.array([[3.0, 4.0], [0.0, 0.0], [1e-20, 0.0], [-2.0, 0.0]], np.float32)
    out = oracle.normalize(x)
    np.testing.assert_array_equal(out[0], np.float32([0.6, 0.8]))
    np.testing.assert_array_equal(out[1], [0.0, 0.0])            # 0 / max(0, eps)
    assert out[2][0] == np.float32(np.float32(1e-20) / np.float32(1e-12))  # eps clamp active
    np.testing.assert_array_equal(out[3], [-1.0, 0.0])


def test_normalize_vs_float64():
    x = f32(randn((500, 32), 1))
    ref = x.astype(np.float64) / np.linalg.norm(x.astype(np.float64), axis=-1, keepdims=True)
    _ulp_close(oracle.normalize(x), ref, ulps=4)


# ------------------------------------------------------------- route vectors

@pytest.mark.parametrize("h_in,group", [(8, 4), (6, 3), (2, 1)])
def test_route_vectors_vs_float64(h_in, group):
    x = f32(randn((64, h_in, 32), 2))
    w = f32(randn((16, 32), 3)) * 0.1
    got = oracle.route_vectors(x, w, group)
    ref = oracle.np_route_vectors64(x, w, group)
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=2e-7)


def test_route_vectors_head_grouping_exact():
    """Integer inputs and a one-hot W make every step exact: the result is the
    normalized mean over heads h*g .. h*g+g-1 (GQA head j -> KV head j // g)."""
    rng = np.random.default_rng(4)
    n, h_in, g, d, d_s = 10, 8, 4, 16, 4
    x = rng.integers(-8, 9, (n, h_in, d)).astype(np.float32)
    w = np.zeros((d_s, d), np.float32)
    w[np.arange(d_s), [3, 0, 7, 12]] = 1.0
    got = oracle.route_vectors(x, w, g)
    sel = x[:, :, [3, 0, 7, 12]].reshape(n, h_in // g, g, d_s).mean(2)  # exact (dyadic)
    ref = sel / np.maximum(np.sqrt((sel.astype(np.float64) ** 2).sum(-1, keepdims=True)), 1e-12)
    _ulp_close(got, np.transpose(ref, (1, 0, 2)), ulps=2)


# ----------------------------------------------------------------- code top-k

def test_code_topk_one_hot_codebook_is_coordinate_sort():
    """chat = identity rows => score(c) = xhat[c]; top codes = coordinates sorted desc."""
    d_s = 32
    xhat = oracle.normalize(f32(randn((1, 200, d_s), 5)))
    chat = np.eye(d_s, dtype=np.float32)[None]
    codes = oracle.code_topk(xhat, chat, 7)
    ref = np.argsort(-xhat[0], axis=-1, kind="stable")[:, :7]
    np.testing.assert_array_equal(codes[0], ref)


def test_code_topk_ties_go_to_lowest_index():
    xhat = oracle.normalize(f32(randn((1, 40, 8), 6)))
    base = oracle.normalize(f32(randn((1, 10, 8), 7)))
    chat = np.concatenate([base, base], axis=1)  # c and c+10 tie exactly
    codes, scores = oracle.code_topk(xhat, chat, 6, with_scores=True)
    for r in range(40):
        for m in range(5):
            s0, s1 = scores[0, r, m], scores[0, r, m + 1]
            assert s0 > s1 or (s0 == s1 and codes[0, r, m] < codes[0, r, m + 1])
        assert codes[0, r, 0] % 10 == codes[0, r, 1] % 10 and codes[0, r, 0] < codes[0, r, 1]


def test_code_topk_vs_float64_where_unambiguous():
    xhat = oracle.normalize(f32(randn((2, 300, 32), 8)))
    chat = oracle.normalize(f32(randn((2, 512, 32), 9)))
    got = oracle.code_topk(xhat, chat, 16)
    sc = np.einsum("hrs,hcs->hrc", xhat.astype(np.float64), chat.astype(np.float64))
    order = np.argsort(-sc, axis=-1, kind="stable")
    srt = np.take_along_axis(sc, order, -1)
    safe = (srt[..., :16] - np.concatenate([srt[..., 1:17]], -1)).min(-1) > 1e-5
    assert safe.mean() > 0.9
    np.testing.assert_array_equal(got[safe], order[..., :16][safe])


def test_code_topk_temperature_power_of_two_keeps_order():
    xhat = oracle.normalize(f32(randn((1, 100, 16), 10)))
    chat = oracle.normalize(f32(randn((1, 64, 16), 11)))
    np.testing.assert_array_equal(oracle.code_topk(xhat, chat, 8, 0.5), oracle.code_topk(xhat, chat, 8))


# ------------------------------------------------------------- inverted index

def test_build_index_vs_dict():
    rng = np.random.default_rng(12)
    h, n, b, n_c = 3, 400, 4, 37
    kc = np.stack([np.stack([rng.choice(n_c, b, replace=False) for _ in range(n)]) for _ in range(h)])
    off, post = oracle.build_index(kc, n_c)
    for hh in range(h):
        buckets = {c: [] for c in range(n_c)}
        for j in range(n):
            for c in kc[hh, j]:
                buckets[int(c)].append(j)
        flat = [j for c in range(n_c) for j in buckets[c]]
        np.testing.assert_array_equal(post[hh], flat)
        np.testing.assert_array_equal(np.diff(off[hh]), [len(buckets[c]) for c in range(n_c)])
        assert off[hh, 0] == 0 and off[hh, -1] == n * b


# ------------------------------------------------------------------- select

def _tiny_router_case(seed, n=40, h_q=4, h_kv=2, d=16, d_s=8, n_c=24, a=4, b=2):
    q = f32(randn((n, h_q, d), seed))
    k = f32(randn((n, h_kv, d), seed + 1))
    w_qr = f32(randn((d_s, d), seed + 2)) * 0.2
    w_kr = f32(randn((d_s, d), seed + 3)) * 0.2
    cb = f32(randn((h_kv, n_c, d_s), seed + 4))
    return q, k, w_qr, w_kr, cb, a, b


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("top_k", [5, 12, 40, 55])
def test_select_matches_brute_force(causal, top_k):
    q, k, w_qr, w_kr, cb, a, b = _tiny_router_case(20)
    mode = oracle.MASK_CAUSAL if causal else oracle.MASK_NONE
    (got, ncand, nraw), ex = oracle.router_forward(q, k, w_qr, w_kr, cb, a, b, top_k, mode,
                                                   with_stats=True)
    ref = oracle.brute_select(q, k, ex["q_codes"], ex["k_codes"], top_k, causal)
    np.testing.assert_array_equal(got, ref)
    mask = oracle.brute_candidate_mask(ex["q_codes"], ex["k_codes"], causal)
    np.testing.assert_array_equal(ncand, mask.sum(-1).T)
    if top_k > q.shape[0]:
        assert (got[..., q.shape[0]:] == 0).all()


def test_select_dense_tril_mask_equals_causal():
    q, k, w_qr, w_kr, cb, a, b = _tiny_router_case(30)
    n = q.shape[0]
    (c1, _, _), _ = oracle.router_forward(q, k, w_qr, w_kr, cb, a, b, 9, oracle.MASK_CAUSAL, with_stats=True)
    tril = np.tril(np.ones((n, n), np.uint8))
    (c2, _, _), _ = oracle.router_forward(q, k, w_qr, w_kr, cb, a, b, 9, oracle.MASK_DENSE, tril,
                                          with_stats=True)
    np.testing.assert_array_equal(c1, c2)


def test_select_all_codes_means_all_causal_keys():
    """a = N_c: every causal key is a candidate, so the row is the exact top-k of
    mean_g(q.k)/sqrt(d) over j <= i, then the non-causal keys in ascending order."""
    q, k, w_qr, w_kr, cb, a, b = _tiny_router_case(40, n_c=12, a=12)
    n, h_q, d = q.shape
    h_kv = k.shape[1]
    got, _ = oracle.router_forward(q, k, w_qr, w_kr, cb, a, b, 10)
    g = h_q // h_kv
    sc = np.einsum("nhgd,mhd->nhm", q.reshape(n, h_kv, g, d).astype(np.float64), k.astype(np.float64)) / g / np.sqrt(d)
    for i in range(n):
        for h in range(h_kv):
            order = sorted(range(i + 1), key=lambda j: (-sc[i, h, j], j))[:10]
            order += list(range(i + 1, n))[: 10 - len(order)]
            np.testing.assert_array_equal(got[i, h], order)


def test_select_no_candidates_is_lowest_index_filler():
    q, k, w_qr, w_kr, cb, a, b = _tiny_router_case(50)
    n = q.shape[0]
    qc = np.zeros((k.shape[1], n, a), np.int32) + np.arange(a, dtype=np.int32)        # codes 0..a-1
    kc = np.zeros((k.shape[1], n, b), np.int32) + np.arange(a, a + b, dtype=np.int32)  # disjoint
    off, post = oracle.build_index(kc, a + b)
    out, ncand, _ = oracle.select(q, k, qc, off, post, b, 7, with_stats=True)
    assert (ncand == 0).all()
    assert (out == np.arange(7)).all()


# ---------------------------------------------------------------- attention

@pytest.mark.parametrize("causal", [False, True])
def test_sparse_attention_vs_numpy64(causal):
    n, h_q, h_kv, d, kk = 50, 6, 2, 16, 12
    q, k, v = f32(randn((n, h_q, d), 60)), f32(randn((n, h_kv, d), 61)), f32(randn((n, h_kv, d), 62))
    idx = np.random.default_rng(63).integers(0, n, (n, h_kv, kk))
    idx[:, :, :2] = 0
    got = oracle.sparse_attention(q, k, v, idx, causal=causal)
    ref = oracle.np_sparse_attention64(q, k, v, idx, causal=causal)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)


def _reference_flat_gather64(q, k, v, idx, scale):
    """ssa/attention.py:64-113 as its code runs it, in float64: K and V flattened
    to [n*h_kv, d], index j of KV head h offset by h*n, then the grouped
    logits, softmax and weighted sum."""
    q, k, v = (torch.from_numpy(np.asarray(t, np.float64)) for t in (q, k, v))
    n, h_q, d = q.shape
    h_kv, kk = k.shape[1], idx.shape[-1]
    flat = torch.from_numpy(idx).reshape(-1)
    offs = (torch.arange(h_kv) * n)[None, :, None].expand(n, h_kv, kk).reshape(-1)
    kg = k.reshape(n * h_kv, d)[flat + offs].reshape(n, h_kv, kk, d)
    vg = v.reshape(n * h_kv, d)[flat + offs].reshape(n, h_kv, kk, d)
    qg = q.reshape(n, h_kv, h_q // h_kv, d)
    w = torch.softmax(torch.einsum("nhgd,nhkd->nhgk", qg, kg) / scale, dim=-1)
    return torch.einsum("nhgk,nhkd->nhgd", w, vg).reshape(n, h_q, d).numpy()


def test_flat_gather_view_is_the_reference_code_gather():
    """flat_gather_view(t)[j, h] is row j + h*n of t flattened to [n*h_kv, d], so
    the oracle fed with that layout computes what ssa/attention.py:76-113's code
    does (not its docstring's K[j, h]); h_kv = 1 leaves the rows unchanged."""
    from ssa_amd.attention import flat_gather_view

    n, h_q, h_kv, d, kk = 37, 6, 3, 8, 9
    t = torch.randn(2, n, h_kv, d, dtype=torch.float64)
    view = flat_gather_view(t)
    assert view.shape == t.shape and view.data_ptr() == t.data_ptr()   # a view, no copy
    flat = t.reshape(2, n * h_kv, d)
    for j in range(n):
        for h in range(h_kv):
            assert torch.equal(view[:, j, h], flat[:, j + h * n])
    one = torch.randn(n, 1, d)
    assert torch.equal(flat_gather_view(one), one)
    q, k, v = (f32(randn(s, 90 + i)) for i, s in enumerate(((n, h_q, d), (n, h_kv, d), (n, h_kv, d))))
    idx = np.random.default_rng(3).integers(0, n, size=(n, h_kv, kk)).astype(np.int64)
    ref = _reference_flat_gather64(q, k, v, idx, d ** 0.5)
    kf = np.ascontiguousarray(flat_gather_view(torch.from_numpy(k)).numpy())
    vf = np.ascontiguousarray(flat_gather_view(torch.from_numpy(v)).numpy())
    np.testing.assert_allclose(oracle.sparse_attention(q, kf, vf, idx), ref, rtol=1e-12, atol=1e-12)
    # the docstring semantics differ from the code's whenever h_kv > 1
    assert np.abs(oracle.sparse_attention(q, k, v, idx) - ref).max() > 1e-3


def test_attention_k_equals_n_matches_torch_sdpa():
    """Library cross-check: k = n sparse (causal) == dense == torch SDPA (float64)."""
    n, h_q, h_kv, d = 64, 8, 2, 32
    q, k, v = f32(randn((n, h_q, d), 70)), f32(randn((n, h_kv, d), 71)), f32(randn((n, h_kv, d), 72))
    idx = np.broadcast_to(np.arange(n), (n, h_kv, n)).copy()
    sp = oracle.sparse_attention(q, k, v, idx, causal=True)
    de = oracle.dense_attention(q, k, v, causal=True)
    g = h_q // h_kv
    tq = torch.from_numpy(q).double().transpose(0, 1)
    tk = torch.from_numpy(k).double().repeat_interleave(g, 1).transpose(0, 1)
    tv = torch.from_numpy(v).double().repeat_interleave(g, 1).transpose(0, 1)
    ts = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=True)
    ts = ts.transpose(0, 1).numpy()
    np.testing.assert_allclose(sp, ts, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(de, ts, rtol=1e-10, atol=1e-10)
    de_nc = oracle.dense_attention(q, k, v, causal=False)
    sp_nc = oracle.sparse_attention(q, k, v, idx, causal=False)  # reference semantics: no mask
    np.testing.assert_allclose(sp_nc, de_nc, rtol=1e-10, atol=1e-10)


def test_sparse_attention_fully_masked_row_is_zero():
    n = 8
    q, k, v = f32(randn((n, 2, 4), 80)), f32(randn((n, 1, 4), 81)), f32(randn((n, 1, 4), 82))
    idx = np.full((n, 1, 3), n - 1)
    out = oracle.sparse_attention(q, k, v, idx, causal=True)
    assert (out[: n - 1] == 0).all() and np.abs(out[n - 1]).sum() > 0


def test_brute_force_catches_planted_mistakes():
    """The brute-force checker is sensitive to the mistakes it guards against:
    a dropped GQA mean (head 0 only) or a reversed tie order changes the answer."""
    q, k, w_qr, w_kr, cb, a, b = _tiny_router_case(90)
    (good, _, _), ex = oracle.router_forward(q, k, w_qr, w_kr, cb, a, b, 6, with_stats=True)
    qc, kc = ex["q_codes"], ex["k_codes"]
    h_kv = k.shape[1]
    g = q.shape[1] // h_kv
    q_head0 = np.repeat(q[:, ::g], g, axis=1)  # every group member replaced by head 0
    assert not np.array_equal(oracle.brute_select(q_head0, k, qc, kc, 6, True), good)
    assert np.array_equal(oracle.brute_select(q, k, qc, kc, 6, True), good)


@pytest.mark.parametrize("mistake", ["sign", "mask", "kv_transposed", "scale_multiplier",
                                     "w_swapped", "group_index"])
def test_checks_catch_planted_mistakes(mistake):
    """Plausible mistakes, planted in the oracle's inputs or call, are caught by
    the independent checks: the brute-force selection, the float64 attention
    restatement, or the golden vectors' codes."""
    q, k, w_qr, w_kr, cb, a, b = _tiny_router_case(91)
    (good, _, _), ex = oracle.router_forward(q, k, w_qr, w_kr, cb, a, b, 6, with_stats=True)
    qc, kc = ex["q_codes"], ex["k_codes"]
    ref = oracle.brute_select(q, k, qc, kc, 6, True)
    np.testing.assert_array_equal(good, ref)
    idx = good
    att_ref = oracle.np_sparse_attention64(q, k, k[:, :, ::-1].copy(), idx)
    v = k[:, :, ::-1].copy()
    if mistake == "sign":
        bad = oracle.router_forward(-q, k, w_qr, w_kr, cb, a, b, 6, with_stats=False)[0]
        assert not np.array_equal(bad, ref)
    elif mistake == "mask":
        bad = oracle.router_forward(q, k, w_qr, w_kr, cb, a, b, 6, oracle.MASK_NONE)[0]
        assert not np.array_equal(bad, ref)
    elif mistake == "kv_transposed":
        bad = oracle.sparse_attention(q, v, k, idx)
        assert not np.allclose(bad, att_ref, rtol=1e-3, atol=1e-3)
        np.testing.assert_allclose(oracle.sparse_attention(q, k, v, idx), att_ref, rtol=1e-9, atol=1e-9)
    elif mistake == "scale_multiplier":
        d = q.shape[-1]
        bad = oracle.sparse_attention(q, k, v, idx, scale=1.0 / d ** 0.5)
        assert not np.allclose(bad, att_ref, rtol=1e-3, atol=1e-3)
    elif mistake == "w_swapped":
        bad = oracle.router_forward(q, k, w_kr, w_qr, cb, a, b, 6)[1]["q_codes"]
        assert not np.array_equal(bad, qc)
    elif mistake == "group_index":
        # query head j paired with kv head j % h_kv instead of j // g
        h_kv = k.shape[1]
        g = q.shape[1] // h_kv
        perm = np.array([(j % h_kv) * g + j // h_kv for j in range(q.shape[1])])
        bad = oracle.router_forward(q[:, perm], k, w_qr, w_kr, cb, a, b, 6)[0]
        assert not np.array_equal(bad, ref)
