"""Host-side behaviour of the drop-in Python API, without a GPU: constructor
parameters, names and RNG draw order (ssa/router.py:28-70,
ssa/ssa_layer.py:29-66), mask handling, the input helpers of ssa/utils.py
checked against their closed forms, the PyTorch dense path, and the rule that
the hot path has no CPU fallback."""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import ssa_amd
from ssa_amd import _lib, kernels
from ssa_amd.router import CodebookRouter, mask_mode_for
from ssa_amd.ssa_layer import SSAAttention, ToyTransformerBlock, head_rope_tables
from ssa_amd.utils import (apply_rope, build_causal_mask, expand_kv_for_gqa, precompute_rope_freqs,
                           validate_indices)


def test_public_names():
    for name in ("CodebookRouter", "sparse_exact_attention", "dense_attention", "SSAAttention",
                 "ToyTransformerBlock", "apply_rope", "precompute_rope_freqs", "build_causal_mask",
                 "expand_kv_for_gqa"):
        assert hasattr(ssa_amd, name)


def test_router_init_order_and_names():
    torch.manual_seed(7)
    r = CodebookRouter(head_dim=64, route_dim=16, num_kv_heads=2, num_codebook=128,
                       codes_per_key=2, codes_per_query=8, top_k=32)
    torch.manual_seed(7)
    w_qr = torch.nn.Linear(64, 16, bias=False).weight
    w_kr = torch.nn.Linear(64, 16, bias=False).weight
    cb = torch.randn(2, 128, 16) / 16**0.5
    assert list(r.state_dict()) == ["codebook", "W_qr.weight", "W_kr.weight"]
    assert torch.equal(r.W_qr.weight, w_qr)
    assert torch.equal(r.W_kr.weight, w_kr)
    assert torch.equal(r.codebook, cb)
    assert r.temperature == 1.0
    # positional argument order of ssa/router.py:28-38
    r2 = CodebookRouter(32, 8, 4, 256, 3, 5, 17, 0.5)
    assert (r2.head_dim, r2.route_dim, r2.num_kv_heads, r2.num_codebook, r2.codes_per_key,
            r2.codes_per_query, r2.top_k, r2.temperature) == (32, 8, 4, 256, 3, 5, 17, 0.5)


def test_layer_init_order_and_names():
    torch.manual_seed(3)
    layer = SSAAttention(hidden_size=64, num_q_heads=4, num_kv_heads=2, head_dim=16,
                         route_dim=8, num_codebook=32, codes_per_key=2, codes_per_query=4,
                         top_k=8)
    torch.manual_seed(3)
    q = torch.nn.Linear(64, 64, bias=False)
    k = torch.nn.Linear(64, 32, bias=False)
    v = torch.nn.Linear(64, 32, bias=False)
    o = torch.nn.Linear(64, 64, bias=False)
    w_qr = torch.nn.Linear(16, 8, bias=False)
    w_kr = torch.nn.Linear(16, 8, bias=False)
    cb = torch.randn(2, 32, 8) / 8**0.5
    sd = layer.state_dict()
    assert set(sd) == {"q_proj.weight", "k_proj.weight", "v_proj.weight", "o_proj.weight",
                       "router.codebook", "router.W_qr.weight", "router.W_kr.weight"}
    for key, ref in (("q_proj.weight", q.weight), ("k_proj.weight", k.weight),
                     ("v_proj.weight", v.weight), ("o_proj.weight", o.weight),
                     ("router.W_qr.weight", w_qr.weight), ("router.W_kr.weight", w_kr.weight),
                     ("router.codebook", cb)):
        assert torch.equal(sd[key], ref), key


def test_hard_false_rejected():
    r = CodebookRouter(head_dim=16, route_dim=8, num_kv_heads=1, num_codebook=16, top_k=4)
    q = torch.randn(8, 1, 16)
    with pytest.raises(NotImplementedError):
        r(q, q, hard=False)


def test_no_cpu_fallback():
    r = CodebookRouter(head_dim=16, route_dim=8, num_kv_heads=1, num_codebook=16,
                       codes_per_key=2, codes_per_query=4, top_k=4)
    q = torch.randn(8, 2, 16)
    k = torch.randn(8, 1, 16)
    idx = torch.zeros(8, 1, 4, dtype=torch.int64)
    with pytest.raises(RuntimeError, match="HIP"):
        r(q, k, causal_mask=True)
    with pytest.raises(RuntimeError, match="HIP"):
        ssa_amd.sparse_exact_attention(q, k, k, idx)
    with pytest.raises(RuntimeError, match="HIP"):
        kernels.route_vectors(q.unsqueeze(0), r.W_qr.weight, 2)
    with pytest.raises(RuntimeError, match="HIP"):
        r.get_code_assignment(k)
    layer = SSAAttention(hidden_size=32, num_q_heads=2, num_kv_heads=1, head_dim=16, route_dim=8,
                         num_codebook=16, codes_per_key=2, codes_per_query=4, top_k=4)
    with pytest.raises(RuntimeError, match="HIP"):
        layer(torch.randn(1, 8, 32))


def test_router_shape_checks():
    r = CodebookRouter(head_dim=16, route_dim=8, num_kv_heads=2, num_codebook=16, top_k=4)
    with pytest.raises(AssertionError):
        r(torch.randn(8, 3, 16), torch.randn(8, 2, 16))
    with pytest.raises(ValueError):
        r(torch.randn(8, 4, 16), torch.randn(8, 1, 16))
    with pytest.raises(ValueError):
        r(torch.randn(8, 4, 8), torch.randn(8, 2, 8))
    with pytest.raises(ValueError):
        r(torch.randn(8, 16), torch.randn(8, 16))


def test_mask_mode_for():
    n = 6
    assert mask_mode_for(None, n) == (_lib.MASK_NONE, None)
    assert mask_mode_for(False, n) == (_lib.MASK_NONE, None)
    assert mask_mode_for(True, n) == (_lib.MASK_CAUSAL, None)
    assert mask_mode_for(build_causal_mask(n), n) == (_lib.MASK_CAUSAL, None)
    plain = torch.ones(n, n, dtype=torch.bool).tril()      # same values, untagged: honoured as given
    mode, m = mask_mode_for(plain, n)
    assert mode == _lib.MASK_DENSE and torch.equal(m, plain)
    mode, m = mask_mode_for(torch.eye(n), n)
    assert mode == _lib.MASK_DENSE and m.dtype == torch.bool
    with pytest.raises(ValueError):
        mask_mode_for(torch.ones(n, n + 1, dtype=torch.bool), n)
    with pytest.raises(TypeError):
        mask_mode_for("causal", n)


def test_build_causal_mask():
    m = build_causal_mask(5)
    assert m.dtype == torch.bool
    assert torch.equal(m, torch.tensor([[j <= i for j in range(5)] for i in range(5)]))


def test_precompute_rope_freqs_closed_form():
    d, n, theta = 64, 9, 1e4
    f = precompute_rope_freqs(d, n, theta).double()
    assert f.shape == (n, d // 2)
    for p in range(n):
        for m in range(d // 4):
            want = p * theta ** (-(2.0 * m) / (d / 2))
            assert f[p, m].item() == pytest.approx(want, rel=1e-6, abs=1e-6)
            assert f[p, m + d // 4].item() == f[p, m].item()


def test_apply_rope_closed_form_and_pair_norm():
    """Rotation of pairs (j, j + d/4) by the angle of row x.shape[-2], first d/2
    features only (ssa/utils.py:7-41; the pair-norm check is the reference's
    own, tests/test_attention.py:137-159)."""
    n, h, d = 5, 4, 16
    x = torch.randn(n, h, d, dtype=torch.float64)
    freqs = precompute_rope_freqs(d, 32, 1e4).double()
    y = apply_rope(x, freqs)
    q4 = d // 4
    for i in range(n):
        for r in range(h):
            for j in range(q4):
                a = freqs[r, j].item()
                x1, x2 = x[i, r, j].item(), x[i, r, j + q4].item()
                assert y[i, r, j].item() == pytest.approx(x1 * math.cos(a) - x2 * math.sin(a), abs=1e-12)
                assert y[i, r, j + q4].item() == pytest.approx(x2 * math.cos(a) + x1 * math.sin(a),
                                                               abs=1e-12)
    assert torch.equal(y[..., d // 2:], x[..., d // 2:])
    pn_x = x[..., :q4] ** 2 + x[..., q4:2 * q4] ** 2
    pn_y = y[..., :q4] ** 2 + y[..., q4:2 * q4] ** 2
    torch.testing.assert_close(pn_y, pn_x, atol=1e-6, rtol=0)
    assert torch.equal(y[:, 0], x[:, 0]), "angle row 0 is the identity"


def test_head_rope_tables_give_the_reference_layer_rotation():
    """The layer's host-side tables (head_rope_tables) plus the rotation the kernel
    applies (oracle.rope, bit-exact with ssa_rope on the GPU) equal the
    reference's per-batch apply_rope calls (ssa/ssa_layer.py:106-117), with and
    without position_ids."""
    import oracle

    B, h, d = 3, 4, 16
    freqs = precompute_rope_freqs(d, 32, 1e4)
    # n = 1: the reference's one angle row broadcasts over the heads
    for n in (7, 1):
        x = torch.randn(B, n, h, d)
        for pos in (None, torch.randint(0, 32, (B, n))):
            cos, sin = head_rope_tables(freqs, n, h, d, pos)
            got = oracle.rope(x.numpy(), cos.numpy(), sin.numpy(), d // 2, by_head=True)
            fb = [freqs[:n] if pos is None else freqs[pos[b]] for b in range(B)]
            ref = torch.stack([apply_rope(x[b], fb[b]) for b in range(B)])
            np.testing.assert_array_equal(got, ref.numpy())
    with pytest.raises(ValueError, match="angle rows"):
        head_rope_tables(freqs[:3], 3, h, d)


def test_expand_kv_for_gqa():
    """The reference helper tiles the KV heads: expanded head j is KV head
    j % h_kv (ssa/utils.py:103-106), unlike the attention functions, which
    give query head j KV head j // g.  No reference code path calls it."""
    kv = torch.randn(5, 2, 8)
    e = expand_kv_for_gqa(kv, 6, 2)
    assert e.shape == (5, 6, 8)
    for j in range(6):
        assert torch.equal(e[:, j], kv[:, j % 2])


def test_validate_indices():
    validate_indices(torch.tensor([[0, 3], [1, 2]]), 4, 2)
    with pytest.raises(AssertionError):
        validate_indices(torch.tensor([[0, 4]]), 4, 2)
    with pytest.raises(AssertionError):
        validate_indices(torch.tensor([[-1, 0]]), 4, 2)
    with pytest.raises(AssertionError):
        validate_indices(torch.tensor([[0, 1, 2]]), 4, 2)


def _attn64(q, k, v, mask, scale):
    n, hq, d = q.shape
    g = hq // k.shape[1]
    out = np.zeros((n, hq, d))
    for i in range(n):
        for j in range(hq):
            s = np.array([q[i, j] @ k[t, j // g] / scale for t in range(n)])
            s = np.where(mask[i], s, -np.inf) if mask is not None else s
            w = np.exp(s - s.max())
            w /= w.sum()
            out[i, j] = w @ v[:, j // g]
    return out


@pytest.mark.parametrize("causal", [False, True])
def test_dense_attention_textbook(causal):
    n, hq, hkv, d = 6, 4, 2, 8
    q, k, v = (torch.randn(n, h, d, dtype=torch.float64) for h in (hq, hkv, hkv))
    mask = build_causal_mask(n) if causal else None
    got = ssa_amd.dense_attention(q, k, v, causal_mask=mask, scale=2.5).numpy()
    ref = _attn64(q.numpy(), k.numpy(), v.numpy(), None if mask is None else mask.numpy(), 2.5)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)
    # library cross-check
    ke = k.repeat_interleave(hq // hkv, dim=1).transpose(0, 1)
    ve = v.repeat_interleave(hq // hkv, dim=1).transpose(0, 1)
    sd = F.scaled_dot_product_attention(q.transpose(0, 1), ke, ve, attn_mask=mask,
                                        scale=1.0 / math.sqrt(d)).transpose(0, 1)
    np.testing.assert_allclose(ssa_amd.dense_attention(q, k, v, causal_mask=mask).numpy(),
                               sd.numpy(), rtol=1e-10, atol=1e-10)


def test_dense_layer_path_on_cpu():
    """use_dense=True is the reference's comparison path (plain PyTorch)."""
    torch.manual_seed(0)
    blk = ToyTransformerBlock(hidden_size=32, num_q_heads=2, num_kv_heads=1, head_dim=16,
                              route_dim=8, num_codebook=16, codes_per_key=2, codes_per_query=4,
                              top_k=4)
    x = torch.randn(2, 8, 32)
    y = blk(x, use_dense=True)
    assert y.shape == x.shape and torch.isfinite(y).all()
    # batch independence (tests/test_integration.py:87-100)
    y0 = blk(x[:1], use_dense=True)
    torch.testing.assert_close(y[:1], y0, atol=1e-6, rtol=0)


def _reference_aux_loss(layer, x):
    """ssa/ssa_layer.py:140-257 step by step (dense n x n teacher and student for
    every row, then the sampled rows), on the layer's own parameters."""
    B, n, _ = x.shape
    hq, hkv, d = layer.num_q_heads, layer.num_kv_heads, layer.head_dim
    g, r = hq // hkv, layer.router
    q = layer.q_proj(x).view(B, n, hq, d)
    k = layer.k_proj(x).view(B, n, hkv, d)
    k_exp = k.unsqueeze(3).expand(-1, -1, -1, g, -1).reshape(B, n, hq, d)
    sample = torch.randperm(n)[:min(n, 64)]
    mask = build_causal_mask(n)
    total = 0.0
    for b in range(B):
        t = torch.einsum("shd,thd->sht", q[b], k_exp[b]) / d ** 0.5
        tw = F.softmax(t.masked_fill(~mask.unsqueeze(1), float("-inf")), dim=-1)
        qr = r.W_qr(q[b]).reshape(n, hkv, g, r.route_dim).mean(dim=2)
        kr = r.W_kr(k[b])
        cb = F.normalize(r.codebook, dim=-1)
        qsc = torch.einsum("shd,hcd->shc", F.normalize(qr, dim=-1), cb)
        ksc = torch.einsum("shd,hcd->shc", F.normalize(kr, dim=-1), cb)
        st = torch.einsum("shc,thc->sht", qsc, ksc).masked_fill(~mask.unsqueeze(1), float("-inf"))
        sw = F.softmax(st.unsqueeze(2).expand(-1, -1, g, -1).reshape(n, hq, n), dim=-1)
        total = total + F.kl_div(torch.log(sw[sample] + 1e-10), tw[sample], reduction="batchmean",
                                 log_target=False)
    return total / B


@pytest.mark.parametrize("n", [40, 150])
def test_auxiliary_loss_matches_the_reference_algorithm(n):
    """compute_auxiliary_loss (sampled rows only) equals the reference's dense
    algorithm on the same parameters and the same randperm draw, value and
    gradients; n = 150 > 64 samples a subset of the rows."""
    torch.manual_seed(3)
    layer = SSAAttention(hidden_size=64, num_q_heads=4, num_kv_heads=2, head_dim=16, route_dim=8,
                         num_codebook=32, codes_per_key=2, codes_per_query=4, top_k=8)
    x = torch.randn(2, n, 64)
    torch.manual_seed(11)
    got = layer.compute_auxiliary_loss(x)
    g_got = torch.autograd.grad(got, [layer.router.W_qr.weight, layer.router.codebook, layer.q_proj.weight])
    torch.manual_seed(11)
    ref = _reference_aux_loss(layer, x)
    g_ref = torch.autograd.grad(ref, [layer.router.W_qr.weight, layer.router.codebook, layer.q_proj.weight])
    assert got.dim() == 0 and float(got) > 0
    torch.testing.assert_close(got, ref, rtol=1e-5, atol=1e-6)
    for a, b in zip(g_got, g_ref):
        # the q_proj gradient is NaN in both: the teacher's masked weights are
        # exactly 0, and kl_div's derivative in its target is target / target
        torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-6, equal_nan=True)
    assert bool(torch.isnan(g_ref[2]).any()) and bool(torch.isfinite(g_got[0]).all())
    # _get_routing_logits keeps the reference's full [n, h_kv, n] form
    q = layer.q_proj(x[0]).view(n, 4, 16)
    k = layer.k_proj(x[0]).view(n, 2, 16)
    full = layer._get_routing_logits(q, k, build_causal_mask(n))
    rows = torch.tensor([0, 5, n - 1])
    part = layer._get_routing_logits(q, k, build_causal_mask(n)[rows], rows=rows)
    assert full.shape == (n, 2, n)
    torch.testing.assert_close(part, full[rows], rtol=1e-6, atol=1e-6)
    assert bool(torch.isinf(full[0, :, 1:]).all()), "causal: future keys masked"
