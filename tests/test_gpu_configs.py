"""Parity at the small and layer-level BASELINE configurations, at the north
star's tolerances (fp32 1e-5; bf16 1e-3 on the fp32 attention output).

* c1 -- the README quick-start layer (README.md:107-123): SSAAttention(hidden
  512, 8/2 heads, d 64, d_s 32, N_c 2048, b 4, a 16, k 256), fp32, default init
  from a fixed seed in the reference's construction order, x ~ N(0, 1) of shape
  (2, 1024, 512), freqs = precompute_rope_freqs(64, 1024, 1e4).
* c2 -- the dense-equivalence check end to end: router at k = n = 2048 (N_c
  1024, a 16, b 4) on i.i.d. N(0, 1) fp32 Q/K/V, then attention; with the
  causal option it equals dense causal attention, without it (the reference's
  stage 3, which applies no mask) dense attention over all keys.
* c4 -- the random-init decoder attention block: RMSNorm, then one full
  SSAAttention forward with projections (d_model 4096, 32/8 heads, d 128,
  N_c 4096, a 16, b 4, k 512, RoPE theta 1e6), bf16, B 4, n 8192; checked on
  sampled rows of every batch element (the oracle is too slow for all rows).

Every check feeds the oracle the layer's own projections (torch GEMMs, not
part of this build's kernels): RoPE, code assignments, candidate indices are
bit-exact; attention within the tolerance.
"""

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import f32

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _layer_oracle_rows(layer, q_lin, k_lin, freqs, q, k, v, b, rows, orc, causal_attention):
    """Oracle RoPE of the projections (bit-exact with the layer's q/k), then the
    oracle router and attention for the sampled rows of batch element b."""
    from ssa_amd.ssa_layer import head_rope_tables

    h_q, h_kv, d = layer.num_q_heads, layer.num_kv_heads, layer.head_dim
    # the angle tables as the layer computes them on the device (freqs.cos(),
    # freqs.sin() in the reference); the rotation itself is what is checked
    cos, sin = (t.cpu().numpy() for t in head_rope_tables(freqs.to(q.device), q.shape[1], h_q, d))
    round_out = q.dtype == torch.bfloat16
    for lin, rot_t, name in ((q_lin, q, "q"), (k_lin, k, "k")):
        ref = orc.rope(orc.to_f32(lin[b:b + 1, rows]), cos, sin, d // 2, True)[0]
        if round_out:
            ref = orc.bf16_round(ref)
        np.testing.assert_array_equal(orc.to_f32(rot_t[b, rows]), ref, err_msg=f"RoPE {name}")
    qf, kf, vf = orc.to_f32(q[b]), orc.to_f32(k[b]), orc.to_f32(v[b])
    r = layer.router
    ref_idx, ex = orc.router_forward(qf, kf, f32(r.W_qr.weight), f32(r.W_kr.weight),
                                     f32(r.codebook), r.codes_per_query, r.codes_per_key, r.top_k,
                                     orc.MASK_CAUSAL, rows=rows, sorted=False)
    att = orc.sparse_attention(qf, kf, vf, ref_idx, causal=causal_attention, rows=rows)
    return ref_idx, ex, att


# ------------------------------------------------------------------- c1

@pytest.fixture(scope="module")
def c1(dev):
    from ssa_amd import SSAAttention, precompute_rope_freqs

    _say("c1: README layer, fp32, B 2, n 1024")
    torch.manual_seed(0)
    layer = SSAAttention(hidden_size=512, num_q_heads=8, num_kv_heads=2, head_dim=64,
                         route_dim=32, num_codebook=2048, codes_per_key=4, codes_per_query=16,
                         top_k=256)
    x = torch.randn(2, 1024, 512)
    freqs = precompute_rope_freqs(64, 1024, 1e4)
    layer = layer.to(dev).eval()
    with torch.no_grad():
        xd, fd = x.to(dev), freqs.to(dev)
        out = layer(xd, freqs=fd)
        q, k, v = layer.project(xd, None, fd)
        q_lin = layer.q_proj(xd).view(2, 1024, 8, 64)
        k_lin = layer.k_proj(xd).view(2, 1024, 2, 64)
        idx_sorted = torch.stack([layer.router(q[b], k[b], causal_mask=True) for b in range(2)])
        res = layer.router.route(q, k, causal_mask=True, sorted=False)
        from ssa_amd import sparse_exact_attention
        att = sparse_exact_attention(q, k, v, res.indices)
    torch.cuda.synchronize()
    return dict(layer=layer, x=x, freqs=freqs, out=out, q=q, k=k, v=v, q_lin=q_lin, k_lin=k_lin,
                idx_sorted=idx_sorted, res=res, att=att)


@pytest.mark.parametrize("b", [0, 1])
def test_c1_layer_bit_exact_routing_and_1e5_attention(c1, orc, b):
    layer = c1["layer"]
    n = 1024
    rows = np.arange(n)
    ref_idx, ex, att = _layer_oracle_rows(layer, c1["q_lin"], c1["k_lin"], c1["freqs"], c1["q"],
                                          c1["k"], c1["v"], b, rows, orc, False)
    res = c1["res"]
    np.testing.assert_array_equal(res.q_codes[b].cpu().numpy(), ex["q_codes"])
    np.testing.assert_array_equal(res.k_codes[b].cpu().numpy(), ex["k_codes"])
    np.testing.assert_array_equal(res.indices[b].cpu().numpy(), ref_idx)
    # the drop-in forward's default (score) order
    ref_sorted = orc.select(orc.to_f32(c1["q"][b]), orc.to_f32(c1["k"][b]), ex["q_codes"],
                            ex["offsets"], ex["postings"], 4, 256, orc.MASK_CAUSAL)
    np.testing.assert_array_equal(c1["idx_sorted"][b].cpu().numpy(), ref_sorted)
    # stage 3 with the reference's semantics (no mask), fp32 tolerance 1e-5
    np.testing.assert_allclose(c1["att"][b].cpu().numpy(), att, rtol=1e-5, atol=1e-5)
    # the layer's output: o_proj of that attention output
    w_o = f32(layer.o_proj.weight).astype(np.float64)
    ref_out = att.reshape(n, -1) @ w_o.T
    np.testing.assert_allclose(c1["out"][b].cpu().numpy(), ref_out, rtol=1e-5, atol=1e-5)


# ------------------------------------------------------------------- c2

@pytest.fixture(scope="module")
def c2(dev):
    from ssa_amd import CodebookRouter, sparse_exact_attention

    _say("c2: router at k = n = 2048, fp32")
    n, h_q, h_kv, d = 2048, 8, 2, 64
    g = torch.Generator().manual_seed(2)
    q, k, v = (torch.randn(n, h, d, generator=g) for h in (h_q, h_kv, h_kv))
    torch.manual_seed(3)
    router = CodebookRouter(head_dim=d, route_dim=32, num_kv_heads=h_kv, num_codebook=1024,
                            codes_per_key=4, codes_per_query=16, top_k=n).to(dev)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    with torch.no_grad():
        idx = router(qd, kd, causal_mask=True)
        out_causal = sparse_exact_attention(qd, kd, vd, idx, causal=True)
        out_ref_semantics = sparse_exact_attention(qd, kd, vd, idx)
    torch.cuda.synchronize()
    return dict(q=q, k=k, v=v, router=router, idx=idx, out_causal=out_causal,
                out_ref=out_ref_semantics)


def test_c2_router_at_k_equals_n_bit_exact(c2, orc):
    r = c2["router"]
    ref_idx, _ = orc.router_forward(c2["q"].numpy(), c2["k"].numpy(), f32(r.W_qr.weight),
                                    f32(r.W_kr.weight), f32(r.codebook), 16, 4, 2048,
                                    orc.MASK_CAUSAL)
    got = c2["idx"].cpu().numpy()
    np.testing.assert_array_equal(got, ref_idx)
    # every row lists each key exactly once
    assert np.array_equal(np.sort(got, -1), np.broadcast_to(np.arange(2048), got.shape))


def test_c2_ssa_equals_dense(c2, orc):
    """SSA(k = n) == dense attention within 1e-5 (fp32): causal with the causal
    option, over all keys with the reference's unmasked stage 3 (survey F3)."""
    q, k, v = c2["q"].numpy(), c2["k"].numpy(), c2["v"].numpy()
    dense_causal = orc.dense_attention(q, k, v, causal=True)
    np.testing.assert_allclose(c2["out_causal"].cpu().numpy(), dense_causal, rtol=1e-5, atol=1e-5)
    dense_all = orc.dense_attention(q, k, v, causal=False)
    np.testing.assert_allclose(c2["out_ref"].cpu().numpy(), dense_all, rtol=1e-5, atol=1e-5)
    # and the reference's own dense path (ssa/attention.py:118-158) run by torch
    from ssa_amd import build_causal_mask, dense_attention
    td = dense_attention(c2["q"].double(), c2["k"].double(), c2["v"].double(),
                         causal_mask=build_causal_mask(2048))
    np.testing.assert_allclose(c2["out_causal"].cpu().numpy(), td.numpy(), rtol=1e-5, atol=1e-5)


# ------------------------------------------------------------------- c4

@pytest.fixture(scope="module")
def c4(dev):
    import bench

    _say("c4: decoder block, bf16, B 4, n 8192, d_model 4096")
    blk = bench.make_block(bench.CONFIGS["c4"], 0, dev)
    with torch.no_grad():
        x = blk["x"]
        h = blk["norm"](x)
        out = blk["layer"](h, freqs=blk["freqs"])
        layer = blk["layer"]
        q, k, v = layer.project(h, None, blk["freqs"])
        B, n = h.shape[:2]
        q_lin = layer.q_proj(h).view(B, n, layer.num_q_heads, layer.head_dim)
        k_lin = layer.k_proj(h).view(B, n, layer.num_kv_heads, layer.head_dim)
        res = layer.router.route(q, k, causal_mask=True, sorted=False, index_dtype=torch.int32,
                                 with_order=True, with_prefix=True)
        att32 = torch.empty(q.shape, device=dev, dtype=torch.float32)
        from ssa_amd import kernels
        kernels.sparse_attention(q, k, v, res.indices, None, False, out=att32, row_order=res.order,
                                 row_prefix=res.prefix)
        att_bf16 = kernels.sparse_attention(q, k, v, res.indices, None, False, row_order=res.order,
                                            row_prefix=res.prefix)
        again = layer.o_proj(att_bf16.reshape(B, n, -1))
    torch.cuda.synchronize()
    return dict(layer=layer, freqs=blk["freqs"], out=out, q=q, k=k, v=v, q_lin=q_lin, k_lin=k_lin,
                res=res, att32=att32, again=again)


def test_c4_output_is_o_proj_of_the_attention(c4):
    """The layer's output is o_proj of the bf16 attention output (same kernels,
    same inputs and processing order, run again outside the layer)."""
    assert torch.equal(c4["out"], c4["again"])


@pytest.mark.parametrize("b", [0, 3])
def test_c4_rows_vs_oracle(c4, orc, b):
    n = c4["q"].shape[1]
    rng = np.random.default_rng(10 + b)
    rows = np.array(sorted(set(rng.choice(n, 40, replace=False).tolist()) | {0, 1, 511, n - 1}),
                    dtype=np.int64)
    ref_idx, ex, att = _layer_oracle_rows(c4["layer"], c4["q_lin"], c4["k_lin"], c4["freqs"],
                                          c4["q"], c4["k"], c4["v"], b, rows, orc, False)
    res = c4["res"]
    np.testing.assert_array_equal(res.q_codes[b][:, rows].cpu().numpy(), ex["q_codes"][:, rows])
    np.testing.assert_array_equal(res.k_codes[b].cpu().numpy(), ex["k_codes"])
    np.testing.assert_array_equal(res.offsets[b].cpu().numpy(), ex["offsets"])
    np.testing.assert_array_equal(res.postings[b].cpu().numpy(), ex["postings"])
    np.testing.assert_array_equal(res.indices[b][rows].to(torch.int64).cpu().numpy(), ref_idx)
    np.testing.assert_allclose(c4["att32"][b][rows].cpu().numpy(), att, rtol=1e-3, atol=1e-3)
