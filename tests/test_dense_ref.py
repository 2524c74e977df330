"""Pins of oracle/dense_ref.py, the reference's dense algorithm restated in torch
on the CPU (the bench's CPU baseline).  CPU only.

It must agree with the linear oracle: the same code assignments, the same
selected sets on rows whose candidates fill the top_k (the reference leaves the
-inf filler unspecified, survey Appendix B rule 5), candidate counts equal, and
the same attention outputs where the selections agree.
"""

import numpy as np
import torch

import oracle
from oracle import dense_ref
from tests.helpers import clustered_qk, router_params


def test_dense_ref_agrees_with_linear_oracle():
    n, h_q, h_kv, d, d_s, n_c, a, b, k = 300, 4, 2, 32, 16, 64, 8, 2, 24
    q, kk = clustered_qk(n, h_q, h_kv, d, 6, 0.3, seed=3)
    v = torch.randn(n, h_kv, d, generator=torch.Generator().manual_seed(4))
    w_qr, w_kr, cb = router_params(d, d_s, h_kv, n_c, seed=5)
    rows = torch.arange(n)
    with torch.no_grad():
        qc, ka = dense_ref.route_codes(q, kk, w_qr, w_kr, cb, a, b)
        idx, out = dense_ref.forward_rows(q, kk, v, w_qr, w_kr, cb, a, b, k, rows)
    ref_idx, ex = oracle.router_forward(q.numpy(), kk.numpy(), w_qr.numpy(), w_kr.numpy(),
                                        cb.numpy(), a, b, k, oracle.MASK_CAUSAL, with_stats=True)
    ref_idx, n_cand, _ = ref_idx
    # code sets (torch's topk order within equal scores aside, the sets agree)
    np.testing.assert_array_equal(np.sort(qc.numpy(), -1), np.sort(ex["q_codes"].transpose(1, 0, 2), -1))
    np.testing.assert_array_equal(np.sort(ka.numpy(), -1), np.sort(ex["k_codes"].transpose(1, 0, 2), -1))
    full = n_cand >= k                                  # [n, h_kv]
    assert full.sum() > 50 and (~full).sum() > 50
    got = np.sort(idx.numpy(), -1)
    ref = np.sort(ref_idx, -1)
    np.testing.assert_array_equal(got[full], ref[full])
    # attention where the selections agree (every full row)
    ref_att = oracle.sparse_attention(q.numpy(), kk.numpy(), v.numpy(), idx.numpy())
    np.testing.assert_allclose(out.numpy(), ref_att, rtol=1e-5, atol=1e-5)


def test_dense_ref_mask_is_the_set_definition():
    g = torch.Generator().manual_seed(9)
    qc = torch.randint(0, 12, (40, 2, 3), generator=g)
    kc = torch.randint(0, 12, (40, 2, 2), generator=g)
    m = dense_ref.candidate_mask(qc, kc, chunk=7)
    brute = oracle.brute_candidate_mask(qc.permute(1, 0, 2).numpy(), kc.permute(1, 0, 2).numpy(),
                                        causal=False)
    np.testing.assert_array_equal(m.permute(1, 0, 2).numpy(), brute)
