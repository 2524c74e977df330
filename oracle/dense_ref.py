"""The reference's dense algorithm on the CPU -- TEST INFRASTRUCTURE / CPU BASELINE ONLY.

The reference's own op sequence in torch eager on the CPU, for a set of query
rows against every key (the reference runs it with rows = all n):

* routing, ssa/router.py:102-141: project, GQA mean, F.normalize, codebook
  einsum / temperature, topk(b) for keys and topk(a) for queries;
* _select_candidates, ssa/router.py:170-214: dense rescoring
  einsum("shgd,thd->shgt") / sqrt(d), causal masked_fill(-inf), mean over the
  group, the candidate mask, masked_fill(-inf), topk(min(k, n)), zero padding;
* _build_candidate_mask, ssa/router.py:216-259: broadcast compare of the
  query codes with chunks of 128 keys' codes;
* sparse_exact_attention, ssa/attention.py:64-113: gather, grouped einsum /
  scale, softmax, einsum with V.  The gather takes K[indices[i, h], h] as the
  function's docstring states (ssa/attention.py:57-60); the reference's
  flat-index arithmetic (:79-92) offsets by h * n into a [n * h_kv, d] view
  of an [n, h_kv, d] tensor, which picks other rows whenever h_kv > 1.

Memory is O(rows * n * h_q): with every row it is the reference's O(n^2)
footprint (about 280 GB at n = 32768, GQA 32/8), so the bench times it on a
sample of query rows, each of which does exactly the per-row work of the full
algorithm (all n keys scored and masked), and scales to n rows.  Nothing in
the product path imports this module.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def route_codes(q, k, w_qr, w_kr, codebook, a: int, b: int, temperature: float = 1.0):
    """ssa/router.py:102-141 -> (top_q_codes [n, h_kv, a], k_code_assign [n, h_kv, b])."""
    n, h_q, _ = q.shape
    h_kv = k.shape[1]
    d_s = w_qr.shape[0]
    q_route = (q @ w_qr.T).view(n, h_kv, h_q // h_kv, d_s).mean(dim=2)
    k_route = k @ w_kr.T
    qn = F.normalize(q_route, dim=-1)
    kn = F.normalize(k_route, dim=-1)
    cn = F.normalize(codebook, dim=-1)
    q_scores = torch.einsum("shd,hcd->shc", qn, cn) / temperature
    k_scores = torch.einsum("shd,hcd->shc", kn, cn) / temperature
    _, k_assign = k_scores.topk(b, dim=-1)
    _, q_codes = q_scores.topk(a, dim=-1)
    return q_codes, k_assign


def candidate_mask(q_codes_rows, k_assign, chunk: int = 128):
    """ssa/router.py:241-257 for the given query rows: [rows, h_kv, n] bool."""
    r, h, a = q_codes_rows.shape
    n, _, b = k_assign.shape
    mask = torch.zeros(r, h, n, dtype=torch.bool)
    step = min(chunk, n)
    q_exp = q_codes_rows.view(r, 1, h, 1, a)
    for s in range(0, n, step):
        e = min(s + step, n)
        k_exp = k_assign[s:e].view(1, e - s, h, b, 1)
        mask[:, :, s:e] = (q_exp == k_exp).any(dim=-1).any(dim=-1).permute(0, 2, 1)
    return mask


def select(q, k, q_codes, k_assign, top_k: int, rows, causal: bool = True):
    """ssa/router.py:170-214 for query rows `rows` (int64 tensor) against every key."""
    n, h_q, d = q.shape
    h_kv = k.shape[1]
    g = h_q // h_kv
    qg = q[rows].view(len(rows), h_kv, g, d)
    scores = torch.einsum("shgd,thd->shgt", qg, k) / (d ** 0.5)
    if causal:
        allowed = rows[:, None] >= torch.arange(n)[None, :]
        scores = scores.masked_fill(~allowed[:, None, None, :], float("-inf"))
    routing = scores.mean(dim=2)
    routing = routing.masked_fill(~candidate_mask(q_codes[rows], k_assign), float("-inf"))
    kk = min(top_k, n)
    _, idx = routing.topk(kk, dim=-1)
    if kk < top_k:
        idx = torch.cat([idx, torch.zeros(len(rows), h_kv, top_k - kk, dtype=idx.dtype)], dim=-1)
    return idx


def sparse_attention(q, k, v, idx, rows, scale=None):
    """ssa/attention.py:64-113 for query rows `rows`; idx [len(rows), h_kv, k]."""
    n, h_q, d = q.shape
    h_kv = k.shape[1]
    g = h_q // h_kv
    if scale is None:
        scale = d ** 0.5
    heads = torch.arange(h_kv)[None, :, None]
    kg = k[idx, heads]                      # [r, h_kv, k, d]
    vg = v[idx, heads]
    qg = q[rows].reshape(len(rows), h_kv, g, d)
    w = F.softmax(torch.einsum("nhgd,nhkd->nhgk", qg, kg) / scale, dim=-1)
    return torch.einsum("nhgk,nhkd->nhgd", w, vg).reshape(len(rows), h_q, d)


def forward_rows(q, k, v, w_qr, w_kr, codebook, a: int, b: int, top_k: int, rows,
                 causal: bool = True):
    """Router (all keys' codes, the rows' query codes), selection and attention
    for query rows `rows`: the reference's forward restricted to those rows."""
    q_codes, k_assign = route_codes(q, k, w_qr, w_kr, codebook, a, b)
    idx = select(q, k, q_codes, k_assign, top_k, rows, causal)
    return idx, sparse_attention(q, k, v, idx, rows)
