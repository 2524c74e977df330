"""Writes tests/golden/ssa_golden.npz: small end-to-end SSA forward vectors.

The reference ships no golden vectors, so these come from an independent
float64 PyTorch restatement written in the reference's own operation order
(it does not run or import the reference):

  routing      q.W_qr^T per head, mean over the g heads of a KV group, k.W_kr^T,
               F.normalize of both and of the codebook, einsum scores
               / temperature, top-b / top-a codes     (ssa/router.py:102-141)
  candidates   broadcast compare of query codes against key codes, causal or
               dense mask                             (ssa/router.py:216-259)
  selection    dense rescoring mean_g(q.k) / sqrt(d) of every key, non-candidates
               at -inf, top-k by score                (ssa/router.py:151-214)
  attention    gather, softmax(q.K / sqrt(d)), .V     (ssa/attention.py:12-115)

where the reference leaves a choice open, the build's contract decides:
ties and the -inf filler go to the lowest index (filler = lowest non-candidate
indices ascending) and k > n pads with index 0.  Each case's seed is advanced
until every ranking boundary the output depends on (code top-a / top-b and
their order, the k-th candidate and the order of the selected keys) has a
score gap of at least MARGIN, so fp32 implementations with any summation order
must reproduce the indices exactly.

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "ssa_golden.npz")
MARGIN = 1e-4

CASES = {
    # name: n, h_q, h_kv, d, d_s, n_c, a, b, k, mask ("causal" | "none" | "dense")
    "causal_gqa": dict(n=48, h_q=4, h_kv=2, d=32, d_s=8, n_c=16, a=4, b=2, k=12, mask="causal"),
    "pad_k_gt_n": dict(n=20, h_q=2, h_kv=1, d=16, d_s=8, n_c=8, a=3, b=2, k=24, mask="causal"),
    "nomask_mha": dict(n=32, h_q=2, h_kv=2, d=16, d_s=4, n_c=12, a=2, b=1, k=8, mask="none"),
    "dense_mask": dict(n=40, h_q=6, h_kv=2, d=16, d_s=8, n_c=16, a=4, b=3, k=10, mask="dense"),
}


def normalize(x):
    return x / x.norm(dim=-1, keepdim=True).clamp_min(1e-12)


def ranked(scores):
    """Indices by (score desc, index asc) along the last axis."""
    idx = np.argsort(-scores, axis=-1, kind="stable")
    return idx


def min_gap(sorted_scores, upto):
    """Smallest gap between consecutive finite scores among the first upto+1."""
    s = sorted_scores[..., : upto + 1]
    s = np.where(np.isfinite(s), s, np.nan)
    g = s[..., :-1] - s[..., 1:]
    return np.nanmin(g) if np.isfinite(g).any() else np.inf


def make_case(c, seed):
    n, h_q, h_kv, d, d_s, n_c, a, b, k = (c[x] for x in ("n", "h_q", "h_kv", "d", "d_s", "n_c", "a", "b", "k"))
    g = h_q // h_kv
    gen = torch.Generator().manual_seed(seed)
    # inputs rounded to fp32 (the stored values are exactly what every implementation reads)
    q = torch.randn(n, h_q, d, generator=gen).float().double()
    kk = torch.randn(n, h_kv, d, generator=gen).float().double()
    v = torch.randn(n, h_kv, d, generator=gen).float().double()
    w_qr = (torch.rand(d_s, d, generator=gen) * 2 - 1).div(d ** 0.5).float().double()
    w_kr = (torch.rand(d_s, d, generator=gen) * 2 - 1).div(d ** 0.5).float().double()
    cb = (torch.randn(h_kv, n_c, d_s, generator=gen) / d_s ** 0.5).float().double()
    if c["mask"] == "dense":
        allowed = (torch.rand(n, n, generator=gen) < 0.6).numpy()
    elif c["mask"] == "causal":
        allowed = np.tril(np.ones((n, n), dtype=bool))
    else:
        allowed = np.ones((n, n), dtype=bool)

    # routing (project, then mean over the group; normalize; cosine scores)
    q_route = torch.einsum("nhd,sd->nhs", q, w_qr).view(n, h_kv, g, d_s).mean(2)
    k_route = torch.einsum("nhd,sd->nhs", kk, w_kr)
    qs = torch.einsum("nhs,hcs->nhc", normalize(q_route), normalize(cb)).numpy()
    ks = torch.einsum("nhs,hcs->nhc", normalize(k_route), normalize(cb)).numpy()
    q_codes = ranked(qs)[..., :a]
    k_codes = ranked(ks)[..., :b]
    gap = min(min_gap(np.take_along_axis(qs, ranked(qs), -1), a),
              min_gap(np.take_along_axis(ks, ranked(ks), -1), b))

    # candidate mask by broadcast compare, then the mask
    cand = (q_codes[:, None, :, :, None] == k_codes[None, :, :, None, :]).any(-1).any(-1)  # [i, j, h]
    cand = cand.transpose(0, 2, 1) & allowed[:, None, :]                                  # [i, h, j]

    # dense rescoring: mean over the group of per-head q.k / sqrt(d)
    s = torch.einsum("ihgd,jhd->ihgj", q.view(n, h_kv, g, d), kk) / d ** 0.5
    s = s.mean(2).numpy()                                                                 # [i, h, j]
    s_c = np.where(cand, s, -np.inf)
    order = ranked(s_c)
    k_eff = min(k, n)
    idx = np.zeros((n, h_kv, k), dtype=np.int64)
    n_cand = cand.sum(-1)
    for i in range(n):
        for h in range(h_kv):
            m = int(min(n_cand[i, h], k_eff))
            sel = order[i, h, :m]
            filler = np.flatnonzero(~cand[i, h])[: k_eff - m]
            idx[i, h, :k_eff] = np.concatenate([sel, filler])
            # boundaries: the order of the selected keys, and the k-th vs the next
            # candidate when some candidates are cut
            srt = s_c[i, h, order[i, h]]
            upto = k_eff if n_cand[i, h] > k_eff else m - 1
            if upto > 0:
                gap = min(gap, min_gap(srt, upto))

    # attention over the indices: reference semantics (no mask) and causal
    out = {}
    for causal in (False, True):
        o = np.zeros((n, h_q, d))
        qn, kn, vn = q.numpy(), kk.numpy(), v.numpy()
        for i in range(n):
            for hq in range(h_q):
                h = hq // g
                js = idx[i, h]
                if causal:
                    js = js[js <= i]
                if js.size == 0:
                    continue
                lg = kn[js, h] @ qn[i, hq] / d ** 0.5
                w = np.exp(lg - lg.max())
                o[i, hq] = (w / w.sum()) @ vn[js, h]
        out["out_causal" if causal else "out"] = o
    arrays = dict(q=q.float().numpy(), k=kk.float().numpy(), v=v.float().numpy(),
                  w_qr=w_qr.float().numpy(), w_kr=w_kr.float().numpy(), codebook=cb.float().numpy(),
                  mask=allowed, q_codes=q_codes.astype(np.int32), k_codes=k_codes.astype(np.int32),
                  n_cand=n_cand.astype(np.int32), indices=idx, **out)
    return arrays, gap


def main():
    blobs = {}
    for name, c in CASES.items():
        seed = 0
        while True:
            arrays, gap = make_case(c, seed)
            if gap >= MARGIN:
                break
            seed += 1
        print(f"{name}: seed {seed}, min ranking gap {gap:.3g}")
        for key, val in arrays.items():
            blobs[f"{name}/{key}"] = val
        blobs[f"{name}/params"] = np.array(
            [c[x] for x in ("n", "h_q", "h_kv", "d", "d_s", "n_c", "a", "b", "k")] + [seed], dtype=np.int64)
        blobs[f"{name}/mask_kind"] = np.array(c["mask"])
    np.savez_compressed(OUT, **blobs)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
