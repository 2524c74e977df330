"""The committed golden vectors (tests/golden/ssa_golden.npz, written by
tests/golden/make_golden.py from an independent float64 restatement with every
ranking margin >= 1e-4) against the CPU oracle and, on a GPU, against the HIP
path through the drop-in API.  Indices are compared exactly; attention outputs
within 1e-5 (oracle, float64) and 2e-5 (GPU, fp32 inputs)."""

import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ssa_golden.npz")


def _cases():
    z = np.load(GOLDEN)   # allow_pickle stays False: plain numeric and string arrays
    names = sorted({k.split("/")[0] for k in z.files})
    out = {}
    for nm in names:
        c = {k.split("/", 1)[1]: z[k] for k in z.files if k.startswith(nm + "/")}
        p = c["params"]
        c.update(dict(zip(("n", "h_q", "h_kv", "d", "d_s", "n_c", "a", "b", "top_k", "seed"),
                          (int(x) for x in p))))
        c["mask_kind"] = str(c["mask_kind"])
        out[nm] = c
    return out


CASES = _cases()


def _mask_mode(orc, c):
    return {"causal": orc.MASK_CAUSAL, "none": orc.MASK_NONE, "dense": orc.MASK_DENSE}[c["mask_kind"]]


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_matches_golden(orc, name):
    c = CASES[name]
    g = c["h_q"] // c["h_kv"]
    chat = orc.normalize(c["codebook"])
    qc = orc.code_topk(orc.route_vectors(c["q"], c["w_qr"], g), chat, c["a"])
    kc = orc.code_topk(orc.route_vectors(c["k"], c["w_kr"], 1), chat, c["b"])
    np.testing.assert_array_equal(qc.transpose(1, 0, 2), c["q_codes"])
    np.testing.assert_array_equal(kc.transpose(1, 0, 2), c["k_codes"])
    off, post = orc.build_index(kc, c["n_c"])
    mode = _mask_mode(orc, c)
    for sorted_ in (True, False):
        idx, ncand, _ = orc.select(c["q"], c["k"], qc, off, post, c["b"], c["top_k"], mode,
                                   mask=c["mask"] if mode == orc.MASK_DENSE else None,
                                   with_stats=True, sorted=sorted_)
        np.testing.assert_array_equal(ncand, c["n_cand"])
        if sorted_:
            np.testing.assert_array_equal(idx, c["indices"])
        else:
            # same set; the selected keys ascending, then the same filler
            k_eff = min(c["top_k"], c["n"])
            m = np.minimum(c["n_cand"], k_eff)
            for i in range(c["n"]):
                for h in range(c["h_kv"]):
                    want = np.concatenate([np.sort(c["indices"][i, h, :m[i, h]]),
                                           c["indices"][i, h, m[i, h]:]])
                    np.testing.assert_array_equal(idx[i, h], want)
    for causal, key in ((False, "out"), (True, "out_causal")):
        o = orc.sparse_attention(c["q"], c["k"], c["v"], c["indices"], causal=causal)
        np.testing.assert_allclose(o, c[key], rtol=1e-5, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASES))
def test_gpu_matches_golden(dev, name):
    import torch

    from ssa_amd import CodebookRouter, sparse_exact_attention

    c = CASES[name]
    r = CodebookRouter(head_dim=c["d"], route_dim=c["d_s"], num_kv_heads=c["h_kv"],
                       num_codebook=c["n_c"], codes_per_key=c["b"], codes_per_query=c["a"],
                       top_k=c["top_k"]).to(dev)
    with torch.no_grad():
        r.W_qr.weight.copy_(torch.from_numpy(c["w_qr"]))
        r.W_kr.weight.copy_(torch.from_numpy(c["w_kr"]))
        r.codebook.copy_(torch.from_numpy(c["codebook"]))
    q, k, v = (torch.from_numpy(c[x]).to(dev) for x in ("q", "k", "v"))
    mask = {"causal": True, "none": None,
            "dense": torch.from_numpy(c["mask"]).to(dev)}[c["mask_kind"]]
    res = r.route(q, k, causal_mask=mask, with_stats=True)
    np.testing.assert_array_equal(res.q_codes[0].permute(1, 0, 2).cpu().numpy(), c["q_codes"])
    np.testing.assert_array_equal(res.k_codes[0].permute(1, 0, 2).cpu().numpy(), c["k_codes"])
    np.testing.assert_array_equal(res.stats[0, :, :, 0].T.cpu().numpy(), c["n_cand"])
    idx = res.indices_view
    assert idx.dtype == torch.int64
    np.testing.assert_array_equal(idx.cpu().numpy(), c["indices"])
    for causal, key in ((False, "out"), (True, "out_causal")):
        o = sparse_exact_attention(q, k, v, idx, causal=causal)
        np.testing.assert_allclose(o.cpu().numpy(), c[key], rtol=2e-5, atol=2e-5)
