"""CPU checks of the block-granular oracle (ssa/triton_kernel.py:141-294)."""

import numpy as np
import pytest

import oracle as orc


@pytest.mark.parametrize("n,h,k,bs,nkb", [(200, 2, 16, 32, None), (256, 1, 8, 64, 2), (77, 3, 5, 8, 4),
                                          (64, 2, 70, 16, None)])
def test_block_indices_equals_brute_force(n, h, k, bs, nkb):
    rng = np.random.default_rng(n + k)
    idx = rng.integers(0, n, (n, h, k))
    got = orc.block_indices(idx, bs, nkb)
    nb = (n + bs - 1) // bs
    want = orc.brute_block_indices(idx, bs, min(k, nb) if nkb is None else nkb)
    np.testing.assert_array_equal(got, want)
    assert got.shape == (nb, h, min(k, nb) if nkb is None else nkb)


def test_block_indices_known_answer_padding_counts_block_zero():
    """n = 5, block 4: query block 1 holds row 4 and three zero-padded rows,
    whose 6 references to block 0 outweigh row 4's two references to block 1."""
    idx = np.array([[4, 4], [4, 0], [4, 1], [4, 2], [4, 4]])[:, None, :]
    got = orc.block_indices(idx, 4, 1)
    np.testing.assert_array_equal(got[:, 0, 0], [1, 0])
    np.testing.assert_array_equal(orc.brute_block_indices(idx, 4, 1)[:, 0, 0], [1, 0])


def test_block_indices_ranking_invariants():
    rng = np.random.default_rng(5)
    n, h, k, bs, nkb = 300, 2, 12, 16, 6
    idx = rng.integers(0, n, (n, h, k))
    got = orc.block_indices(idx, bs, nkb)
    nb = (n + bs - 1) // bs
    blk = np.concatenate([idx // bs, np.zeros((nb * bs - n, h, k), np.int64)]).reshape(nb, bs, h, k)
    for bq in range(nb):
        for hh in range(h):
            cnt = np.bincount(blk[bq, :, hh].ravel(), minlength=nb)
            assert cnt.sum() == bs * k
            sel = got[bq, hh]
            assert len(set(sel.tolist())) == nkb
            c = cnt[sel]
            assert (np.diff(c) <= 0).all()                      # counts descending
            rest = np.setdiff1d(np.arange(nb), sel)
            assert cnt[rest].max(initial=-1) <= c.min()          # nothing better left out
            ties = sel[c == c.min()]
            assert (rest[cnt[rest] == c.min()] > ties.max()).all()  # ties by lower id


def test_block_attention_all_blocks_is_causal_dense():
    rng = np.random.default_rng(7)
    n, h_q, h_kv, d, bs = 100, 4, 2, 16, 16
    q, k, v = (rng.standard_normal((n, h, d)).astype(np.float32) for h in (h_q, h_kv, h_kv))
    nb = (n + bs - 1) // bs
    blocks = np.broadcast_to(np.arange(nb)[::-1], (nb, h_kv, nb)).copy()
    got = orc.block_sparse_attention64(q, k, v, blocks, bs)
    np.testing.assert_allclose(got, orc.dense_attention(q, k, v, causal=True), rtol=1e-5, atol=1e-5)


def test_block_attention_equals_token_path_on_expanded_indices():
    rng = np.random.default_rng(8)
    n, h_q, h_kv, d, bs, nkb = 128, 2, 1, 8, 16, 3
    q, k, v = (rng.standard_normal((n, h, d)).astype(np.float32) for h in (h_q, h_kv, h_kv))
    nb = n // bs
    blocks = np.stack([rng.permutation(nb)[:nkb] for _ in range(nb * h_kv)]).reshape(nb, h_kv, nkb)
    tok = (blocks[:, :, :, None] * bs + np.arange(bs)).reshape(nb, h_kv, nkb * bs)
    tok = np.repeat(tok, bs, axis=0)  # row i takes its block's list
    got = orc.block_sparse_attention64(q, k, v, blocks, bs)
    want = orc.np_sparse_attention64(q, k, v, tok, causal=True)
    rows = np.array([(tok[i] <= i).any() for i in range(n)])
    np.testing.assert_allclose(got[rows], want[rows], rtol=1e-10, atol=1e-12)
    assert (got[~rows] == 0).all()
