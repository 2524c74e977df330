"""Candidate selection (ssa/router.py:151-214) through the workspace path in index
order: the wave-per-row union, the matrix-core screen of rows with more than k
candidates (bf16, d = 64 or 128) and the exact pass for the rows the screen
cannot settle.  Every case must give the indices and stats of the
one-block-per-row kernel, which the oracle pins, bit for bit.

Codes are synthetic so that the candidate counts are controlled: a query's
candidates are the keys sharing one of its codes (ssa/router.py:241-257).
"""

import numpy as np
import pytest
import torch

from tests.helpers import f32, randn

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _codes(B, h_kv, n, n_c, a, b, seed):
    """q_codes [B,h,n,a], k_codes [B,h,n,b]: distinct codes per row."""
    rng = np.random.default_rng(seed)
    qc = np.argsort(rng.random((B, h_kv, n, n_c)), axis=-1)[..., :a].astype(np.int32)
    kc = np.argsort(rng.random((B, h_kv, n, n_c)), axis=-1)[..., :b].astype(np.int32)
    return qc, kc


def _case(orc, dev, B, n, h_kv, g, d, n_c, a, b, seed, k_from=None):
    q = randn((B, n, h_kv * g, d), seed, torch.bfloat16)
    k = randn((B, n, h_kv, d), seed + 1, torch.bfloat16)
    if k_from is not None:  # key j repeats key k_from[j]: exact score ties
        k = k[:, torch.as_tensor(k_from)]
    qc, kc = _codes(B, h_kv, n, n_c, a, b, seed + 2)
    offs, posts = zip(*(orc.build_index(kc[bb], n_c) for bb in range(B)))
    t = lambda x: torch.as_tensor(np.stack(x)).to(dev)
    return dict(q=q.to(dev), k=k.to(dev), qc=torch.as_tensor(qc).to(dev), off=t(offs), post=t(posts),
                qh=q, kh=k, qcn=qc, offn=np.stack(offs), postn=np.stack(posts), n_c=n_c, b=b)


def _select(c, top_k, mode, mask=None, **kw):
    from ssa_amd import kernels

    return kernels.select(c["q"], c["k"], c["qc"], c["off"], c["post"], c["b"], top_k, mode,
                          mask=mask, sorted=False, with_stats=True, **kw)


def _check_oracle(orc, c, got, top_k, mode, mask=None, rows=None):
    for bb in range(got.shape[0]):
        ref = orc.select(f32(c["qh"][bb]), f32(c["kh"][bb]), c["qcn"][bb], c["offn"][bb], c["postn"][bb],
                         c["b"], top_k, mode, mask, rows=rows, sorted=False)
        g = got[bb].cpu().numpy()
        np.testing.assert_array_equal(g if rows is None else g[rows], ref)


@pytest.mark.parametrize("d,g", [(128, 1), (128, 4), (128, 8), (128, 16), (64, 2), (64, 8), (64, 16)])
def test_screen_equals_block_path_and_oracle(dev, orc, d, g):
    """B=2, n=1500, h_kv=2, k=64, a=4 of N_c=64 codes, b=2: most rows have
    100-300 candidates, so most rows pass through the screen."""
    _say(f"select screen d={d} g={g}")
    from ssa_amd import _lib

    B, n, h_kv, top_k = 2, 1500, 2, 64
    c = _case(orc, dev, B, n, h_kv, g, d, 64, 4, 2, 100 + g + d)
    got, st = _select(c, top_k, _lib.MASK_CAUSAL)
    ref, st_ref = _select(c, top_k, _lib.MASK_CAUSAL, use_workspace=False)
    assert int((st[..., 0] > top_k).sum()) > B * h_kv * n // 2, "most rows must be screened"
    assert torch.equal(got, ref)
    assert torch.equal(st, st_ref)
    _check_oracle(orc, c, got, top_k, orc.MASK_CAUSAL)


@pytest.mark.parametrize("sorted_", [False, True])
def test_screen_xcd_slices_equal_block_path(dev, orc, sorted_):
    """B=2, h_kv=4: eight (batch, kv head) pairs, so each XCD's screen and pick
    waves walk their own slice of every shard's list; with the full workspace
    and with one that lists only some rows, the indices and stats equal the
    one-block-per-row kernel's, which the oracle pins on sampled rows."""
    _say(f"select screen xcd slices sorted={sorted_}")
    from ssa_amd import _lib, kernels

    B, n, h_kv, top_k = 2, 1400, 4, 64
    c = _case(orc, dev, B, n, h_kv, 2, 128, 64, 4, 2, 31)
    args = (c["q"], c["k"], c["qc"], c["off"], c["post"], c["b"], top_k, _lib.MASK_CAUSAL)
    ref, st_ref = kernels.select(*args, sorted=sorted_, with_stats=True, use_workspace=False)
    L = _lib.load()
    base = int(L.ssa_select_workspace_bytes(B, n, h_kv, 0))
    full = int(L.ssa_select_workspace_bytes(B, n, h_kv, top_k))
    for ws in (full, base + (full - base) // 5):
        got, st = kernels.select(*args, sorted=sorted_, with_stats=True, use_workspace=ws)
        assert int((st[..., 0] > top_k).sum()) > B * h_kv * n // 2, "most rows must be screened"
        assert torch.equal(got, ref), ws
        assert torch.equal(st, st_ref), ws
    if not sorted_:
        _check_oracle(orc, c, ref, top_k, orc.MASK_CAUSAL, rows=np.arange(0, n, 97))


@pytest.mark.parametrize("mode", ["none", "dense"])
def test_screen_mask_modes(dev, orc, mode):
    _say(f"select screen mask={mode}")
    from ssa_amd import _lib

    B, n, h_kv, top_k = 1, 1200, 2, 48
    c = _case(orc, dev, B, n, h_kv, 4, 128, 64, 4, 2, 7)
    mask = None
    if mode == "dense":
        gm = torch.Generator().manual_seed(8)
        mask = (torch.rand(n, n, generator=gm) < 0.7) | torch.eye(n, dtype=torch.bool)
    lm = _lib.MASK_NONE if mode == "none" else _lib.MASK_DENSE
    om = orc.MASK_NONE if mode == "none" else orc.MASK_DENSE
    got, st = _select(c, top_k, lm, mask=None if mask is None else mask.to(dev))
    ref, st_ref = _select(c, top_k, lm, mask=None if mask is None else mask.to(dev), use_workspace=False)
    assert torch.equal(got, ref) and torch.equal(st, st_ref)
    _check_oracle(orc, c, got, top_k, om, None if mask is None else mask.numpy().astype(np.uint8))


def test_screen_workspace_sizes(dev, orc):
    """The minimum workspace (no candidate lists: every heavy row exact), one that
    holds the lists of only some rows, the recommended size and a larger one:
    identical results."""
    _say("select screen workspace sizes")
    from ssa_amd import _lib

    B, n, h_kv, top_k = 2, 1500, 2, 64
    c = _case(orc, dev, B, n, h_kv, 4, 128, 64, 4, 2, 11)
    L = _lib.load()
    base = int(L.ssa_select_workspace_bytes(B, n, h_kv, 0))
    full = int(L.ssa_select_workspace_bytes(B, n, h_kv, top_k))
    ref, st_ref = _select(c, top_k, _lib.MASK_CAUSAL, use_workspace=False)
    for ws in (base, base + (full - base) // 16, base + (full - base) // 3, full, 2 * full):
        got, st = _select(c, top_k, _lib.MASK_CAUSAL, use_workspace=ws)
        assert torch.equal(got, ref), ws
        assert torch.equal(st, st_ref), ws


def test_screen_rows_longer_than_the_screen(dev, orc):
    """N_c=8, a=4, b=2: late rows have up to ~0.8 i candidates, beyond what one
    screened row holds (3072), so both the screen and the exact pass run; rows
    of 2049-3072 candidates take the pick pass's workspace reads (its LDS holds
    2048 scores per row)."""
    _say("select screen long rows")
    from ssa_amd import _lib

    B, n, h_kv, top_k = 1, 6000, 1, 256
    c = _case(orc, dev, B, n, h_kv, 4, 128, 8, 4, 2, 13)
    got, st = _select(c, top_k, _lib.MASK_CAUSAL)
    ref, st_ref = _select(c, top_k, _lib.MASK_CAUSAL, use_workspace=False)
    cand = st[..., 0]
    assert int((cand > 3072).sum()) > 0 and int(((cand > top_k) & (cand <= 3072)).sum()) > 0
    assert int(((cand > 2048) & (cand <= 3072)).sum()) > 0
    assert torch.equal(got, ref) and torch.equal(st, st_ref)
    rows = np.array([0, 1, 255, 256, 257, 3000, 3900, 4000, 5998, 5999])
    _check_oracle(orc, c, got, top_k, orc.MASK_CAUSAL, rows=rows)


@pytest.mark.parametrize("period", [2, 3, 40])
def test_screen_exact_ties(dev, orc, period):
    """Keys repeated with a period (key j = key j - j % period, or key j % period):
    equal scores, ranked by index.  Period 40 makes every row's candidates take
    at most 40 distinct scores, far more ties at the k-th score than the screen
    settles, so those rows go to the exact pass."""
    _say(f"select screen ties period={period}")
    from ssa_amd import _lib

    B, n, h_kv, top_k = 1, 1500, 2, 64
    src = np.arange(n) % period if period > 3 else np.arange(n) - np.arange(n) % period
    c = _case(orc, dev, B, n, h_kv, 4, 128, 64, 4, 2, 17, k_from=src)
    got, st = _select(c, top_k, _lib.MASK_CAUSAL)
    ref, st_ref = _select(c, top_k, _lib.MASK_CAUSAL, use_workspace=False)
    assert torch.equal(got, ref) and torch.equal(st, st_ref)
    _check_oracle(orc, c, got, top_k, orc.MASK_CAUSAL)


def test_screen_int64_output(dev, orc):
    _say("select screen int64")
    from ssa_amd import _lib

    c = _case(orc, dev, 1, 1000, 2, 8, 64, 64, 4, 2, 19)
    got32, _ = _select(c, 32, _lib.MASK_CAUSAL, index_dtype=torch.int32)
    got64, _ = _select(c, 32, _lib.MASK_CAUSAL, index_dtype=torch.int64)
    assert got64.dtype == torch.int64 and torch.equal(got32.to(torch.int64), got64)


@pytest.mark.parametrize("sorted_,ws", [(False, True), (False, False), (True, True)])
def test_select_row_order(dev, orc, sorted_, ws):
    """Rows processed in query order (grouped by smallest code) or reversed: the same
    indices and stats.  An order entry outside [0, n) skips its slot, so the one
    query it displaced is not written and every other row is unchanged."""
    _say(f"select row order sorted={sorted_} ws={ws}")
    from ssa_amd import _lib, kernels

    B, n, h_kv, top_k = 2, 1500, 2, 64
    c = _case(orc, dev, B, n, h_kv, 4, 128, 64, 4, 2, 23)
    kw = dict(sorted=sorted_, with_stats=True, use_workspace=ws)
    args = (c["q"], c["k"], c["qc"], c["off"], c["post"], c["b"], top_k, _lib.MASK_CAUSAL)
    ref, st_ref = kernels.select(*args, **kw)
    order = kernels.query_order(c["qc"], c["n_c"])
    for o in (order, order.flip(-1).contiguous()):
        got, st = kernels.select(*args, row_order=o, **kw)
        assert torch.equal(got, ref) and torch.equal(st, st_ref)
    bad = order.clone()
    skipped = int(bad[1, 0, 700])
    bad[1, 0, 700] = n
    got = kernels.select(*args, row_order=bad, sorted=sorted_, use_workspace=ws)
    keep = torch.ones(n, dtype=torch.bool, device=dev)
    keep[skipped] = False
    assert torch.equal(got[0], ref[0]) and torch.equal(got[1, :, 1], ref[1, :, 1])
    assert torch.equal(got[1, keep, 0], ref[1, keep, 0])


@pytest.mark.parametrize("d,g,top_k,n,i64", [
    (128, 4, 512, 1500, False),
    (64, 8, 1024, 2600, True),
    (128, 1, 100, 900, True),
    (64, 2, 40, 700, False),
])
def test_select_score_order_sort_pass(dev, orc, d, g, top_k, n, i64):
    """Score order through the workspace (index-order passes, then the per-row
    rescore-and-sort pass: key rows in registers, a register bitonic network)
    equals the one-block-per-row kernel bit for bit: rows of 1 to top_k
    selected keys (every slot count per lane, 64 to 1024 sorted slots), exact
    score ties (repeated keys), int32 and int64 indices."""
    _say(f"select score order d={d} g={g} top_k={top_k} n={n} i64={i64}")
    from ssa_amd import _lib, kernels

    rng = np.random.default_rng(31)
    k_from = np.arange(n)
    dup = rng.choice(n, n // 5, replace=False)
    k_from[dup] = rng.integers(0, n, n // 5)  # a fifth of the keys repeat another key
    c = _case(orc, dev, 1, n, 2, g, d, 32, 6, 3, 37 + g, k_from=k_from)
    args = (c["q"], c["k"], c["qc"], c["off"], c["post"], c["b"], top_k, _lib.MASK_CAUSAL)
    dt = torch.int64 if i64 else torch.int32
    ref, st_ref = kernels.select(*args, sorted=True, with_stats=True, use_workspace=False, index_dtype=dt)
    got, st = kernels.select(*args, sorted=True, with_stats=True, use_workspace=True, index_dtype=dt)
    assert torch.equal(st, st_ref)
    C = st[..., 0]
    assert int(C.min()) <= 1 and int((C >= top_k).sum()) > 0, "short and full rows"
    assert torch.equal(got, ref)
