"""CPU oracle for the SSA forward hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or as the timed
CPU baseline).  The product package ``ssa_amd`` never imports it.

Two layers:

* ``C`` -- ctypes bindings of ``libssa_oracle.so`` (``ssa_oracle.c``): the
  canonical fp32 restatement whose selections the HIP kernels must match bit
  for bit.  Each function cites the reference lines it follows.
* Independent checks that pin the C restatement (``brute_*`` and ``np_*``):
  pure-Python loops over the reference's set definitions and float64 numpy
  restatements, used only by the tests.

Every array crossing into C is a contiguous numpy array; bf16 tensors are
widened to float32 exactly by the caller (``to_f32``).
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libssa_oracle.so")

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_flt = ctypes.c_float
_dbl = ctypes.c_double

_lib = None


def build() -> str:
    """Compile libssa_oracle.so with the committed Makefile."""
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
    L = ctypes.CDLL(LIB_PATH)
    L.oracle_version.restype = _int
    L.oracle_set_threads.argtypes = [_int]
    L.oracle_get_threads.restype = _int
    L.oracle_score_key.argtypes = [_flt]
    L.oracle_score_key.restype = ctypes.c_uint32
    L.oracle_normalize.argtypes = [_f32p, _i64, _int, _f32p]
    L.oracle_route_vectors.argtypes = [_f32p, _i64, _int, _int, _int, _f32p, _int, _f32p]
    L.oracle_code_topk.argtypes = [_f32p, _int, _i64, _f32p, _int, _int, _flt, _int, _i32p, _vp]
    L.oracle_build_index.argtypes = [_i32p, _int, _i64, _int, _int, _i32p, _i32p]
    L.oracle_select.argtypes = [
        _f32p, _f32p, _i64, _int, _int, _int, _i32p, _int, _i32p, _i32p, _int, _int, _int, _int,
        _vp, _flt, _int, _vp, _i64, _i64p, _vp, _vp,
    ]
    L.oracle_sparse_attention.argtypes = [
        _f32p, _f32p, _f32p, _i64, _int, _int, _int, _i64p, _int, _dbl, _int, _vp, _i64, _f64p,
    ]
    L.oracle_dense_attention.argtypes = [
        _f32p, _f32p, _f32p, _i64, _int, _int, _int, _dbl, _int, _f64p,
    ]
    L.oracle_sparse_attention_backward.argtypes = [
        _f32p, _f32p, _f32p, _i64, _int, _int, _int, _i64p, _int, _dbl, _int, _f64p, _f64p,
        _f64p, _f64p,
    ]
    _lib = L
    return L


def set_threads(t: int) -> None:
    lib().oracle_set_threads(int(t))


def get_threads() -> int:
    return int(lib().oracle_get_threads())


def to_f32(x) -> np.ndarray:
    """torch tensor (any float dtype, any device) or array -> contiguous float32 numpy."""
    try:
        import torch

        if isinstance(x, torch.Tensor):
            return np.ascontiguousarray(x.detach().to("cpu", torch.float32).numpy())
    except ImportError:  # pragma: no cover
        pass
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32))


def _c(a, dtype):
    return np.ascontiguousarray(np.asarray(a, dtype=dtype))


def score_div_for(d: int) -> float:
    """fp32 divisor the reference uses for rescoring: head_dim**0.5 (ssa/router.py:182)."""
    return float(np.float32(d ** 0.5))


def bf16_round(a) -> np.ndarray:
    """float32 values rounded to the nearest bf16 (ties to even), kept as float32."""
    a = np.asarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = (u & 0xFFFFFFFF).astype(np.uint32).view(np.float32).copy()
    out[np.isnan(a)] = np.nan
    return out


def rope(x, cos, sin, rot: int, by_head: bool, round_bf16: bool = False,
         inverse: bool = False) -> np.ndarray:
    """Rotary embedding in float32 numpy (the arithmetic ssa_rope must match bit for bit).

    Follows apply_rope / _rotate_half (ssa/utils.py:7-48) as SSAAttention calls it
    on [n, heads, d] (ssa/ssa_layer.py:115-117: rot = d/2, angle row = head, only
    x[..., :d/2] rotates) and Hugging Face's apply_rotary_pos_emb in the Qwen2
    path (training/train_qwen.py:134-135: rot = d, angle row = position):
    y = x * cos + rotate_half(x) * sin over features j < rot, pairs (j, j + rot/2),
    features >= rot unchanged.  Three rounded float32 ops, no fusion; with
    ``round_bf16`` (bf16 x and bf16 tables in torch) each op's result rounds to
    bf16.  ``inverse`` is the transpose of the rotation.

    x: [B, n, h, d]; cos/sin: [rows, w] or [B or 1, rows, w] with w >= rot."""
    x = np.asarray(x, dtype=np.float32)
    cos = np.asarray(cos, dtype=np.float32)
    sin = np.asarray(sin, dtype=np.float32)
    if cos.ndim == 2:
        cos, sin = cos[None], sin[None]
    B, n, h, d = x.shape
    r = rot // 2
    rows = h if by_head else n
    c = cos[:, :rows, :rot]
    s = sin[:, :rows, :rot]
    # broadcast the table rows onto [B, n, h, rot]
    c = c[:, None, :, :] if by_head else c[:, :, None, :]
    s = s[:, None, :, :] if by_head else s[:, :, None, :]
    rnd = bf16_round if round_bf16 else (lambda v: v)
    x1, x2 = x[..., :r], x[..., r:rot]
    c1, c2, s1, s2 = c[..., :r], c[..., r:], s[..., :r], s[..., r:]
    if not inverse:
        y1 = rnd(rnd(x1 * c1) + rnd((-x2) * s1))
        y2 = rnd(rnd(x2 * c2) + rnd(x1 * s2))
    else:
        y1 = rnd(rnd(x1 * c1) + rnd(x2 * s2))
        y2 = rnd(rnd(x2 * c2) + rnd((-x1) * s1))
    out = x.copy()
    out[..., :r] = y1
    out[..., r:rot] = y2
    return out


# ----------------------------------------------------------------- C layer

def normalize(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty_like(x)
    d_s = x.shape[-1]
    lib().oracle_normalize(x, x.size // d_s if d_s else 0, d_s, out)
    return out


def route_vectors(x, w, group: int) -> np.ndarray:
    """x [n, h_in, d], w [d_s, d] -> [h_in/group, n, d_s] (ssa/router.py:102-117)."""
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    n, h_in, d = x.shape
    d_s = w.shape[0]
    out = np.empty((h_in // group, n, d_s), np.float32)
    lib().oracle_route_vectors(x, n, h_in, group, d, w, d_s, out)
    return out


def code_topk(xhat, chat, top: int, temperature: float = 1.0, with_scores: bool = False):
    """xhat [h, rows, d_s], chat [h, n_c, d_s] -> codes [h, rows, top] int32
    (ssa/router.py:121-130,141)."""
    xhat = _c(xhat, np.float32)
    chat = _c(chat, np.float32)
    h, rows, d_s = xhat.shape
    n_c = chat.shape[1]
    codes = np.empty((h, rows, top), np.int32)
    scores = np.empty((h, rows, top), np.float32) if with_scores else None
    lib().oracle_code_topk(
        xhat, h, rows, chat, n_c, d_s, float(temperature), top, codes,
        scores.ctypes.data if with_scores else None,
    )
    return (codes, scores) if with_scores else codes


def build_index(k_codes, n_c: int):
    """k_codes [h, n, b] -> offsets [h, n_c+1], postings [h, n*b]."""
    kc = _c(k_codes, np.int32)
    h, n, b = kc.shape
    offsets = np.empty((h, n_c + 1), np.int32)
    postings = np.empty((h, n * b), np.int32)
    lib().oracle_build_index(kc, h, n, b, n_c, offsets, postings)
    return offsets, postings


MASK_NONE, MASK_CAUSAL, MASK_DENSE = 0, 1, 2


def select(q, k, q_codes, offsets, postings, b: int, top_k: int, mask_mode: int = MASK_CAUSAL,
           mask=None, score_div: Optional[float] = None, rows=None, with_stats: bool = False,
           sorted: bool = True):
    """Stage (c) for one batch element (ssa/router.py:151-259).

    q [n, h_q, d], k [n, h_kv, d] float32; q_codes [h_kv, n, a]; returns int64
    [len(rows) or n, h_kv, top_k] (+ per-row candidate and raw-posting counts).
    """
    q = _c(q, np.float32)
    k = _c(k, np.float32)
    n, h_q, d = q.shape
    h_kv = k.shape[1]
    qc = _c(q_codes, np.int32)
    a = qc.shape[-1]
    off = _c(offsets, np.int32)
    post = _c(postings, np.int32)
    n_c = off.shape[-1] - 1
    if score_div is None:
        score_div = score_div_for(d)
    mk = None
    if mask_mode == MASK_DENSE:
        mk = _c(mask, np.uint8)
        assert mk.shape == (n, n)
    if rows is not None:
        rows_a = _c(rows, np.int64)
        nr = rows_a.shape[0]
    else:
        rows_a, nr = np.zeros(1, np.int64), n
    out = np.empty((nr, h_kv, top_k), np.int64)
    n_cand = np.empty((nr, h_kv), np.int32)
    n_raw = np.empty((nr, h_kv), np.int32)
    lib().oracle_select(
        q, k, n, h_q, h_kv, d, qc, a, off, post, n_c, b, top_k, mask_mode,
        mk.ctypes.data if mk is not None else None, float(score_div), int(bool(sorted)),
        rows_a.ctypes.data if rows is not None else None, nr, out,
        n_cand.ctypes.data, n_raw.ctypes.data,
    )
    return (out, n_cand, n_raw) if with_stats else out


def sparse_attention(q, k, v, idx, scale=None, causal: bool = False, rows=None) -> np.ndarray:
    """Stage (d) for one batch element in float64 (ssa/attention.py:12-115).

    idx is [n, h_kv, kk], or [len(rows), h_kv, kk] aligned with ``rows``."""
    q = _c(q, np.float32)
    k = _c(k, np.float32)
    v = _c(v, np.float32)
    ix = _c(idx, np.int64)
    n, h_q, d = q.shape
    h_kv = k.shape[1]
    kk = ix.shape[-1]
    scale = (d ** 0.5) if scale is None else float(scale)
    if rows is not None:
        rows_a = _c(rows, np.int64)
        nr = rows_a.shape[0]
    else:
        rows_a, nr = np.zeros(1, np.int64), n
    out = np.empty((nr, h_q, d), np.float64)
    lib().oracle_sparse_attention(
        q, k, v, n, h_q, h_kv, d, ix, kk, scale, int(bool(causal)),
        rows_a.ctypes.data if rows is not None else None, nr, out,
    )
    return out


def sparse_attention_backward(q, k, v, idx, dout, scale=None, causal: bool = False):
    """Gradients (dq, dk, dv) of ``sparse_attention`` in float64 for one batch
    element, given the output gradient ``dout`` [n, h_q, d] (the autograd
    backward of ssa/attention.py:64-113).  Indices must lie in [0, n)."""
    q = _c(q, np.float32)
    k = _c(k, np.float32)
    v = _c(v, np.float32)
    ix = _c(idx, np.int64)
    do = _c(dout, np.float64)
    n, h_q, d = q.shape
    h_kv = k.shape[1]
    kk = ix.shape[-1]
    scale = (d ** 0.5) if scale is None else float(scale)
    dq = np.empty((n, h_q, d), np.float64)
    dk = np.empty((n, h_kv, d), np.float64)
    dv = np.empty((n, h_kv, d), np.float64)
    lib().oracle_sparse_attention_backward(q, k, v, n, h_q, h_kv, d, ix, kk, scale,
                                           int(bool(causal)), do, dq, dk, dv)
    return dq, dk, dv


def dense_attention(q, k, v, causal: bool = False, scale=None) -> np.ndarray:
    """Dense SDPA in float64 (ssa/attention.py:118-158)."""
    q = _c(q, np.float32)
    k = _c(k, np.float32)
    v = _c(v, np.float32)
    n, h_q, d = q.shape
    h_kv = k.shape[1]
    scale = (d ** 0.5) if scale is None else float(scale)
    out = np.empty((n, h_q, d), np.float64)
    lib().oracle_dense_attention(q, k, v, n, h_q, h_kv, d, scale, int(bool(causal)), out)
    return out


def router_forward(q, k, w_qr, w_kr, codebook, a: int, b: int, top_k: int,
                   mask_mode: int = MASK_CAUSAL, mask=None, temperature: float = 1.0,
                   rows=None, with_stats: bool = False, sorted: bool = True):
    """Whole CodebookRouter.forward for one batch element (ssa/router.py:73-149)."""
    q = _c(q, np.float32)
    k = _c(k, np.float32)
    n, h_q, d = q.shape
    h_kv = k.shape[1]
    g = h_q // h_kv
    qhat = route_vectors(q, w_qr, g)
    khat = route_vectors(k, w_kr, 1)
    chat = normalize(codebook)
    q_codes = code_topk(qhat, chat, a, temperature)
    k_codes = code_topk(khat, chat, b, temperature)
    offsets, postings = build_index(k_codes, chat.shape[1])
    res = select(q, k, q_codes, offsets, postings, b, top_k, mask_mode, mask,
                 rows=rows, with_stats=with_stats, sorted=sorted)
    extras = dict(qhat=qhat, khat=khat, chat=chat, q_codes=q_codes, k_codes=k_codes,
                  offsets=offsets, postings=postings)
    return res, extras


# --------------------------------------------- independent checks (pinning)

def np_route_vectors64(x, w, group: int) -> np.ndarray:
    """float64 restatement of route_vectors (projection, GQA mean, normalize)."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    n, h_in, d = x.shape
    proj = x @ w.T  # [n, h_in, d_s]
    m = proj.reshape(n, h_in // group, group, -1).mean(axis=2)
    nrm = np.maximum(np.sqrt((m * m).sum(-1, keepdims=True)), 1e-12)
    return np.transpose(m / nrm, (1, 0, 2))


def brute_candidate_mask(q_codes, k_codes, causal: bool) -> np.ndarray:
    """Set definition of ssa/router.py:224-235 with the reference's broadcast compare
    (:251-257) written as plain loops: mask[h, i, j] = any(q_codes[h,i,:] == k_codes[h,j,:])."""
    h, n, a = q_codes.shape
    out = np.zeros((h, n, n), bool)
    for hh in range(h):
        for i in range(n):
            qs = set(int(c) for c in q_codes[hh, i])
            for j in range(n):
                if causal and j > i:
                    continue
                if qs.intersection(int(c) for c in k_codes[hh, j]):
                    out[hh, i, j] = True
    return out


def brute_select(q, k, q_codes, k_codes, top_k: int, causal: bool) -> np.ndarray:
    """Pure-Python restatement of ssa/router.py:177-214 for tiny n.

    Scores are the float64 mean over the group of q.k/sqrt(d); selection sorts
    (score desc, index asc); filler is the lowest non-candidate indices; k > n
    pads zeros.  Returns [n, h_kv, top_k] int64.  Ties closer than float32
    resolution may order differently from the fp32 oracle; callers compare
    with that in mind.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    n, h_q, d = q.shape
    h_kv = k.shape[1]
    g = h_q // h_kv
    mask = brute_candidate_mask(q_codes, k_codes, causal)
    out = np.zeros((n, h_kv, top_k), np.int64)
    k_eff = min(top_k, n)
    for h in range(h_kv):
        for i in range(n):
            cands = [j for j in range(n) if mask[h, i, j]]
            sc = {j: float(np.mean([q[i, h * g + gg] @ k[j, h] / np.sqrt(d) for gg in range(g)]))
                  for j in cands}
            order = sorted(cands, key=lambda j: (-sc[j], j))[:k_eff]
            fill = [j for j in range(n) if j not in sc][: k_eff - len(order)]
            row = order + fill
            out[i, h, : len(row)] = row
    return out


def np_sparse_attention64(q, k, v, idx, scale=None, causal: bool = False) -> np.ndarray:
    """float64 numpy restatement of ssa/attention.py:64-113 (gather, einsum, softmax)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    idx = np.asarray(idx, np.int64)
    n, h_q, d = q.shape
    h_kv = k.shape[1]
    g = h_q // h_kv
    scale = d ** 0.5 if scale is None else scale
    kg = k[idx, np.arange(h_kv)[None, :, None]]  # [n, h_kv, kk, d]
    vg = v[idx, np.arange(h_kv)[None, :, None]]
    qg = q.reshape(n, h_kv, g, d)
    lg = np.einsum("nhgd,nhkd->nhgk", qg, kg) / scale
    if causal:
        fut = idx[:, :, None, :] > np.arange(n)[:, None, None, None]
        lg = np.where(fut, -np.inf, lg)
    mx = lg.max(-1, keepdims=True)
    mx = np.where(np.isfinite(mx), mx, 0.0)
    p = np.exp(lg - mx)
    den = p.sum(-1, keepdims=True)
    p = np.where(den > 0, p / np.where(den > 0, den, 1.0), 0.0)
    return np.einsum("nhgk,nhkd->nhgd", p, vg).reshape(n, h_q, d)


# ---------------------------------------------------------------------------
# Block-granular variant (ssa/triton_kernel.py).  numpy restatements; the
# product kernels are ssa_block_indices / ssa_block_sparse_attention.


def block_indices(indices, block_size: int, n_k_blocks: Optional[int] = None) -> np.ndarray:
    """Key blocks per query block (ssa/triton_kernel.py:226-294): token indices
    [n, h, top_k] -> int64 [ceil(n / bs), h, n_k_blocks] (default min(top_k,
    blocks)).  Key j is in block j // bs (:259); rows past n are zero-padded
    (:262-268), so each adds top_k references to block 0; a query block's
    counts come from its bs x top_k entries (:287-288); the n_k_blocks most
    referenced blocks are kept (:291-292), equal counts by lower block id
    (torch.topk leaves that order open)."""
    idx = np.asarray(indices, dtype=np.int64)
    n, h, k = idx.shape
    nb = (n + block_size - 1) // block_size
    nkb = min(k, nb) if n_k_blocks is None else n_k_blocks
    blk = idx // block_size
    pad = nb * block_size - n
    if pad:
        blk = np.concatenate([blk, np.zeros((pad, h, k), np.int64)], axis=0)
    blk = blk.reshape(nb, block_size, h, k)
    out = np.empty((nb, h, nkb), np.int64)
    ids = np.arange(nb)
    for bq in range(nb):
        for hh in range(h):
            cnt = np.bincount(blk[bq, :, hh, :].ravel(), minlength=nb)
            out[bq, hh] = np.lexsort((ids, -cnt))[:nkb]
    return out


def brute_block_indices(indices, block_size: int, n_k_blocks: int) -> np.ndarray:
    """The same ranking from pure-Python counting over (query block, head):
    an independent check of ``block_indices``."""
    idx = np.asarray(indices, dtype=np.int64)
    n, h, k = idx.shape
    nb = (n + block_size - 1) // block_size
    out = np.empty((nb, h, n_k_blocks), np.int64)
    for bq in range(nb):
        for hh in range(h):
            counts = {c: 0 for c in range(nb)}
            for r in range(bq * block_size, (bq + 1) * block_size):
                for t in range(k):
                    counts[int(idx[r, hh, t]) // block_size if r < n else 0] += 1
            ranked = sorted(counts, key=lambda c: (-counts[c], c))
            out[bq, hh] = ranked[:n_k_blocks]
    return out


def block_sparse_attention64(q, k, v, blocks, block_size: int, scale_div=None) -> np.ndarray:
    """float64 causal attention of row i over the keys of the blocks listed for
    block i // bs (ssa/triton_kernel.py:84-130 with an exact, normalised
    softmax): keys past n are skipped; a row with no key gives zeros."""
    q, k, v = (np.asarray(x, np.float64) for x in (q, k, v))
    blocks = np.asarray(blocks, np.int64)
    n, h_q, d = q.shape
    h_kv = k.shape[1]
    g = h_q // h_kv
    sd = np.sqrt(d) if scale_div is None else scale_div
    out = np.zeros_like(q)
    for i in range(n):
        for hq in range(h_q):
            hh = hq // g
            keys = (blocks[i // block_size, hh][:, None] * block_size + np.arange(block_size)[None, :]).ravel()
            keys = keys[(keys < n) & (keys <= i)]
            if keys.size == 0:
                continue
            s = k[keys, hh] @ q[i, hq] / sd
            p = np.exp(s - s.max())
            out[i, hq] = (p / p.sum()) @ v[keys, hh]
    return out
