"""Tensor-level wrappers over the libssa_hip entry points (one per C-ABI call).

All sequence tensors are batched ``[B, n, heads, d]`` views whose last
dimension is contiguous; other strides are passed through, so transposed
layouts such as HF's ``[B, heads, n, d]`` (permuted) need no copy.  Outputs and
workspaces come from the PyTorch caching allocator on the input's device, and
every call is enqueued on the current stream without synchronising.
"""

from __future__ import annotations

import math
from typing import NamedTuple, Optional, Tuple, Union

import torch

from . import _lib
from ._lib import call, ptr, stream_of


def _check_rows(x: torch.Tensor, name: str) -> None:
    if x.dim() != 4:
        raise ValueError(f"{name} must be [B, n, heads, d], got shape {tuple(x.shape)}")
    if x.stride(-1) != 1:
        raise ValueError(f"{name} must have a contiguous last dimension")


def _f32c(t: torch.Tensor) -> torch.Tensor:
    return t.detach().to(torch.float32).contiguous()


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, rot: int, by_head: bool,
         inverse: bool = False, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Rotary embedding of ``x`` [B, n, h, d] (ssa_rope): features j < rot rotate in
    pairs (j, j + rot/2) as ``x * cos + rotate_half(x) * sin``; the rest pass through.

    ``cos``/``sin`` are ``[rows, >= rot]`` (one table) or ``[B, rows, >= rot]``
    with a contiguous last dimension; the angle row is the head index
    (``by_head``, SSAAttention's apply_rope call) or the token position (Hugging
    Face).  ``inverse`` applies the transpose (the gradient).  ``out`` defaults
    to a new contiguous tensor of x's dtype; ``out is x`` rotates in place."""
    _check_rows(x, "x")
    _lib.require_device(x, cos, sin)
    B, n, h, d = x.shape
    if cos.shape != sin.shape or cos.dtype != sin.dtype:
        raise ValueError("cos and sin tables must have the same shape and dtype")
    if cos.stride(-1) != 1 or sin.stride(-1) != 1 or cos.stride() != sin.stride():
        cos, sin = cos.contiguous(), sin.contiguous()
    if cos.dim() == 2:
        t_sb, t_sr, rows = 0, cos.stride(0), cos.shape[0]
    elif cos.dim() == 3 and cos.shape[0] in (1, B):
        t_sb = cos.stride(0) if cos.shape[0] == B else 0
        t_sr, rows = cos.stride(1), cos.shape[1]
    else:
        raise ValueError(f"rope tables must be [rows, w] or [B, rows, w], got {tuple(cos.shape)}")
    if cos.shape[-1] < rot:
        raise ValueError(f"rope tables are {cos.shape[-1]} wide, rot={rot} needs that many")
    if out is None:
        out = torch.empty((B, n, h, d), device=x.device, dtype=x.dtype)
    call("ssa_rope", ptr(x), _lib.elem_dtype(x), B, n, h, d, x.stride(0), x.stride(1), x.stride(2),
         ptr(cos), ptr(sin), _lib.elem_dtype(cos), t_sb, t_sr, rows, int(rot),
         _lib.ROPE_BY_HEAD if by_head else _lib.ROPE_BY_POSITION, int(bool(inverse)),
         ptr(out), _lib.elem_dtype(out), out.stride(0), out.stride(1), out.stride(2), stream_of(x))
    return out


def route_vectors(x: torch.Tensor, w: torch.Tensor, group: int) -> torch.Tensor:
    """normalize(mean_g(x . w^T)) -> float32 [B, heads/group, n, d_s] (ssa/router.py:102-117)."""
    _check_rows(x, "x")
    _lib.require_device(x, w)
    B, n, h_in, d = x.shape
    w = _f32c(w)
    d_s = w.shape[0]
    out = torch.empty((B, h_in // group, n, d_s), device=x.device, dtype=torch.float32)
    call("ssa_route_vectors", ptr(x), _lib.elem_dtype(x), B, n, h_in, group, d,
         x.stride(0), x.stride(1), x.stride(2), ptr(w), d_s, ptr(out), stream_of(x))
    return out


def normalize_rows(x: torch.Tensor) -> torch.Tensor:
    """Row-wise F.normalize of a float32 matrix (ssa/router.py:118)."""
    _lib.require_device(x)
    x = _f32c(x)
    out = torch.empty_like(x)
    d_s = x.shape[-1]
    call("ssa_normalize_rows", ptr(x), x.numel() // d_s, d_s, ptr(out), stream_of(x))
    return out


def code_topk(xhat: torch.Tensor, chat: torch.Tensor, top: int,
              temperature: float = 1.0, exhaustive: bool = False) -> torch.Tensor:
    """Top-`top` codes per row, int32 [B, h, rows, top] (ssa/router.py:121-130,141).

    ``exhaustive=True`` skips the matrix-core screen and scores every code in
    fp32 (same result; used to cross-check the screen)."""
    _lib.require_device(xhat, chat)
    xhat = xhat.contiguous()
    chat = chat.contiguous()
    B, h, rows, d_s = xhat.shape
    n_c = chat.shape[1]
    codes = torch.empty((B, h, rows, top), device=xhat.device, dtype=torch.int32)
    ws, ws_bytes = None, 0
    if not exhaustive:
        ws_bytes = int(_lib.load().ssa_code_topk_workspace_bytes(B, h, rows, n_c))
        ws = torch.empty(max(ws_bytes, 1), device=xhat.device, dtype=torch.uint8)
    call("ssa_code_topk", ptr(xhat), B, h, rows, ptr(chat), n_c, d_s, float(temperature), top,
         ptr(codes), ptr(ws), ws_bytes, stream_of(xhat))
    return codes


def route_codes(q: torch.Tensor, k: torch.Tensor, w_qr: torch.Tensor, w_kr: torch.Tensor,
                codebook: torch.Tensor, a: int, b: int,
                temperature: float = 1.0) -> Tuple[torch.Tensor, torch.Tensor]:
    """Stage (a): (q_codes int32 [B,h_kv,n,a], k_codes int32 [B,h_kv,n,b])."""
    _check_rows(q, "q")
    _check_rows(k, "k")
    _lib.require_device(q, k, w_qr, w_kr, codebook)
    if q.dtype != k.dtype:
        raise TypeError(f"q and k must share a dtype ({q.dtype} vs {k.dtype})")
    B, n, h_q, d = q.shape
    h_kv = k.shape[2]
    w_qr, w_kr, codebook = _f32c(w_qr), _f32c(w_kr), _f32c(codebook)
    n_c, d_s = codebook.shape[1], codebook.shape[2]
    dev = q.device
    q_codes = torch.empty((B, h_kv, n, a), device=dev, dtype=torch.int32)
    k_codes = torch.empty((B, h_kv, n, b), device=dev, dtype=torch.int32)
    ws_bytes = _lib.load().ssa_route_workspace_bytes(B, n, h_kv, n_c, d_s)
    ws = torch.empty(max(int(ws_bytes), 1), device=dev, dtype=torch.uint8)
    call("ssa_route_codes", ptr(q), ptr(k), _lib.elem_dtype(q), B, n, h_q, h_kv, d,
         q.stride(0), q.stride(1), q.stride(2), k.stride(0), k.stride(1), k.stride(2),
         ptr(w_qr), ptr(w_kr), ptr(codebook), d_s, n_c, a, b, float(temperature),
         ptr(q_codes), ptr(k_codes), ptr(ws), ws_bytes, stream_of(q))
    return q_codes, k_codes


def build_index(k_codes: torch.Tensor, n_c: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Stage (b): offsets int32 [B,h,n_c+1], postings int32 [B,h,n*b] (ascending per bucket)."""
    _lib.require_device(k_codes)
    k_codes = k_codes.contiguous()
    B, h, n, b = k_codes.shape
    dev = k_codes.device
    offsets = torch.empty((B, h, n_c + 1), device=dev, dtype=torch.int32)
    postings = torch.empty((B, h, n * b), device=dev, dtype=torch.int32)
    ws_bytes = _lib.load().ssa_index_workspace_bytes(B, n, h, b, n_c)
    ws = torch.empty(max(int(ws_bytes), 1), device=dev, dtype=torch.uint8)
    call("ssa_build_index", ptr(k_codes), B, n, h, b, n_c, ptr(offsets), ptr(postings), ptr(ws),
         ws_bytes, stream_of(k_codes))
    return offsets, postings


def query_order(q_codes: torch.Tensor, n_c: int) -> torch.Tensor:
    """Query positions per (batch, kv head) sorted stably by their smallest code
    ``q_codes.min(-1)``: int32 [B, h, n], a processing order for sparse_attention
    (rows sharing that code share its bucket's keys)."""
    _lib.require_device(q_codes)
    q_codes = q_codes.contiguous()
    B, h, n, a = q_codes.shape
    order = torch.empty((B, h, n), device=q_codes.device, dtype=torch.int32)
    ws_bytes = _lib.load().ssa_query_order_workspace_bytes(B, n, h, n_c)
    ws = torch.empty(max(int(ws_bytes), 1), device=q_codes.device, dtype=torch.uint8)
    call("ssa_query_order", ptr(q_codes), B, n, h, a, n_c, ptr(order), ptr(ws), ws_bytes,
         stream_of(q_codes))
    return order


def select(q: torch.Tensor, k: torch.Tensor, q_codes: torch.Tensor, offsets: torch.Tensor,
           postings: torch.Tensor, b: int, top_k: int, mask_mode: int = _lib.MASK_CAUSAL,
           mask: Optional[torch.Tensor] = None, score_div: Optional[float] = None,
           index_dtype: torch.dtype = torch.int64,
           with_stats: bool = False, sorted: bool = True, use_workspace: Union[bool, int] = True,
           row_order: Optional[torch.Tensor] = None, q_pos0: Optional[int] = None,
           row_prefix: Optional[torch.Tensor] = None):
    """Stage (c): candidate indices [B, n_q, h_kv, top_k] (ssa/router.py:151-214).

    ``q`` and ``q_codes`` may hold fewer rows (n_q) than ``k`` has keys (n): a
    block of queries at key positions ``q_pos0 .. q_pos0 + n_q - 1`` (default:
    the last n_q positions, as in decoding against a cache).  With n_q = n this
    is the whole sequence.

    ``mask`` (MASK_DENSE) is a bool/uint8 ``[n, n]`` or ``[B, n, n]`` tensor with a
    contiguous last dimension.  ``with_stats`` also returns int32 ``[B, h_kv, n, 2]``
    (unique candidates, postings read inside the mask window) per row.
    ``sorted=False`` lists the same selected set in ascending index order (then
    the same filler).  ``use_workspace=False`` runs the one-block-per-row kernel
    for every row; an int gives the workspace size in bytes instead of the
    recommended ``ssa_select_workspace_bytes(B, n, h_kv, top_k)`` (same results).
    ``row_order`` (int32 [B, h_kv, n], a permutation of 0..n-1 per head, e.g.
    ``query_order``) only sets the order in which rows are processed.
    ``row_prefix`` (int32 [B, h_kv, n_q], written): X per row, the key prefix
    [0, X) its indices hold exactly once (the lowest-key filler), for
    ``sparse_attention``'s dense-prefix pass.
    """
    _check_rows(q, "q")
    _check_rows(k, "k")
    _lib.require_device(q, k, q_codes, offsets, postings, mask)
    B, n_q, h_q, d = q.shape
    n = k.shape[1]
    if q_pos0 is None:
        q_pos0 = n - n_q
    h_kv = k.shape[2]
    a = q_codes.shape[-1]
    n_c = offsets.shape[-1] - 1
    q_codes, offsets, postings = q_codes.contiguous(), offsets.contiguous(), postings.contiguous()
    if score_div is None:
        score_div = float(torch.tensor(d ** 0.5, dtype=torch.float32))
    m_sb = m_si = 0
    if mask_mode == _lib.MASK_DENSE:
        if mask is None:
            raise ValueError("MASK_DENSE needs a mask tensor")
        if mask.dtype == torch.bool:
            mask = mask.view(torch.uint8)
        if mask.stride(-1) != 1:
            mask = mask.contiguous()
        if mask.dim() == 2:
            m_sb, m_si = 0, mask.stride(0)
        else:
            m_sb, m_si = mask.stride(0), mask.stride(1)
    if row_order is not None:
        _lib.require_device(row_order)
        if row_order.dtype != torch.int32 or tuple(row_order.shape) != (B, h_kv, n_q):
            raise ValueError(f"row_order must be int32 [{B}, {h_kv}, {n_q}]")
        row_order = row_order.contiguous()
    if row_prefix is not None:
        _lib.require_device(row_prefix)
        if (row_prefix.dtype != torch.int32 or tuple(row_prefix.shape) != (B, h_kv, n_q)
                or not row_prefix.is_contiguous()):
            raise ValueError(f"row_prefix must be a contiguous int32 [{B}, {h_kv}, {n_q}] tensor")
    out = torch.empty((B, n_q, h_kv, top_k), device=q.device, dtype=index_dtype)
    stats = torch.empty((B, h_kv, n_q, 2), device=q.device, dtype=torch.int32) if with_stats else None
    ws_bytes, ws = 0, None
    if use_workspace is True:
        ws_bytes = int(_lib.load().ssa_select_workspace_bytes(B, n_q, h_kv, top_k))
    elif use_workspace is not False:
        ws_bytes = int(use_workspace)
    if ws_bytes > 0:
        ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8)
    call("ssa_select_block", ptr(q), ptr(k), _lib.elem_dtype(q), B, n, n_q, q_pos0, h_q, h_kv, d,
         q.stride(0), q.stride(1), q.stride(2), k.stride(0), k.stride(1), k.stride(2),
         ptr(q_codes), a, ptr(offsets), ptr(postings), n_c, b, top_k, mask_mode, ptr(mask),
         m_sb, m_si, float(score_div), int(bool(sorted)), ptr(row_order), ptr(out), _lib.index_dtype(out),
         ptr(stats), ptr(row_prefix), ptr(ws), ws_bytes, stream_of(q))
    return (out, stats) if with_stats else out


def sparse_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, idx: torch.Tensor,
                     scale_div: Optional[float] = None, causal: bool = False,
                     out: Optional[torch.Tensor] = None,
                     error_flag: Optional[torch.Tensor] = None,
                     row_order: Optional[torch.Tensor] = None,
                     q_pos0: Optional[int] = None, dense_prefix: bool = True,
                     row_prefix: Optional[torch.Tensor] = None,
                     row_stats: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Stage (d): gathered exact attention, [B, n_q, h_q, d] in q's dtype (ssa/attention.py:12-115).

    ``row_order`` (int32 [B, h_kv, n_q], a permutation of 0..n_q-1 per head) only
    sets the order in which rows are processed; results are the same.  ``q`` and
    ``idx`` may hold fewer rows (n_q) than ``k``/``v`` have keys: query row r
    then sits at key position ``q_pos0 + r`` (default n - n_q), which is what
    ``causal`` compares the indices with.  ``dense_prefix`` (bf16, d 64 or 128):
    the keys [0, X) a row's indices hold exactly once are attended in blocks of
    neighbouring rows that load them once (a workspace of the library's size);
    ``row_prefix`` (int32 [B, h_kv, n_q], from ``select``) gives X per row, which
    the pass otherwise finds from the indices."""
    for name, t in (("q", q), ("k", k), ("v", v), ("indices", idx)):
        _check_rows(t, name)
    _lib.require_device(q, k, v, idx)
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError(f"q, k, v must share a dtype ({q.dtype}, {k.dtype}, {v.dtype})")
    B, n_q, h_q, d = q.shape
    n = k.shape[1]
    if q_pos0 is None:
        q_pos0 = n - n_q
    h_kv = k.shape[2]
    top_k = idx.shape[-1]
    if scale_div is None:
        scale_div = math.sqrt(d)
    if out is None:
        out = torch.empty((B, n_q, h_q, d), device=q.device, dtype=q.dtype)
    if row_order is not None:
        _lib.require_device(row_order)
        if row_order.dtype != torch.int32 or tuple(row_order.shape) != (B, h_kv, n_q):
            raise ValueError(f"row_order must be int32 [{B}, {h_kv}, {n_q}]")
        row_order = row_order.contiguous()
    ws_bytes = 0
    if dense_prefix:
        ws_bytes = int(_lib.load().ssa_sparse_attention_workspace_bytes(
            _lib.elem_dtype(q), B, n_q, h_q, h_kv, d, top_k))
    ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8) if ws_bytes else None
    if row_prefix is not None:
        _lib.require_device(row_prefix)
        if (row_prefix.dtype != torch.int32 or tuple(row_prefix.shape) != (B, h_kv, n_q)
                or not row_prefix.is_contiguous()):
            raise ValueError(f"row_prefix must be a contiguous int32 [{B}, {h_kv}, {n_q}] tensor")
    _check_stats(row_stats, B, h_kv, n_q, h_q)
    call("ssa_sparse_attention_block", ptr(q), ptr(k), ptr(v), _lib.elem_dtype(q), B, n, n_q, q_pos0,
         h_q, h_kv, d,
         q.stride(0), q.stride(1), q.stride(2), k.stride(0), k.stride(1), k.stride(2),
         v.stride(0), v.stride(1), v.stride(2), ptr(idx), _lib.index_dtype(idx), top_k,
         idx.stride(0), idx.stride(1), idx.stride(2), float(scale_div), int(bool(causal)),
         ptr(row_order), ptr(row_prefix), ptr(out), _lib.elem_dtype(out), out.stride(0), out.stride(1),
         out.stride(2), ptr(error_flag), ptr(row_stats), ptr(ws), ws_bytes, stream_of(q))
    return out


def _check_stats(row_stats, B, h_kv, n, h_q):
    if row_stats is None:
        return
    _lib.require_device(row_stats)
    if (row_stats.dtype != torch.float32 or tuple(row_stats.shape) != (B, h_kv, n, h_q // h_kv, 2)
            or not row_stats.is_contiguous()):
        raise ValueError(f"row_stats must be a contiguous fp32 [{B}, {h_kv}, {n}, {h_q // h_kv}, 2] tensor")


def row_stats_buffer(q: torch.Tensor, h_kv: int) -> torch.Tensor:
    """NaN-filled fp32 [B, h_kv, n, g, 2] for sparse_attention(row_stats=...):
    the matrix-core forward writes each (row, head)'s softmax reference and
    1 / sum, which sparse_attention_backward(row_stats=...) then reuses; entries
    left NaN (other paths) are recomputed by the backward."""
    B, n, h_q = q.shape[0], q.shape[1], q.shape[2]
    return torch.full((B, h_kv, n, h_q // h_kv, 2), float("nan"), device=q.device, dtype=torch.float32)


def block_indices(idx: torch.Tensor, block_size: int, n_k_blocks: Optional[int] = None,
                  error_flag: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Key blocks per query block, int64 [B, ceil(n / block_size), h_kv, n_k_blocks]
    (ssa/triton_kernel.py:226-294) from token selections ``idx`` [B, n, h_kv, top_k];
    n_k_blocks defaults to min(top_k, number of blocks).  Ranked by reference
    count, then lower block id."""
    _check_rows(idx, "indices")
    _lib.require_device(idx)
    B, n, h_kv, top_k = idx.shape
    nb = (n + block_size - 1) // block_size
    if n_k_blocks is None:
        n_k_blocks = min(top_k, nb)
    out = torch.empty((B, nb, h_kv, n_k_blocks), device=idx.device, dtype=torch.int64)
    call("ssa_block_indices", ptr(idx), _lib.index_dtype(idx), B, n, h_kv, top_k,
         idx.stride(0), idx.stride(1), idx.stride(2), int(block_size), int(n_k_blocks), ptr(out),
         _lib.index_dtype(out), out.stride(0), out.stride(1), out.stride(2), ptr(error_flag),
         stream_of(idx))
    return out


def block_sparse_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, blocks: torch.Tensor,
                           block_size: int, scale_div: Optional[float] = None,
                           out: Optional[torch.Tensor] = None,
                           error_flag: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Causal exact attention of each query over the key blocks listed for its
    query block: ``blocks`` [B, ceil(n / block_size), h_kv, n_k_blocks]
    (ssa/triton_kernel.py:141-223, with an exact normalised softmax)."""
    for name, t in (("q", q), ("k", k), ("v", v), ("block_indices", blocks)):
        _check_rows(t, name)
    _lib.require_device(q, k, v, blocks)
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError(f"q, k, v must share a dtype ({q.dtype}, {k.dtype}, {v.dtype})")
    B, n, h_q, d = q.shape
    h_kv = k.shape[2]
    nb = (n + block_size - 1) // block_size
    if tuple(blocks.shape[:3]) != (B, nb, h_kv):
        raise ValueError(f"block_indices must be [{B}, {nb}, {h_kv}, n_k_blocks], got {tuple(blocks.shape)}")
    if scale_div is None:
        scale_div = math.sqrt(d)
    if out is None:
        out = torch.empty((B, n, h_q, d), device=q.device, dtype=q.dtype)
    call("ssa_block_sparse_attention", ptr(q), ptr(k), ptr(v), _lib.elem_dtype(q), B, n, h_q, h_kv, d,
         q.stride(0), q.stride(1), q.stride(2), k.stride(0), k.stride(1), k.stride(2),
         v.stride(0), v.stride(1), v.stride(2), ptr(blocks), _lib.index_dtype(blocks),
         int(block_size), blocks.shape[-1], blocks.stride(0), blocks.stride(1), blocks.stride(2),
         float(scale_div), ptr(out), _lib.elem_dtype(out), out.stride(0), out.stride(1), out.stride(2),
         ptr(error_flag), stream_of(q))
    return out


class Routing(NamedTuple):
    """What one selection was made from, for the bucket-mode backward: the
    stage (a) codes, the stage (b) key index and whether the selection's mask
    was causal (else none; an explicit mask has no bucket mode)."""
    q_codes: torch.Tensor   # int32 [B, h_kv, n, a]
    k_codes: torch.Tensor   # int32 [B, h_kv, n, b]
    offsets: torch.Tensor   # int32 [B, h_kv, N_c + 1]
    postings: torch.Tensor  # int32 [B, h_kv, n * b]
    causal: bool


def sparse_attention_backward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, idx: torch.Tensor,
                              out: torch.Tensor, dout: torch.Tensor,
                              scale_div: Optional[float] = None, causal: bool = False,
                              error_flag: Optional[torch.Tensor] = None,
                              row_order: Optional[torch.Tensor] = None,
                              row_prefix: Optional[torch.Tensor] = None,
                              routing: Optional[Routing] = None, bitmap_rows: int = -1,
                              row_stats: Optional[torch.Tensor] = None
                              ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Gradients of stage (d) w.r.t. q, k, v (fp32, shapes of q, k, v), given the
    forward output ``out`` and its gradient ``dout`` (the autograd backward of
    ssa/attention.py:64-113).

    With ``row_prefix`` and ``routing`` (the selection that produced ``idx``,
    n >= top_k) the candidate slots' dk and dv come from the bucket pass
    (ssa_sparse_attention_backward_routed); ``bitmap_rows`` sizes its key
    bitmaps for rows without filler (-1: half the rows).  ``row_stats``
    (``row_stats_buffer`` filled by the forward) saves the row kernel's first
    pass for the rows it covers.  Same results."""
    for name, t in (("q", q), ("k", k), ("v", v), ("indices", idx), ("out", out), ("dout", dout)):
        _check_rows(t, name)
    _lib.require_device(q, k, v, idx, out, dout)
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError(f"q, k, v must share a dtype ({q.dtype}, {k.dtype}, {v.dtype})")
    B, n, h_q, d = q.shape
    h_kv = k.shape[2]
    top_k = idx.shape[-1]
    if tuple(out.shape) != (B, n, h_q, d) or tuple(dout.shape) != (B, n, h_q, d):
        raise ValueError("out and dout must have q's shape")
    if scale_div is None:
        scale_div = math.sqrt(d)
    dq = torch.zeros((B, n, h_q, d), device=q.device, dtype=torch.float32)
    dk = torch.empty((B, n, h_kv, d), device=q.device, dtype=torch.float32)
    dv = torch.empty((B, n, h_kv, d), device=q.device, dtype=torch.float32)
    if row_order is not None:
        _lib.require_device(row_order)
        if row_order.dtype != torch.int32 or tuple(row_order.shape) != (B, h_kv, n):
            raise ValueError(f"row_order must be int32 [{B}, {h_kv}, {n}]")
        row_order = row_order.contiguous()
    ws_bytes, ws = 0, None
    if row_prefix is not None:
        _lib.require_device(row_prefix)
        if (row_prefix.dtype != torch.int32 or tuple(row_prefix.shape) != (B, h_kv, n)
                or not row_prefix.is_contiguous()):
            raise ValueError(f"row_prefix must be a contiguous int32 [{B}, {h_kv}, {n}] tensor")
        if routing is None:
            ws_bytes = int(_lib.load().ssa_sparse_attention_backward_workspace_bytes(
                _lib.elem_dtype(q), _lib.elem_dtype(dout), B, n, h_q, h_kv, d))
    _check_stats(row_stats, B, h_kv, n, h_q)
    common = (ptr(q), ptr(k), ptr(v), _lib.elem_dtype(q), B, n, h_q,
              h_kv, d, q.stride(0), q.stride(1), q.stride(2), k.stride(0), k.stride(1), k.stride(2),
              v.stride(0), v.stride(1), v.stride(2), ptr(idx), _lib.index_dtype(idx), top_k,
              idx.stride(0), idx.stride(1), idx.stride(2), float(scale_div), int(bool(causal)),
              ptr(row_order), ptr(out), _lib.elem_dtype(out), out.stride(0), out.stride(1),
              out.stride(2), ptr(dout), _lib.elem_dtype(dout), dout.stride(0), dout.stride(1),
              dout.stride(2), ptr(dq), ptr(dk), ptr(dv), ptr(error_flag), ptr(row_prefix), ptr(row_stats))
    if row_prefix is not None and routing is not None:
        qc, kc, off, post = (_contig_i32(t, name) for t, name in (
            (routing.q_codes, "q_codes"), (routing.k_codes, "k_codes"), (routing.offsets, "offsets"),
            (routing.postings, "postings")))
        _lib.require_device(qc, kc, off, post)
        a, b, n_c = qc.shape[-1], kc.shape[-1], off.shape[-1] - 1
        if (tuple(qc.shape[:3]) != (B, h_kv, n) or tuple(kc.shape[:3]) != (B, h_kv, n)
                or tuple(off.shape[:2]) != (B, h_kv) or tuple(post.shape) != (B, h_kv, n * b)):
            raise ValueError("routing tensors do not match q, k (see kernels.Routing)")
        ws_bytes = int(_lib.load().ssa_sparse_attention_backward_routed_workspace_bytes(
            _lib.elem_dtype(q), _lib.elem_dtype(dout), B, n, h_q, h_kv, d, top_k, a, b, n_c, int(bitmap_rows)))
        ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8) if ws_bytes else None
        call("ssa_sparse_attention_backward_routed", *common, ptr(qc), a, ptr(kc), b, ptr(off), ptr(post),
             n_c, int(bool(routing.causal)), ptr(ws), ws_bytes, stream_of(q))
        return dq, dk, dv
    ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8) if ws_bytes else None
    call("ssa_sparse_attention_backward", *common, ptr(ws), ws_bytes, stream_of(q))
    return dq, dk, dv


def _contig_i32(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.int32:
        raise TypeError(f"{name} must be int32")
    return t if t.is_contiguous() else t.contiguous()
