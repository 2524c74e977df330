"""Stage 3 of SSA: exact softmax attention over selected keys (ssa/attention.py).

``sparse_exact_attention`` runs the gathered-KV HIP kernel of libssa_hip;
``dense_attention`` is the reference's plain PyTorch SDPA, kept for the
``use_dense`` comparison path and k = n checks.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from . import _lib, kernels


class _SparseAttention(torch.autograd.Function):
    """Stage (d) with its HIP backward (ssa_sparse_attention_backward): gradients
    flow to q, k and v as through the reference's gather/softmax/einsum
    (ssa/attention.py:64-113); the indices get none, as in the reference."""

    @staticmethod
    def forward(ctx, q, k, v, indices, scale, causal, row_order, flag, row_prefix, routing):
        # The backward's D = dO . o uses an fp32 copy of the output: a bf16 one
        # would carry its 2^-9 rounding into every gradient.
        out32 = torch.empty(q.shape, device=q.device, dtype=torch.float32)
        # the forward's softmax stats spare the backward its first pass (bf16 path)
        stats = kernels.row_stats_buffer(q, k.shape[2]) if q.dtype == torch.bfloat16 else None
        kernels.sparse_attention(q, k, v, indices, scale, causal, out=out32, error_flag=flag,
                                 row_order=row_order, row_prefix=row_prefix, row_stats=stats)
        ctx.scale, ctx.causal = scale, causal
        ctx.has_order = row_order is not None
        ctx.has_prefix = row_prefix is not None
        ctx.has_stats = stats is not None
        ctx.routing_causal = None if routing is None else bool(routing.causal)
        saved = ([q, k, v, indices, out32] + ([row_order] if row_order is not None else [])
                 + ([row_prefix] if row_prefix is not None else [])
                 + ([stats] if stats is not None else [])
                 + (list(routing[:4]) if routing is not None else []))
        ctx.save_for_backward(*saved)
        return out32 if q.dtype == torch.float32 else out32.to(q.dtype)

    @staticmethod
    def backward(ctx, dout):
        q, k, v, indices, out, *rest = ctx.saved_tensors
        order = rest.pop(0) if ctx.has_order else None
        prefix = rest.pop(0) if ctx.has_prefix else None
        stats = rest.pop(0) if ctx.has_stats else None
        routing = kernels.Routing(*rest[:4], ctx.routing_causal) if ctx.routing_causal is not None else None
        if dout.stride(-1) != 1:
            dout = dout.contiguous()
        dq, dk, dv = kernels.sparse_attention_backward(q, k, v, indices, out, dout, ctx.scale,
                                                       ctx.causal, row_order=order, row_prefix=prefix,
                                                       routing=routing, row_stats=stats)
        return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), None, None, None, None, None, None, None


def flat_gather_view(t: torch.Tensor) -> torch.Tensor:
    """The ``[.., n, h_kv, d]`` view whose element ``[j, h]`` is row ``j + h*n`` of
    ``t.reshape(n*h_kv, d)``: the rows ssa/attention.py:76-96 gathers for index j
    of KV head h (it flattens K to [n*h_kv, d] and offsets head h's indices by
    h*n).  No copy for a contiguous ``t``; differentiable (a view)."""
    *lead, n, h_kv, d = t.shape
    return t.reshape(*lead, n * h_kv, d).view(*lead, h_kv, n, d).transpose(-3, -2)


def sparse_exact_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    indices: torch.Tensor,
    scale: Optional[float] = None,
    *,
    causal: bool = False,
    check_indices: bool = True,
    row_order: Optional[torch.Tensor] = None,
    row_prefix: Optional[torch.Tensor] = None,
    routing: Optional[kernels.Routing] = None,
    reference_flat_gather: bool = False,
) -> torch.Tensor:
    """softmax(q . K[indices]^T / scale) . V[indices] per (query, KV head).

    Drop-in for ssa/attention.py:12-115: ``q [n, h_q, d]``, ``k, v [n, h_kv, d]``,
    ``indices [n, h_kv, top_k]`` (int64 or int32; batched ``[B, ...]`` shapes
    also accepted); ``scale`` is a divisor defaulting to sqrt(d); query head j
    uses KV head ``j // (h_q // h_kv)``; duplicated indices count twice.

    Keyword-only extensions: ``causal=True`` drops indices > query position (a
    row left with no index outputs zeros); ``check_indices`` raises IndexError
    (after a device sync) if any index is outside [0, n), as the reference's
    gather does -- out-of-range slots are never read either way.
    ``row_order`` (int32 [B, h_kv, n], e.g. ``CodebookRouter.route(...,
    with_order=True).order``) sets the order rows are processed in, for cache
    locality; it does not change the result.  ``row_prefix`` (int32 [B, h_kv, n],
    ``route(..., with_prefix=True).prefix``) names the key prefix [0, X) each
    row's indices hold once; bf16 inputs with d 64 or 128 attend it in a dense
    pass (also found from the indices without it; same result up to summation
    order).  ``routing`` (``route(...).routing()``, with ``row_prefix``) is the
    selection the indices came from: the backward then differentiates the
    candidate keys by codebook bucket (same gradients, far fewer atomics).
    ``reference_flat_gather=True`` reproduces what ssa/attention.py:76-96
    computes rather than its docstring's ``K[indices[i, h], h]``: index j of KV
    head h reads row ``j + h*n`` of K and V flattened to ``[n*h_kv, d]``
    (``flat_gather_view``; the same rows when h_kv = 1).  The kernels read
    that layout through strides, with no copy.

    Differentiable in q, k and v (HIP backward kernel); not in ``indices``.
    """
    unbatched = q.dim() == 3
    if unbatched:
        q, k, v, indices = q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0), indices.unsqueeze(0)
    if reference_flat_gather:
        k, v = flat_gather_view(k), flat_gather_view(v)
    seq_len, num_q_heads, head_dim = q.shape[1], q.shape[2], q.shape[3]
    num_kv_heads = k.shape[2]
    assert num_q_heads % num_kv_heads == 0
    if scale is None:
        scale = head_dim**0.5
    _lib.require_device(q, k, v, indices)
    out_dtype = q.dtype
    if q.dtype == torch.float16:
        q, k, v = q.float(), k.float(), v.float()
    q, k, v = (t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v))
    if indices.stride(-1) != 1:
        indices = indices.contiguous()
    flag = torch.zeros(1, device=q.device, dtype=torch.int32) if check_indices else None
    if row_order is not None and unbatched and row_order.dim() == 2:
        row_order = row_order.unsqueeze(0)
    if row_prefix is not None and unbatched and row_prefix.dim() == 2:
        row_prefix = row_prefix.unsqueeze(0)
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        out = _SparseAttention.apply(q, k, v, indices, float(scale), bool(causal), row_order, flag,
                                     row_prefix, routing)
    else:
        out = kernels.sparse_attention(q, k, v, indices, float(scale), causal, error_flag=flag,
                                       row_order=row_order, row_prefix=row_prefix)
    if flag is not None and int(flag.item()) != 0:
        raise IndexError(f"sparse_exact_attention: an index is outside [0, {seq_len})")
    if out.dtype != out_dtype:
        out = out.to(out_dtype)
    return out[0] if unbatched else out


def dense_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal_mask: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
) -> torch.Tensor:
    """Dense scaled dot-product attention with GQA (ssa/attention.py:118-158).

    ``q [n, h_q, d]``, ``k, v [n, h_kv, d]``, optional bool ``[n, n]`` mask
    (True = allowed), ``scale`` a divisor defaulting to sqrt(d).
    """
    seq_len, num_q_heads, head_dim = q.shape
    num_kv_heads = k.shape[1]
    if scale is None:
        scale = head_dim**0.5
    g = num_q_heads // num_kv_heads
    k_exp = k.unsqueeze(2).expand(-1, -1, g, -1).reshape(seq_len, num_q_heads, head_dim)
    v_exp = v.unsqueeze(2).expand(-1, -1, g, -1).reshape(seq_len, num_q_heads, head_dim)
    logits = torch.matmul(q.transpose(0, 1), k_exp.permute(1, 2, 0).contiguous()) / scale
    if causal_mask is not None:
        logits = logits.masked_fill(~causal_mask.unsqueeze(0), float("-inf"))
    w = F.softmax(logits, dim=-1)
    return torch.matmul(w, v_exp.transpose(0, 1).contiguous()).transpose(0, 1)
