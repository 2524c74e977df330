"""SSAAttention: drop-in sparse attention layer (ssa/ssa_layer.py:17-138).

Same constructor, parameter names, initialisation order and forward signature
as the reference.  The per-batch Python loop of the reference is folded into
the kernels' batch dimension; projections stay on PyTorch GEMMs (hipBLASLt).
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import kernels
from .attention import dense_attention, sparse_exact_attention
from .router import CodebookRouter
from .utils import build_causal_mask


class _Rope(torch.autograd.Function):
    """ssa_rope with its transpose as the backward (rotation by the negative
    angle, the same three rounded ops torch's autograd of the op sequence runs)."""

    @staticmethod
    def forward(ctx, x, cos, sin, rot, by_head):
        ctx.save_for_backward(cos, sin)
        ctx.rot, ctx.by_head = rot, by_head
        return kernels.rope(x, cos, sin, rot, by_head)

    @staticmethod
    def backward(ctx, grad):
        cos, sin = ctx.saved_tensors
        grad = grad if grad.stride(-1) == 1 else grad.contiguous()
        return kernels.rope(grad, cos, sin, ctx.rot, ctx.by_head, inverse=True), None, None, None, None


def rope_rows(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, rot: int,
              by_head: bool) -> torch.Tensor:
    """Rotary embedding of x [B, n, h, d] on the HIP kernel (ssa_rope), differentiable
    in x; the result keeps x's dtype."""
    if torch.is_grad_enabled() and x.requires_grad:
        return _Rope.apply(x, cos, sin, rot, by_head)
    return kernels.rope(x, cos, sin, rot, by_head)


def head_rope_tables(freqs: torch.Tensor, n: int, heads: int, head_dim: int,
                     position_ids: Optional[torch.Tensor] = None):
    """cos/sin tables of the reference layer's apply_rope call (ssa/ssa_layer.py:
    106-117 with ssa/utils.py:19-27): per batch element the angle rows are
    freqs[position_ids[b]] (or freqs[:n]) and, because apply_rope sees an
    [n, heads, d] tensor, row j is used for head j; only the first head_dim/2
    features rotate; a single angle row (n = 1) is broadcast over the heads.
    Returns ([B or 1, heads, d/2] cos, sin)."""
    half = head_dim // 2
    ang = freqs[position_ids] if position_ids is not None else freqs[:n]
    if ang.shape[-2] == 1 and heads > 1:
        # one angle row (a single-token forward) broadcasts over every head, as
        # apply_rope's [1, half] tables do against [1, heads, half]
        ang = ang.expand(*ang.shape[:-2], heads, ang.shape[-1])
    if ang.shape[-2] < heads:
        raise ValueError(f"apply_rope indexes the angle table by head: {heads} heads need "
                         f"{heads} angle rows (or one, broadcast), the table has {ang.shape[-2]}")
    if ang.shape[-1] < half:
        raise ValueError(f"freqs must be at least head_dim/2 = {half} wide, got {ang.shape[-1]}")
    ang = ang[..., :heads, :half]
    if ang.dtype not in (torch.float32, torch.bfloat16):
        ang = ang.float()
    if ang.dim() == 2:
        ang = ang.unsqueeze(0)
    return ang.cos().contiguous(), ang.sin().contiguous()


class SSAAttention(nn.Module):
    """Sub-quadratic Selective Attention layer (ssa/ssa_layer.py:17-66).

    Extension: ``causal_attention`` (keyword, default False) makes stage 3
    ignore selected indices above the query position.  Every selected
    candidate is causal already; the flag only concerns the filler indices of
    rows with fewer than top_k candidates.  The default attends them unmasked,
    as the reference does (ssa/ssa_layer.py:129-130 passes the router's indices
    to sparse_exact_attention, which applies no mask); the filler keys are the
    lowest non-candidate indices, so rows i < top_k can attend keys past i.
    With ``causal_attention=True``, top_k = n reproduces causal dense attention
    exactly.  ``reference_flat_gather`` (keyword, default False) makes stage 3
    gather as the reference's code does, index j of KV head h reading row
    j + h*n of K and V flattened to [n*h_kv, d] (ssa/attention.py:76-96), rather
    than K[j, h] as its docstring and router do; see sparse_exact_attention.
    """

    def __init__(
        self,
        hidden_size: int = 512,
        num_q_heads: int = 8,
        num_kv_heads: int = 2,
        head_dim: int = 64,
        route_dim: int = 16,
        num_codebook: int = 512,
        codes_per_key: int = 4,
        codes_per_query: int = 8,
        top_k: int = 64,
        bias: bool = False,
        causal_attention: bool = False,
        reference_flat_gather: bool = False,
    ):
        super().__init__()
        self.hidden_size = hidden_size
        self.num_q_heads = num_q_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.top_k = top_k
        self.causal_attention = causal_attention
        self.reference_flat_gather = reference_flat_gather
        assert num_q_heads % num_kv_heads == 0
        # Same modules and draw order as ssa/ssa_layer.py:52-66.
        self.q_proj = nn.Linear(hidden_size, num_q_heads * head_dim, bias=bias)
        self.k_proj = nn.Linear(hidden_size, num_kv_heads * head_dim, bias=bias)
        self.v_proj = nn.Linear(hidden_size, num_kv_heads * head_dim, bias=bias)
        self.o_proj = nn.Linear(num_q_heads * head_dim, hidden_size, bias=bias)
        self.router = CodebookRouter(
            head_dim=head_dim,
            route_dim=route_dim,
            num_kv_heads=num_kv_heads,
            num_codebook=num_codebook,
            codes_per_key=codes_per_key,
            codes_per_query=codes_per_query,
            top_k=top_k,
        )

    def project(self, hidden_states: torch.Tensor, position_ids: Optional[torch.Tensor] = None,
                freqs: Optional[torch.Tensor] = None):
        """q, k, v as [B, n, heads, d], RoPE applied to q and k when freqs is given."""
        B, n, _ = hidden_states.shape
        q = self.q_proj(hidden_states).view(B, n, self.num_q_heads, self.head_dim)
        k = self.k_proj(hidden_states).view(B, n, self.num_kv_heads, self.head_dim)
        v = self.v_proj(hidden_states).view(B, n, self.num_kv_heads, self.head_dim)
        if freqs is not None:
            cos, sin = head_rope_tables(freqs, n, self.num_q_heads, self.head_dim, position_ids)
            q = rope_rows(q, cos, sin, self.head_dim // 2, by_head=True)
            k = rope_rows(k, cos, sin, self.head_dim // 2, by_head=True)
        return q, k, v

    def forward(
        self,
        hidden_states: torch.Tensor,
        attention_mask: Optional[torch.Tensor] = None,
        position_ids: Optional[torch.Tensor] = None,
        freqs: Optional[torch.Tensor] = None,
        use_dense: bool = False,
    ) -> torch.Tensor:
        """[B, n, hidden] -> [B, n, hidden] (ssa/ssa_layer.py:68-138).

        ``attention_mask`` is accepted and ignored, as in the reference; the
        layer is always causal.
        """
        B, n, _ = hidden_states.shape
        q, k, v = self.project(hidden_states, position_ids, freqs)
        if use_dense:
            mask = build_causal_mask(n, device=hidden_states.device)
            out = torch.stack([dense_attention(q[b], k[b], v[b], causal_mask=mask) for b in range(B)])
        else:
            # Stage 3 does not depend on the order of the selected keys, so the
            # router lists them by index and skips rescoring rows whose
            # candidates all fit in top_k; inside the layer the indices stay
            # int32 (half the bytes of the public int64 output), and the rows
            # of each head are attended grouped by smallest code, so rows sharing
            # candidate keys run together (no result depends on that order).
            res = self.router.route(q, k, causal_mask=True, hard=True, sorted=False,
                                    index_dtype=torch.int32, with_order=True, with_prefix=True)
            out = sparse_exact_attention(q, k, v, res.indices, causal=self.causal_attention,
                                         check_indices=False, row_order=res.order,
                                         row_prefix=res.prefix, routing=res.routing(),
                                         reference_flat_gather=self.reference_flat_gather)
        return self.o_proj(out.reshape(B, n, -1).to(hidden_states.dtype))


    def compute_auxiliary_loss(self, hidden_states: torch.Tensor,
                               freqs: Optional[torch.Tensor] = None) -> torch.Tensor:
        """KL(teacher || student) at up to 64 sampled query positions
        (ssa/ssa_layer.py:140-212): the teacher is dense causal softmax attention
        of the un-rotated q/k projections, the student the softmax of
        ``_get_routing_logits`` expanded over each KV head's query heads;
        batchmean over the sampled rows, averaged over the batch.  ``freqs`` is
        accepted and unused, as in the reference.  The positions come from one
        ``torch.randperm(n)`` draw, as the reference's do; only those rows'
        logits are formed (the reference builds all n x n and then indexes
        them: the same values, row by row), so memory is O(64 n), not O(n^2).
        Training-time regularizer on PyTorch ops (differentiable in the
        router parameters; as in the reference, the gradient reaching q_proj and
        k_proj through the teacher is NaN, since kl_div's derivative in its
        target is target / target at the masked zeros); the forward path does
        not use it."""
        B, n, _ = hidden_states.shape
        g = self.num_q_heads // self.num_kv_heads
        q = self.q_proj(hidden_states).view(B, n, self.num_q_heads, self.head_dim)
        k = self.k_proj(hidden_states).view(B, n, self.num_kv_heads, self.head_dim)
        rows = torch.randperm(n, device=hidden_states.device)[:min(n, 64)]
        allowed = torch.arange(n, device=rows.device)[None, :] <= rows[:, None]   # [s, n]
        total = hidden_states.new_zeros((), dtype=torch.float32)
        for b in range(B):
            # teacher: [h_q, s, n] = q_s . k^T / sqrt(d), key head j // g for query head j
            k_rep = k[b].repeat_interleave(g, dim=1)                  # [n, h_q, d]
            logits = torch.matmul(q[b, rows].transpose(0, 1),
                                  k_rep.permute(1, 2, 0).contiguous()) / (self.head_dim ** 0.5)
            teacher = torch.softmax(logits.masked_fill(~allowed[None], float("-inf")), dim=-1)
            student = self._get_routing_logits(q[b], k[b], allowed, rows=rows)  # [s, h_kv, n]
            student = torch.softmax(student.repeat_interleave(g, dim=1), dim=-1)  # [s, h_q, n]
            tw = teacher.transpose(0, 1)                               # [s, h_q, n]
            # F.kl_div(log(student + 1e-10), teacher, "batchmean"): zero-weight terms add 0
            kl = torch.where(tw > 0, tw * (torch.log(tw) - torch.log(student + 1e-10)),
                             torch.zeros_like(tw)).sum() / rows.numel()
            total = total + kl
        return total / max(B, 1)

    def _get_routing_logits(self, q: torch.Tensor, k: torch.Tensor, causal_mask: torch.Tensor,
                            rows: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Routing-space attention estimate (ssa/ssa_layer.py:214-257):
        ``(q_hat . C^T) . (k_hat . C^T)^T`` per KV head with the router's
        projections (query heads mean-pooled per group), L2-normalized routing
        vectors and codebook, masked where ``causal_mask`` is False.  q [n, h_q, d],
        k [n, h_kv, d]; returns [n, h_kv, n], or [len(rows), h_kv, n] for the
        query ``rows`` with ``causal_mask`` then holding those rows only."""
        n = q.shape[0]
        r = self.router
        g = q.shape[1] // k.shape[1]
        if rows is not None:
            q = q[rows]
        q_route = r.W_qr(q).reshape(q.shape[0], self.num_kv_heads, g, r.route_dim).mean(dim=2)
        k_route = r.W_kr(k)
        cb = F.normalize(r.codebook, dim=-1)                          # [h_kv, N_c, d_s]
        qs = torch.matmul(F.normalize(q_route, dim=-1).transpose(0, 1), cb.transpose(1, 2).contiguous())
        ks = torch.matmul(F.normalize(k_route, dim=-1).transpose(0, 1), cb.transpose(1, 2).contiguous())
        est = torch.matmul(qs, ks.transpose(1, 2).contiguous())      # [h_kv, s, n]
        est = est.masked_fill(~causal_mask[None], float("-inf"))
        return est.transpose(0, 1)


class ToyTransformerBlock(nn.Module):
    """LayerNorm -> SSAAttention -> residual -> LayerNorm -> GELU FFN -> residual
    (ssa/ssa_layer.py:260-285)."""

    def __init__(self, hidden_size: int = 512, **ssa_kwargs):
        super().__init__()
        self.attn = SSAAttention(hidden_size=hidden_size, **ssa_kwargs)
        self.norm1 = nn.LayerNorm(hidden_size)
        self.norm2 = nn.LayerNorm(hidden_size)
        self.ffn = nn.Sequential(
            nn.Linear(hidden_size, hidden_size * 4),
            nn.GELU(),
            nn.Linear(hidden_size * 4, hidden_size),
        )

    def forward(self, x: torch.Tensor, **attn_kwargs) -> torch.Tensor:
        x = self.attn(self.norm1(x), **attn_kwargs) + x
        return self.ffn(self.norm2(x)) + x
