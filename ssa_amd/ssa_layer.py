"""SSAAttention: drop-in sparse attention layer (ssa/ssa_layer.py:17-138).

Same constructor, parameter names, initialisation order and forward signature
as the reference.  The per-batch Python loop of the reference is folded into
the kernels' batch dimension; projections stay on PyTorch GEMMs (hipBLASLt).
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from .attention import dense_attention, sparse_exact_attention
from .router import CodebookRouter
from .utils import build_causal_mask


def _rope_batched(x: torch.Tensor, ang: torch.Tensor) -> torch.Tensor:
    """apply_rope (ssa/utils.py:7-41) on x [B, n, h, d] with per-batch angle rows.

    ``ang`` is ``[rows, rot]`` (shared) or ``[B, rows, rot]``.  As in the
    reference, the angle index runs over x's second-to-last axis (the heads
    when x is [n, h, d]) and only the first d/2 features rotate.  The result
    keeps x's dtype.
    """
    h, d = x.shape[-2], x.shape[-1]
    half = d // 2
    if ang.dim() == 2:
        ang = ang[:h, :half].unsqueeze(0)
    else:
        ang = ang[:, :h, :half]
    cos = ang.cos().unsqueeze(1)  # [B or 1, 1, h, half]
    sin = ang.sin().unsqueeze(1)
    x_rot, x_pass = x[..., :half], x[..., half:]
    cut = half // 2
    rot_half = torch.cat([-x_rot[..., cut:], x_rot[..., :cut]], dim=-1)
    out = torch.cat([x_rot * cos + rot_half * sin, x_pass.to(torch.result_type(x_rot, cos))], dim=-1)
    return out.to(x.dtype)


class SSAAttention(nn.Module):
    """Sub-quadratic Selective Attention layer (ssa/ssa_layer.py:17-66).

    Extension: ``causal_attention`` (default True) makes stage 3 ignore
    selected indices above the query position.  Every selected candidate is
    causal already; the flag only concerns the filler indices of rows with
    fewer than top_k candidates, which the reference attends unmasked
    (its choice of them is unspecified).  With it, top_k = n reproduces causal
    dense attention exactly.
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
        causal_attention: bool = True,
    ):
        super().__init__()
        self.hidden_size = hidden_size
        self.num_q_heads = num_q_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.top_k = top_k
        self.causal_attention = causal_attention
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
            ang = freqs[position_ids] if position_ids is not None else freqs[:n]
            q = _rope_batched(q, ang)
            k = _rope_batched(k, ang)
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
            # of each head are attended grouped by best code, so rows sharing
            # candidate keys run together (no result depends on that order).
            res = self.router.route(q, k, causal_mask=True, hard=True, sorted=False,
                                    index_dtype=torch.int32, with_order=True)
            out = sparse_exact_attention(q, k, v, res.indices, causal=self.causal_attention,
                                         check_indices=False, row_order=res.order)
        return self.o_proj(out.reshape(B, n, -1).to(hidden_states.dtype))


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
