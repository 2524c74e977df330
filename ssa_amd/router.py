"""CodebookRouter: stages (a)-(c) of SSA on the HIP kernels of libssa_hip.

Drop-in for ``ssa.router.CodebookRouter`` (ssa/router.py:14-275): same
constructor, parameter names, initialisation order and ``forward`` signature.
The O(n^2) rescoring and mask of the reference are replaced by an inverted
index plus per-query candidate rescoring; the selected set is the reference's
(ssa/router.py:224-235), ranked by fp32 score with ties to the lowest index.
"""

from __future__ import annotations

from typing import Optional, Union

import torch
import torch.nn as nn

from . import _lib, kernels

MaskArg = Union[None, bool, torch.Tensor]


def _batched(x: torch.Tensor, name: str) -> torch.Tensor:
    if x.dim() == 3:
        return x.unsqueeze(0)
    if x.dim() == 4:
        return x
    raise ValueError(f"{name} must be [n, heads, d] or [B, n, heads, d], got {tuple(x.shape)}")


def _as_kernel_dtype(x: torch.Tensor) -> torch.Tensor:
    # fp16 widens exactly to fp32; scoring is fp32 for every input type.
    if x.dtype == torch.float16:
        return x.float()
    if x.stride(-1) != 1:
        return x.contiguous()
    return x


def mask_mode_for(causal_mask: MaskArg, n: int):
    """(mode, mask tensor or None) for a reference-style ``causal_mask`` argument."""
    if causal_mask is None or causal_mask is False:
        return _lib.MASK_NONE, None
    if causal_mask is True:
        return _lib.MASK_CAUSAL, None
    if not isinstance(causal_mask, torch.Tensor):
        raise TypeError(f"causal_mask must be None, a bool or a tensor, got {type(causal_mask)}")
    if tuple(causal_mask.shape[-2:]) != (n, n):
        raise ValueError(f"causal_mask must be [{n}, {n}], got {tuple(causal_mask.shape)}")
    if getattr(causal_mask, "_ssa_causal", False):
        return _lib.MASK_CAUSAL, None
    return _lib.MASK_DENSE, causal_mask.to(torch.bool)


class CodebookRouter(nn.Module):
    """Content-dependent router selecting ``top_k`` candidate keys per query
    (ssa/router.py:14-70).  Routing is per KV head; query heads of a GQA group
    are mean-pooled after projection."""

    def __init__(
        self,
        head_dim: int = 128,
        route_dim: int = 32,
        num_kv_heads: int = 8,
        num_codebook: int = 2048,
        codes_per_key: int = 4,
        codes_per_query: int = 16,
        top_k: int = 256,
        temperature: float = 1.0,
    ):
        super().__init__()
        self.head_dim = head_dim
        self.route_dim = route_dim
        self.num_kv_heads = num_kv_heads
        self.num_codebook = num_codebook
        self.codes_per_key = codes_per_key
        self.codes_per_query = codes_per_query
        self.top_k = top_k
        self.temperature = temperature
        # Same modules, names and RNG draw order as ssa/router.py:61-68, so seeded
        # construction and saved state_dicts carry over unchanged.
        self.W_qr = nn.Linear(head_dim, route_dim, bias=False)
        self.W_kr = nn.Linear(head_dim, route_dim, bias=False)
        self.codebook = nn.Parameter(
            torch.randn(num_kv_heads, num_codebook, route_dim) / route_dim**0.5
        )

    # ------------------------------------------------------------------ API

    def forward(
        self,
        q_full: torch.Tensor,
        k_full: torch.Tensor,
        causal_mask: MaskArg = None,
        hard: bool = True,
        *,
        sorted: bool = True,
    ) -> torch.Tensor:
        """Candidate key indices (ssa/router.py:73-149).

        Args:
            q_full: ``[n, h_q, d]`` (or batched ``[B, n, h_q, d]``), RoPE applied.
            k_full: ``[n, h_kv, d]`` (or ``[B, n, h_kv, d]``).
            causal_mask: None (no mask), True / ``build_causal_mask(n)`` (causal),
                or any bool ``[n, n]`` mask (True = allowed).
            hard: must be True; the reference's Gumbel branch cannot produce
                indices (ssa/router.py:131-137 vs :253).
            sorted: keyword-only; True (default) orders the selected keys by
                score like torch.topk; False lists the same set in ascending
                index order, which lets rows with at most top_k candidates skip
                rescoring.

        Returns:
            int64 ``[n, h_kv, top_k]`` (``[B, n, h_kv, top_k]`` for batched input),
            ordered by score (desc), ties to the lowest index; rows with fewer
            than top_k candidates continue with the lowest non-candidate indices,
            and top_k > n pads with index 0.
        """
        return self.route(q_full, k_full, causal_mask=causal_mask, hard=hard,
                          sorted=sorted).indices_view

    def route(self, q_full: torch.Tensor, k_full: torch.Tensor, causal_mask: MaskArg = None,
              hard: bool = True, with_stats: bool = False, index_dtype=torch.int64,
              sorted: bool = True, with_order: bool = False, with_prefix: bool = False):
        """Run stages (a)-(c) and keep the intermediates (a RouteResult).

        ``with_order`` also returns ``order`` (int32 [B, h_kv, n]): per head, the
        query positions grouped by their smallest code (ascending within a code).
        Selection already runs its rows in this order, and attention can too:
        rows that share buckets and candidate keys then run together.  It
        changes no result.  ``with_prefix`` also returns ``prefix`` (int32
        [B, h_kv, n]): X per row, the keys [0, X) its indices hold once (the
        lowest-key filler), which ``sparse_exact_attention(row_prefix=...)``
        attends in a dense pass."""
        if not hard:
            raise NotImplementedError(
                "hard=False (Gumbel-softmax assignment) is not supported: the reference's one-hot "
                "[n, h, N_c] assignment cannot feed its candidate mask (ssa/router.py:131-137, :253)")
        unbatched = q_full.dim() == 3
        q = _as_kernel_dtype(_batched(q_full, "q_full"))
        k = _as_kernel_dtype(_batched(k_full, "k_full"))
        n, num_q_heads = q.shape[1], q.shape[2]
        assert num_q_heads % self.num_kv_heads == 0, "num_q_heads must be divisible by num_kv_heads"
        if k.shape[2] != self.num_kv_heads:
            raise ValueError(f"k_full has {k.shape[2]} heads, router expects {self.num_kv_heads}")
        if q.shape[-1] != self.head_dim or k.shape[-1] != self.head_dim:
            raise ValueError(f"head_dim mismatch: router {self.head_dim}, q {q.shape[-1]}, k {k.shape[-1]}")
        if k.dtype != q.dtype:
            k = k.to(q.dtype)
        mode, mask = mask_mode_for(causal_mask, n)
        _lib.require_device(q, k, self.codebook)
        q_codes, k_codes = kernels.route_codes(
            q, k, self.W_qr.weight, self.W_kr.weight, self.codebook,
            self.codes_per_query, self.codes_per_key, float(self.temperature))
        offsets, postings = kernels.build_index(k_codes, self.num_codebook)
        if mask is not None:
            mask = mask.to(q.device)
        order = query_order(q_codes, self.num_codebook) if with_order else None
        prefix = (torch.empty(q.shape[0], self.num_kv_heads, n, device=q.device, dtype=torch.int32)
                  if with_prefix else None)
        res = kernels.select(q, k, q_codes, offsets, postings, self.codes_per_key, self.top_k,
                             mode, mask, index_dtype=index_dtype, with_stats=with_stats,
                             sorted=sorted, row_order=order, row_prefix=prefix)
        idx, stats = res if with_stats else (res, None)
        out = RouteResult(q_codes, k_codes, offsets, postings, idx, stats)
        out.order = order
        out.prefix = prefix
        out.mask_mode = mode
        out.indices_view = idx[0] if unbatched else idx
        return out

    def get_code_assignment(self, k_full: torch.Tensor) -> torch.Tensor:
        """Top-b code ids per key, int64 ``[n, h_kv, b]`` (ssa/router.py:261-275)."""
        unbatched = k_full.dim() == 3
        k = _as_kernel_dtype(_batched(k_full, "k_full"))
        _lib.require_device(k, self.codebook)
        khat = kernels.route_vectors(k, self.W_kr.weight, 1)
        chat = kernels.normalize_rows(self.codebook.reshape(-1, self.route_dim)).view(
            self.num_kv_heads, self.num_codebook, self.route_dim)
        codes = kernels.code_topk(khat, chat, self.codes_per_key, 1.0)  # [B, h, n, b]
        out = codes.permute(0, 2, 1, 3).to(torch.int64)
        return out[0] if unbatched else out


def query_order(q_codes: torch.Tensor, num_codebook: int) -> torch.Tensor:
    """Query positions per (batch, kv head) grouped by their smallest code: the
    inverted index of each query's smallest code, int32 [B, h_kv, n]."""
    return kernels.query_order(q_codes, num_codebook)


class RouteResult:
    """Intermediates of one routing pass, in kernel layouts (batched):
    q_codes int32 [B, h_kv, n, a], k_codes int32 [B, h_kv, n, b],
    offsets int32 [B, h_kv, N_c + 1], postings int32 [B, h_kv, n * b],
    indices [B, n, h_kv, top_k], stats int32 [B, h_kv, n, 2] or None
    (unique candidates, postings read), order int32 [B, h_kv, n] or None (see
    query_order), prefix int32 [B, h_kv, n] or None (X per row, see route);
    indices_view is the reference-shaped view returned by forward()."""

    __slots__ = ("q_codes", "k_codes", "offsets", "postings", "indices", "stats", "order",
                 "prefix", "indices_view", "mask_mode")

    def __init__(self, q_codes, k_codes, offsets, postings, indices, stats):
        self.q_codes = q_codes
        self.k_codes = k_codes
        self.offsets = offsets
        self.postings = postings
        self.indices = indices
        self.stats = stats
        self.order = None
        self.prefix = None
        self.indices_view = indices
        self.mask_mode = None

    def routing(self):
        """kernels.Routing for the bucket-mode backward of attention over these
        indices, or None (an explicit mask, or an unknown one)."""
        if self.mask_mode not in (_lib.MASK_NONE, _lib.MASK_CAUSAL):
            return None
        return kernels.Routing(self.q_codes, self.k_codes, self.offsets, self.postings,
                               self.mask_mode == _lib.MASK_CAUSAL)
