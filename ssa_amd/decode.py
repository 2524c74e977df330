"""Incremental decoding against a key/value cache (ssa_design.md:225-234).

The reference describes decode-time SSA as single-query routing against the
cached keys' inverted index; its code only runs whole sequences.  Here a step
with m new tokens (m = 1 when decoding, more for a prefill chunk):

* appends the new K/V rows to a preallocated cache ``[B, max_len, h_kv, d]``;
* routes the new queries and keys (stage a, only the m new rows);
* appends the new keys' codes and rebuilds the inverted index over all cached
  keys (stage b; 0.13 ms for 32K keys x 8 heads);
* selects and attends only the m new query rows against all cached keys
  (``ssa_select_block`` / ``ssa_sparse_attention_block``: query row r at key
  position len + r).

Row t of a step equals row t of the whole-sequence forward over the same
prefix (same keys, same codes, same index): indices bit for bit, outputs from
the same kernel code.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import kernels
from .router import CodebookRouter


class SSADecodeCache:
    """K/V cache plus routing state of one SSA attention layer.

    ``router`` gives the codebook and top-k settings; ``max_len`` bounds the
    cached sequence (288 GB of HBM holds long caches: K and V of 1 M tokens at
    h_kv = 8, d = 128, bf16 take 4 GB).
    """

    def __init__(self, router: CodebookRouter, batch: int, max_len: int, head_dim: int,
                 dtype: torch.dtype = torch.bfloat16, device: Optional[torch.device] = None):
        device = device or router.codebook.device
        h_kv = router.num_kv_heads
        self.router = router
        self.max_len = max_len
        self.len = 0
        self.k = torch.empty(batch, max_len, h_kv, head_dim, device=device, dtype=dtype)
        self.v = torch.empty(batch, max_len, h_kv, head_dim, device=device, dtype=dtype)
        self.k_codes = torch.empty(batch, h_kv, max_len, router.codes_per_key, device=device,
                                   dtype=torch.int32)

    def reset(self) -> None:
        self.len = 0

    @torch.no_grad()
    def step(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
             causal_attention: bool = True, return_indices: bool = False):
        """Attend the m new tokens' queries ``q [B, m, h_q, d]`` over the cache
        after appending their keys and values ``k, v [B, m, h_kv, d]``.

        Returns ``[B, m, h_q, d]`` (and the int32 ``[B, m, h_kv, top_k]``
        selections, keys ascending, with ``return_indices``).  With
        ``causal_attention`` (the layer's default) selected keys past a query's
        position are dropped in the attention, as ``SSAAttention`` does."""
        r = self.router
        B, m = q.shape[0], q.shape[1]
        n0, n = self.len, self.len + m
        if n > self.max_len:
            raise ValueError(f"cache full: {n} tokens > max_len {self.max_len}")
        if k.shape[1] != m or v.shape[1] != m:
            raise ValueError("q, k and v must hold the same new tokens")
        self.k[:, n0:n] = k
        self.v[:, n0:n] = v
        qc, kc = kernels.route_codes(q, k, r.W_qr.weight, r.W_kr.weight, r.codebook,
                                     r.codes_per_query, r.codes_per_key, r.temperature)
        self.k_codes[:, :, n0:n] = kc
        offsets, postings = kernels.build_index(self.k_codes[:, :, :n].contiguous(), r.num_codebook)
        keys, vals = self.k[:, :n], self.v[:, :n]
        idx = kernels.select(q, keys, qc, offsets, postings, r.codes_per_key, r.top_k,
                             sorted=False, index_dtype=torch.int32, q_pos0=n0)
        out = kernels.sparse_attention(q, keys, vals, idx, None, causal_attention, q_pos0=n0)
        self.len = n
        return (out, idx) if return_indices else out
