"""Incremental decoding against a key/value cache (ssa_design.md:225-234).

The reference describes decode-time SSA as single-query routing against the
cached keys' inverted index, "maintained incrementally, avoiding re-scanning
the full KV cache on each step"; its code only runs whole sequences.  Here:

* a step with a few new tokens is one native call (``ssa_decode_step``): it
  appends their K/V rows and key codes to the cache, routes the new rows
  against the codebook prepared once, rebuilds a small *tail* index over the
  keys appended since the main index was built, and selects and attends each
  new query over all cached keys from both indices.  Nothing in it scans the
  whole cache;
* when the tail reaches ``tail_tokens`` keys, the main index is rebuilt over
  every cached key (``ssa_build_index``), an O(n) pass every ``tail_tokens``
  steps;
* a long chunk (a prefill) routes its rows together, rebuilds the main index
  over the whole cache and selects and attends its rows in one batch.

Row t of a step equals row t of the whole-sequence forward over the same
prefix with the same ``causal_attention`` setting: the same keys, codes and
candidate sets, indices bit for bit, and outputs from the same attention code.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib, kernels
from ._lib import call, ptr, stream_of
from .router import CodebookRouter


class SSADecodeCache:
    """K/V cache plus routing state of one SSA attention layer.

    ``router`` gives the codebook and top-k settings; ``max_len`` bounds the
    cached sequence (288 GB of HBM holds long caches: K and V of 1 M tokens at
    h_kv = 8, d = 128, bf16 take 4 GB).  ``tail_tokens`` keys may be appended
    before the main index is rebuilt.  Call ``prepare()`` after changing the
    router's parameters.
    """

    def __init__(self, router: CodebookRouter, batch: int, max_len: int, head_dim: int,
                 dtype: torch.dtype = torch.bfloat16, device: Optional[torch.device] = None,
                 tail_tokens: int = 512):
        device = device or router.codebook.device
        h_kv = router.num_kv_heads
        self.router = router
        self.batch = batch
        self.max_len = max_len
        self.head_dim = head_dim
        self.dtype = dtype
        self.len = 0
        self.n_base = 0
        self.tail_tokens = int(tail_tokens)
        self.rebuilds = 0
        b, n_c = router.codes_per_key, router.num_codebook
        self.k = torch.empty(batch, max_len, h_kv, head_dim, device=device, dtype=dtype)
        self.v = torch.empty(batch, max_len, h_kv, head_dim, device=device, dtype=dtype)
        self.k_codes = torch.empty(batch, h_kv, max_len, b, device=device, dtype=torch.int32)
        self.offsets = torch.zeros(batch, h_kv, n_c + 1, device=device, dtype=torch.int32)
        self.postings = torch.zeros(batch, h_kv, 1, device=device, dtype=torch.int32)
        self.tail_cap = self.tail_tokens * b
        self.tail_offsets = torch.zeros(batch, h_kv, n_c + 1, device=device, dtype=torch.int32)
        self.tail_postings = torch.zeros(batch, h_kv, self.tail_cap, device=device, dtype=torch.int32)
        self.prep = None
        self.prepare()

    def prepare(self) -> None:
        """Normalize the codebook and keep its bf16 copy and fp32 router weights."""
        r = self.router
        L = _lib.load()
        cb = r.codebook.detach().to(torch.float32).contiguous()
        self.w_qr = r.W_qr.weight.detach().to(torch.float32).contiguous()
        self.w_kr = r.W_kr.weight.detach().to(torch.float32).contiguous()
        nbytes = int(L.ssa_decode_prepare_bytes(r.num_kv_heads, r.num_codebook, r.route_dim))
        self.prep = torch.empty(nbytes, device=cb.device, dtype=torch.uint8)
        call("ssa_decode_prepare", ptr(cb), r.num_kv_heads, r.num_codebook, r.route_dim,
             ptr(self.prep), nbytes, stream_of(cb))
        self._cb = cb  # kept alive until the preparation has run

    def reset(self) -> None:
        self.len = 0
        self.n_base = 0

    def _rebuild(self, n: int) -> None:
        """Main index over the first n cached keys; the tail starts empty."""
        r = self.router
        if n > 0:
            self.offsets, post = kernels.build_index(self.k_codes[:, :, :n].contiguous(), r.num_codebook)
            self.postings = post
        self.n_base = n
        self.rebuilds += 1

    @torch.no_grad()
    def step(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
             causal_attention: bool = False, return_indices: bool = False):
        """Attend the m new tokens' queries ``q [B, m, h_q, d]`` over the cache
        after appending their keys and values ``k, v [B, m, h_kv, d]``.

        Returns ``[B, m, h_q, d]`` (and the int32 ``[B, m, h_kv, top_k]``
        selections, keys ascending, with ``return_indices``).  With
        ``causal_attention`` selected keys past a query's position are dropped
        in the attention; the default (False) attends every selected index, as
        SSAAttention's default does.  A step's rows equal the whole-sequence
        forward's rows when both use the same setting (only rows below top_k,
        whose filler can hold later keys, depend on it)."""
        r = self.router
        B, m = q.shape[0], q.shape[1]
        n0, n = self.len, self.len + m
        if n > self.max_len:
            raise ValueError(f"cache full: {n} tokens > max_len {self.max_len}")
        if k.shape[1] != m or v.shape[1] != m:
            raise ValueError("q, k and v must hold the same new tokens")
        if B != self.batch:
            raise ValueError(f"batch {B} != the cache's {self.batch}")
        if m == 0:
            empty = q.new_empty(q.shape)
            return (empty, torch.empty(B, 0, r.num_kv_heads, r.top_k, dtype=torch.int32,
                                       device=q.device)) if return_indices else empty
        if 2 * m > self.tail_tokens or q.dtype not in (torch.bfloat16, torch.float32):
            return self._chunk(q, k, v, causal_attention, return_indices)
        if n - self.n_base > self.tail_tokens:
            self._rebuild(n0)
        q, k, v = (t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v))
        if k.dtype != self.dtype or v.dtype != self.dtype or q.dtype != self.dtype:
            q, k, v = q.to(self.dtype), k.to(self.dtype), v.to(self.dtype)
        out = torch.empty(q.shape, device=q.device, dtype=q.dtype)
        idx = torch.empty(B, m, r.num_kv_heads, r.top_k, device=q.device, dtype=torch.int32)
        L = _lib.load()
        a, b, d_s, n_c = r.codes_per_query, r.codes_per_key, r.route_dim, r.num_codebook
        ws_bytes = int(L.ssa_decode_workspace_bytes(B, m, r.num_kv_heads, d_s, n_c, a, b, r.top_k))
        ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8)
        d = q.shape[-1]
        score_div = float(torch.tensor(d ** 0.5, dtype=torch.float32))
        kc, vc = self.k, self.v
        call("ssa_decode_step", ptr(q), ptr(k), ptr(v), _lib.elem_dtype(q), B, m, q.shape[2],
             r.num_kv_heads, d, q.stride(0), q.stride(1), q.stride(2), k.stride(0), k.stride(1),
             k.stride(2), v.stride(0), v.stride(1), v.stride(2), ptr(kc), ptr(vc), self.max_len,
             kc.stride(0), kc.stride(1), kc.stride(2), vc.stride(0), vc.stride(1), vc.stride(2), n0,
             ptr(self.w_qr), ptr(self.w_kr), ptr(self.prep), d_s, n_c, a, b, float(r.temperature),
             ptr(self.k_codes), ptr(self.offsets), ptr(self.postings), self.n_base,
             ptr(self.tail_offsets), ptr(self.tail_postings), self.tail_cap, r.top_k, score_div,
             float(d ** 0.5), int(bool(causal_attention)), ptr(idx), ptr(out), _lib.elem_dtype(out),
             out.stride(0), out.stride(1), out.stride(2), ptr(ws), ws_bytes, stream_of(q))
        self.len = n
        return (out, idx) if return_indices else out

    def _chunk(self, q, k, v, causal_attention, return_indices):
        """A long chunk: route it in one batch, rebuild the main index over the
        whole cache, select and attend the chunk's rows."""
        r = self.router
        m = q.shape[1]
        n0, n = self.len, self.len + m
        self.k[:, n0:n] = k
        self.v[:, n0:n] = v
        qc, kc = kernels.route_codes(q, k, r.W_qr.weight, r.W_kr.weight, r.codebook,
                                     r.codes_per_query, r.codes_per_key, r.temperature)
        self.k_codes[:, :, n0:n] = kc
        self._rebuild(n)
        keys, vals = self.k[:, :n], self.v[:, :n]
        idx = kernels.select(q, keys, qc, self.offsets, self.postings, r.codes_per_key, r.top_k,
                             sorted=False, index_dtype=torch.int32, q_pos0=n0)
        out = kernels.sparse_attention(q, keys, vals, idx, None, causal_attention, q_pos0=n0)
        self.len = n
        return (out, idx) if return_indices else out
