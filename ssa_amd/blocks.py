"""Block-granular selections and attention (ssa/triton_kernel.py).

The reference's block-sparse path groups queries and keys into blocks of
``block_size`` positions: ``convert_indices_to_blocks`` (:226-294) turns a
router's token selections into the key blocks each query block references most
often, and ``ssa_triton_attention`` (:141-223) attends every query of a block
to all keys of its listed blocks, causally.  Both run here as HIP kernels
(``ssa_block_indices``, ``ssa_block_sparse_attention``); the attention reuses
the token path's kernels with the blocks expanded to keys on load.

Differences from the reference: equal reference counts rank by lower block id
(torch.topk leaves that order unspecified), and the softmax is exact and
normalised (the reference kernel's running rescale and missing division by the
row sum make its outputs wrong, and it runs P.V in fp16).
"""

from __future__ import annotations

from typing import Optional

import torch

from . import kernels


def _batched(x: torch.Tensor, rank: int):
    return (x.unsqueeze(0), True) if x.dim() == rank else (x, False)


def convert_indices_to_blocks(indices: torch.Tensor, block_size: int) -> torch.Tensor:
    """[seq_len, num_kv_heads, top_k] token indices -> int64
    [ceil(seq_len / block_size), num_kv_heads, min(top_k, n_blocks)] key-block
    indices (ssa/triton_kernel.py:226-294); a leading batch dimension is kept."""
    idx, single = _batched(indices, 3)
    out = kernels.block_indices(idx, block_size)
    return out[0] if single else out


def block_sparse_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                           block_indices: torch.Tensor, block_size: int = 64,
                           scale: Optional[float] = None) -> torch.Tensor:
    """q [seq_len, h_q, d], k/v [seq_len, h_kv, d], block_indices
    [ceil(seq_len / block_size), h_kv, n_k_blocks] -> [seq_len, h_q, d]
    (ssa/triton_kernel.py:141-223; scale defaults to 1/sqrt(d)).  A leading
    batch dimension is kept."""
    qb, single = _batched(q, 3)
    kb, _ = _batched(k, 3)
    vb, _ = _batched(v, 3)
    bb, _ = _batched(block_indices, 3)
    out_dtype = qb.dtype
    if qb.dtype == torch.float16:  # fp16 widens exactly to fp32 (the kernels take f32 / bf16)
        qb, kb, vb = qb.float(), kb.float(), vb.float()
    qb, kb, vb = (t if t.stride(-1) == 1 else t.contiguous() for t in (qb, kb, vb))
    d = qb.shape[-1]
    scale_div = (d ** 0.5) if scale is None else 1.0 / scale
    out = kernels.block_sparse_attention(qb, kb, vb, bb, block_size, scale_div)
    if out.dtype != out_dtype:
        out = out.to(out_dtype)
    return out[0] if single else out


def ssa_triton_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                         block_indices: torch.Tensor, block_size: int = 64,
                         scale: Optional[float] = None) -> torch.Tensor:
    """The reference launcher's name and signature (ssa/triton_kernel.py:141-148):
    the same computation as block_sparse_attention (HIP kernels, no Triton), for
    callers written against the reference."""
    return block_sparse_attention(q, k, v, block_indices, block_size, scale)
