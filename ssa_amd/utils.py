"""Input-preparation helpers with the reference's semantics (ssa/utils.py).

These run as ordinary PyTorch ops on whatever device the tensors live on; they
are not part of the HIP hot path.
"""

from __future__ import annotations

import torch


def apply_rope(x: torch.Tensor, freqs: torch.Tensor) -> torch.Tensor:
    """Rotary embedding with the reference semantics (ssa/utils.py:7-41).

    The rotation angle is indexed by ``x.shape[-2]`` (the second-to-last axis),
    only the first ``head_dim // 2`` features rotate, and the rotate-half pairs
    are ``(j, j + head_dim // 4)``.  With ``x`` of shape ``[n, heads, d]`` (how
    SSAAttention calls it) the angle therefore follows the head index.
    """
    rows = x.shape[-2]
    half = x.shape[-1] // 2
    ang = freqs[:rows, :half]
    cos, sin = ang.cos(), ang.sin()
    for _ in range(x.dim() - 2):
        cos = cos.unsqueeze(0)
        sin = sin.unsqueeze(0)
    x_rot, x_pass = x[..., :half], x[..., half:]
    return torch.cat([x_rot * cos + _rotate_half(x_rot) * sin, x_pass], dim=-1)


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    """[x1, x2] -> [-x2, x1] over the last axis (ssa/utils.py:44-48)."""
    cut = x.shape[-1] // 2
    return torch.cat([-x[..., cut:], x[..., :cut]], dim=-1)


def precompute_rope_freqs(head_dim: int, seq_len: int, theta: float = 10000.0,
                          device=None) -> torch.Tensor:
    """Angles ``[seq_len, head_dim // 2]`` (ssa/utils.py:51-72).

    ``inv_freq[m] = theta ** -(2m / (head_dim // 2))`` for ``m < head_dim // 4``,
    multiplied by the position and duplicated to width ``head_dim // 2``.
    """
    half = head_dim // 2
    inv = 1.0 / (theta ** (torch.arange(0, half, 2, device=device).float() / half))
    pos = torch.arange(seq_len, device=device, dtype=torch.float32)
    ang = torch.outer(pos, inv)
    return torch.cat([ang, ang], dim=-1)


def build_causal_mask(seq_len: int, device=None) -> torch.Tensor:
    """Lower-triangular bool mask, True where attention is allowed (ssa/utils.py:75-86).

    The returned tensor carries ``_ssa_causal = True`` so that CodebookRouter can
    use its causal fast path without reading the n^2 bytes; any other mask is
    honoured element by element.
    """
    m = torch.ones(seq_len, seq_len, device=device, dtype=torch.bool).tril_()
    m._ssa_causal = True
    return m


def expand_kv_for_gqa(kv: torch.Tensor, num_q_heads: int, num_kv_heads: int) -> torch.Tensor:
    """KV heads repeated to num_q_heads (ssa/utils.py:89-106).

    Same layout as the reference helper: the KV heads are tiled, so expanded
    head j is KV head ``j % num_kv_heads``.  The attention functions pair query
    head j with KV head ``j // (num_q_heads // num_kv_heads)`` instead; no
    reference code path calls this helper.
    """
    assert num_q_heads % num_kv_heads == 0, "num_q_heads must be divisible by num_kv_heads"
    g = num_q_heads // num_kv_heads
    return kv.unsqueeze(-3).expand(*kv.shape[:-2], g, kv.shape[-2], kv.shape[-1]).reshape(
        *kv.shape[:-2], num_q_heads, kv.shape[-1])


def validate_indices(indices: torch.Tensor, seq_len: int, max_k: int,
                     name: str = "indices") -> None:
    """Shape and range assertions on candidate indices (ssa/utils.py:109-120)."""
    assert indices.dim() >= 2, f"{name} must have at least 2 dims, got shape {indices.shape}"
    assert indices.shape[-1] <= max_k, f"{name} last dim {indices.shape[-1]} exceeds max_k {max_k}"
    assert indices.max() < seq_len, f"{name} max index {indices.max()} >= seq_len {seq_len}"
    assert indices.min() >= 0, f"{name} min index {indices.min()} < 0"
