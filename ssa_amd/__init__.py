"""ssa_amd -- SSA (Sub-quadratic Selective Attention) forward path for AMD
Instinct MI355X (gfx950).

Re-exports the reference package's public names (ssa/__init__.py:13-28):

    CodebookRouter          stages 1-2: codebook routing + candidate selection
    sparse_exact_attention  stage 3: exact attention over selected keys
    dense_attention         dense SDPA (comparison / k = n checks)
    SSAAttention            drop-in attention layer
    ToyTransformerBlock     LayerNorm + SSAAttention + FFN block
    apply_rope, precompute_rope_freqs, build_causal_mask, expand_kv_for_gqa

The hot path runs in libssa_hip.so (hand-written HIP for gfx950) through a C
ABI (include/ssa_hip.h); there is no CPU or PyTorch fallback for it.
"""

from .attention import dense_attention, sparse_exact_attention
from .router import CodebookRouter
from .ssa_layer import SSAAttention, ToyTransformerBlock
from .utils import (
    apply_rope,
    build_causal_mask,
    expand_kv_for_gqa,
    precompute_rope_freqs,
    validate_indices,
)

__all__ = [
    "CodebookRouter",
    "sparse_exact_attention",
    "dense_attention",
    "SSAAttention",
    "ToyTransformerBlock",
    "apply_rope",
    "precompute_rope_freqs",
    "build_causal_mask",
    "expand_kv_for_gqa",
]
