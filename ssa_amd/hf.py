"""Hugging Face Qwen2 adapter (training/train_qwen.py:44-170 of the reference).

``integrate_ssa_into_qwen`` attaches a ``CodebookRouter`` to every
``Qwen2Attention`` (attributes ``ssa_router`` and ``_ssa_enabled``, as the
reference names them) and ``replace_attention_forward`` patches
``Qwen2Attention.forward``.  The patched forward keeps the reference's
semantics (routing on post-RoPE q and k, causal routing, stage 3 without a mask
unless ``_ssa_causal_attention`` is set on the module) but not its data
movement: the reference transposes each batch element of the ``[B, h, n, d]``
states to ``[n, h, d]`` with ``.contiguous()`` copies and loops over the
batch; here the kernels read the ``[B, n, h, d]`` views of the same storage
through their strides, the whole batch in one launch per stage, and the
attention output is already in the ``[B, n, h*d]`` layout ``o_proj`` takes.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .attention import dense_attention, sparse_exact_attention
from .router import CodebookRouter
from .ssa_layer import rope_rows
from .utils import build_causal_mask


@dataclass
class SSAConfig:
    """SSA settings attached to each attention layer (training/train_qwen.py:44-51)."""

    route_dim: int = 32
    num_codebook: int = 4096
    codes_per_key: int = 4
    codes_per_query: int = 16
    top_k: int = 2048


def integrate_ssa_into_qwen(model, ssa_config: SSAConfig, device="cuda"):
    """Attach a CodebookRouter to each Qwen2Attention (training/train_qwen.py:54-102).

    The router takes the module's head layout and the model's dtype; routing is
    enabled (``_ssa_enabled = True``).  Returns the model."""
    from transformers.models.qwen2.modeling_qwen2 import Qwen2Attention

    for _, module in model.named_modules():
        if isinstance(module, Qwen2Attention):
            router = CodebookRouter(
                head_dim=module.head_dim,
                route_dim=ssa_config.route_dim,
                num_kv_heads=module.config.num_key_value_heads,
                num_codebook=ssa_config.num_codebook,
                codes_per_key=ssa_config.codes_per_key,
                codes_per_query=ssa_config.codes_per_query,
                top_k=ssa_config.top_k,
            ).to(device=device, dtype=module.q_proj.weight.dtype)
            module.ssa_router = router
            module._ssa_enabled = True
    return model


def ssa_attention_bnhd(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                       router: CodebookRouter, causal_attention: bool = False) -> torch.Tensor:
    """SSA over ``[B, n, heads, d]`` views (any strides with a contiguous last
    dimension): routing with the causal mask, then exact attention over the
    selected keys.  Returns ``[B, n, h_q, d]`` (contiguous).  Differentiable in
    query, key and value."""
    res = router.route(query, key, causal_mask=True, hard=True, sorted=False,
                       index_dtype=torch.int32, with_order=True, with_prefix=True)
    return sparse_exact_attention(query, key, value, res.indices, causal=causal_attention,
                                  check_indices=False, row_order=res.order, row_prefix=res.prefix,
                                  routing=res.routing())


def replace_attention_forward(model=None):
    """Patch ``Qwen2Attention.forward`` with SSA (training/train_qwen.py:105-170).

    Modules without ``ssa_router`` or with ``_ssa_enabled`` false take dense
    causal attention, as in the reference.  A key/value cache longer than the
    query block is not supported (the reference's routing needs n_q == n_k too)."""
    from transformers.cache_utils import Cache
    from transformers.models.qwen2.modeling_qwen2 import Qwen2Attention

    def ssa_forward(self, hidden_states, position_embeddings, attention_mask=None,
                    past_key_values=None, **kwargs):
        input_shape = hidden_states.shape[:-1]
        hidden_shape = (*input_shape, -1, self.head_dim)
        cos, sin = position_embeddings
        # apply_rotary_pos_emb (training/train_qwen.py:134-135) on the HIP kernel:
        # positional angles, every feature rotated, the same rounded ops; the
        # [B, n, h, d] projections are read where they lie and the results are
        # handed on as [B, h, n, d] views
        q = rope_rows(self.q_proj(hidden_states).view(hidden_shape), cos, sin, self.head_dim,
                      by_head=False).transpose(1, 2)
        k = rope_rows(self.k_proj(hidden_states).view(hidden_shape), cos, sin, self.head_dim,
                      by_head=False).transpose(1, 2)
        v = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        if past_key_values is not None and isinstance(past_key_values, Cache):
            k, v = past_key_values.update(k, v, self.layer_idx)
        if k.shape[-2] != q.shape[-2]:
            raise NotImplementedError(
                "SSA attention needs as many keys as queries (no decode against a longer cache)")
        # [B, h, n, d] -> [B, n, h, d] views of the same storage
        qv, kv, vv = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
        if hasattr(self, "ssa_router") and getattr(self, "_ssa_enabled", False):
            out = ssa_attention_bnhd(qv, kv, vv, self.ssa_router,
                                     causal_attention=getattr(self, "_ssa_causal_attention", False))
        else:
            n = qv.shape[1]
            mask = build_causal_mask(n, device=hidden_states.device)
            out = torch.stack([dense_attention(qv[b], kv[b], vv[b], causal_mask=mask)
                               for b in range(qv.shape[0])])
        out = out.reshape(*input_shape, -1).to(hidden_states.dtype)
        return self.o_proj(out), None

    Qwen2Attention.forward = ssa_forward
    return model
