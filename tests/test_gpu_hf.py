"""GPU checks of the Qwen2 adapter (ssa_amd.hf) on a small random-init Qwen2.

The patched forward (the HIP RoPE kernel, strided [B, n, h, d] views, batch
folded) must give the same logits as the reference's own structure
(training/train_qwen.py:122-170: transformers' RoPE, per batch element
[n, h, d] contiguous copies, router call with the causal mask, attention) run
with the CPU oracle as router and attention; the router's indices must equal
the oracle's bit for bit on the way.  With routing disabled the adapter must
match transformers' own attention.  Gradients flow through the patched
forward.  Tolerance 1e-4 of max|logits| (fp32 against the float64 oracle).
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")


def _model(dev):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    torch.manual_seed(0)
    cfg = Qwen2Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, max_position_embeddings=512,
                      attn_implementation="eager")
    return Qwen2ForCausalLM(cfg).to(dev).float().eval()


def _reference_structure_forward():
    """training/train_qwen.py:122-170 restated with the CPU oracle in place of the
    router and the attention: transformers' own RoPE, per batch element
    [n, h, d] copies, routing with the causal mask (oracle.router_forward, whose
    indices the module's router must reproduce bit for bit), then the float64
    oracle attention with no mask, as the reference's stage 3."""
    import numpy as np
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb

    import oracle

    def fwd(self, hidden_states, position_embeddings, attention_mask=None, past_key_values=None,
            **kwargs):
        input_shape = hidden_states.shape[:-1]
        hidden_shape = (*input_shape, -1, self.head_dim)
        q = self.q_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        k = self.k_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        v = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        cos, sin = position_embeddings
        q, k = apply_rotary_pos_emb(q, k, cos, sin)
        r = self.ssa_router
        outs = []
        for b in range(input_shape[0]):
            q_b = q[b].transpose(0, 1).contiguous()
            k_b = k[b].transpose(0, 1).contiguous()
            v_b = v[b].transpose(0, 1).contiguous()
            idx, _ = oracle.router_forward(oracle.to_f32(q_b), oracle.to_f32(k_b),
                                           oracle.to_f32(r.W_qr.weight), oracle.to_f32(r.W_kr.weight),
                                           oracle.to_f32(r.codebook), r.codes_per_query,
                                           r.codes_per_key, r.top_k, oracle.MASK_CAUSAL)
            got = r(q_b, k_b, causal_mask=True).cpu().numpy()
            np.testing.assert_array_equal(got, idx)
            att = oracle.sparse_attention(oracle.to_f32(q_b), oracle.to_f32(k_b), oracle.to_f32(v_b), idx)
            outs.append(torch.from_numpy(att).to(hidden_states.device, torch.float32))
        out = torch.stack(outs).reshape(*input_shape, -1).to(hidden_states.dtype)
        return self.o_proj(out), None

    return fwd


def test_qwen2_adapter_matches_reference_structure(dev):
    from transformers.models.qwen2.modeling_qwen2 import Qwen2Attention

    from ssa_amd import hf

    original = Qwen2Attention.forward
    try:
        model = _model(dev)
        ids = torch.randint(0, 512, (2, 96), generator=torch.Generator().manual_seed(1)).to(dev)
        with torch.no_grad():
            dense_ref = model(ids).logits
        hf.integrate_ssa_into_qwen(model, hf.SSAConfig(route_dim=16, num_codebook=64, codes_per_key=4,
                                                       codes_per_query=8, top_k=24), device=dev)
        hf.replace_attention_forward(model)
        with torch.no_grad():
            got = model(ids).logits
        Qwen2Attention.forward = _reference_structure_forward()
        with torch.no_grad():
            ref = model(ids).logits
        tol = 1e-4 * float(ref.abs().max())
        assert float((got - ref).abs().max()) <= tol

        # routing disabled: the adapter's dense path equals transformers' eager attention
        hf.replace_attention_forward(model)
        for m in model.modules():
            if isinstance(m, Qwen2Attention):
                m._ssa_enabled = False
        with torch.no_grad():
            dense = model(ids).logits
        assert float((dense - dense_ref).abs().max()) <= 1e-4 * float(dense_ref.abs().max())

        # gradients through the SSA path
        for m in model.modules():
            if isinstance(m, Qwen2Attention):
                m._ssa_enabled = True
        model.train()
        model(ids).logits.float().pow(2).mean().backward()
        for m in model.modules():
            if isinstance(m, Qwen2Attention):
                for proj in (m.q_proj, m.k_proj, m.v_proj, m.o_proj):
                    assert proj.weight.grad is not None and torch.isfinite(proj.weight.grad).all()
                assert float(m.q_proj.weight.grad.abs().max()) > 0
    finally:
        Qwen2Attention.forward = original
