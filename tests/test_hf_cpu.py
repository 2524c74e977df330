"""CPU checks of the Qwen2 adapter's host logic (ssa_amd.hf): router attachment
with the module's head layout (training/train_qwen.py:54-102), the class patch,
and that the SSA path refuses CPU tensors (no CPU fallback)."""

from __future__ import annotations

import pytest
import torch

transformers = pytest.importorskip("transformers")


def _model():
    from transformers import Qwen2Config, Qwen2ForCausalLM

    torch.manual_seed(0)
    cfg = Qwen2Config(vocab_size=128, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64,
                      attn_implementation="eager")
    return Qwen2ForCausalLM(cfg)


def test_integrate_attaches_routers():
    from transformers.models.qwen2.modeling_qwen2 import Qwen2Attention

    from ssa_amd import hf

    model = hf.integrate_ssa_into_qwen(_model(), hf.SSAConfig(route_dim=8, num_codebook=32, top_k=8),
                                       device="cpu")
    mods = [m for m in model.modules() if isinstance(m, Qwen2Attention)]
    assert len(mods) == 2
    for m in mods:
        r = m.ssa_router
        assert m._ssa_enabled is True
        assert r.codebook.shape == (2, 32, 8)
        assert r.W_qr.weight.shape == (8, 16) and r.W_kr.weight.shape == (8, 16)
        assert r.top_k == 8 and r.codes_per_key == 4 and r.codes_per_query == 16


def test_patch_and_cpu_refusal():
    from transformers.models.qwen2.modeling_qwen2 import Qwen2Attention

    from ssa_amd import hf

    original = Qwen2Attention.forward
    try:
        model = hf.integrate_ssa_into_qwen(_model(), hf.SSAConfig(route_dim=8, num_codebook=32, top_k=8),
                                           device="cpu")
        hf.replace_attention_forward(model)
        assert Qwen2Attention.forward is not original
        with pytest.raises(RuntimeError, match="HIP"):
            model(torch.zeros(1, 8, dtype=torch.long))
    finally:
        Qwen2Attention.forward = original
