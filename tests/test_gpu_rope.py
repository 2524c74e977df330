"""The HIP rotary-embedding kernel (ssa_rope) against the oracle, bit for bit.

Cases: the reference layer's call (angle row = head, rot = d/2,
ssa/ssa_layer.py:115-117 with ssa/utils.py:7-41) in fp32, bf16 with the fp32
table; the Hugging Face Qwen2 call (angle row = position, rot = d, bf16 tables,
training/train_qwen.py:134-135); per-batch tables, strided [B, h, n, d] views,
in place, head dims that take the scalar path, and the inverse.  The same
kernel must also equal the reference op sequence run by torch on the GPU, and
its autograd must equal torch's autograd of that sequence.
"""

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import randn

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _head_tables(freqs, h, d):
    ang = freqs[:h, : d // 2]
    return ang.cos(), ang.sin()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("d", [64, 128, 40, 8])
def test_rope_by_head_bit_exact(dev, dtype, d):
    from ssa_amd import kernels, precompute_rope_freqs

    _say(f"rope by head dtype={dtype} d={d}")
    B, n, h = 2, 37, 8
    x = randn((B, n, h, d), 11, dtype).to(dev)
    cos, sin = _head_tables(precompute_rope_freqs(d, n, 1e4), h, d)
    got = kernels.rope(x, cos.to(dev), sin.to(dev), d // 2, by_head=True)
    ref = oracle.rope(oracle.to_f32(x), cos.numpy(), sin.numpy(), d // 2, True)
    if dtype == torch.bfloat16:  # fp32 arithmetic (promotion), one rounding at the end
        ref = oracle.bf16_round(ref)
    np.testing.assert_array_equal(got.float().cpu().numpy(), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("d", [128, 64, 36])
def test_rope_by_position_bit_exact(dev, dtype, d):
    """Positional RoPE over every feature with per-batch [B, n, d] tables in
    x's type (the Hugging Face layout), on strided [B, h, n, d] storage."""
    from ssa_amd import kernels

    _say(f"rope by position dtype={dtype} d={d}")
    B, h, n = 2, 4, 50
    store = randn((B, h, n, d), 12, dtype).to(dev)
    x = store.transpose(1, 2)                      # [B, n, h, d] view, strided
    inv = 1.0 / (1e6 ** (torch.arange(0, d, 2).float() / d))
    pos = torch.stack([torch.arange(n), torch.arange(n) + 100]).float()
    f = pos[..., None] * inv
    emb = torch.cat([f, f], -1)
    cos, sin = emb.cos().to(dtype), emb.sin().to(dtype)
    got = kernels.rope(x, cos.to(dev), sin.to(dev), d, by_head=False)
    ref = oracle.rope(oracle.to_f32(x), oracle.to_f32(cos), oracle.to_f32(sin), d, False,
                      round_bf16=dtype == torch.bfloat16)
    np.testing.assert_array_equal(got.float().cpu().numpy(), ref)
    inv_got = kernels.rope(x, cos.to(dev), sin.to(dev), d, by_head=False, inverse=True)
    inv_ref = oracle.rope(oracle.to_f32(x), oracle.to_f32(cos), oracle.to_f32(sin), d, False,
                          round_bf16=dtype == torch.bfloat16, inverse=True)
    np.testing.assert_array_equal(inv_got.float().cpu().numpy(), inv_ref)


def test_rope_in_place_and_fp32_output(dev):
    from ssa_amd import kernels, precompute_rope_freqs

    _say("rope in place / fp32 output")
    B, n, h, d = 1, 64, 8, 128
    x = randn((B, n, h, d), 13, torch.bfloat16).to(dev)
    cos, sin = _head_tables(precompute_rope_freqs(d, n, 1e6), h, d)
    cos, sin = cos.to(dev), sin.to(dev)
    out32 = torch.empty(x.shape, device=dev, dtype=torch.float32)
    kernels.rope(x, cos, sin, d // 2, True, out=out32)
    ref = oracle.rope(oracle.to_f32(x), oracle.to_f32(cos), oracle.to_f32(sin), d // 2, True)
    np.testing.assert_array_equal(out32.cpu().numpy(), ref)
    y = x.clone()
    kernels.rope(y, cos, sin, d // 2, True, out=y)
    np.testing.assert_array_equal(y.float().cpu().numpy(), oracle.bf16_round(ref))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rope_equals_torch_op_sequence_on_gpu(dev, dtype):
    """The reference's apply_rope op sequence run by torch on the same GPU
    (SSAAttention's call) and transformers' apply_rotary_pos_emb (bf16 tables)."""
    from ssa_amd import kernels, precompute_rope_freqs
    from ssa_amd.utils import apply_rope

    _say(f"rope vs torch on gpu dtype={dtype}")
    n, h, d = 40, 8, 64
    x = randn((n, h, d), 14, torch.float32).to(dev)
    freqs = precompute_rope_freqs(d, n, 1e4, device=dev)
    ref = apply_rope(x, freqs)
    cos, sin = _head_tables(freqs, h, d)
    got = kernels.rope(x[None], cos, sin, d // 2, True)[0]
    assert torch.equal(got, ref)
    tr = pytest.importorskip("transformers.models.qwen2.modeling_qwen2")
    q = randn((2, h, n, d), 15, dtype).to(dev)
    emb = torch.cat([freqs[:, : d // 2], freqs[:, : d // 2]], -1)[None].expand(2, n, d)
    c, s = emb.cos().to(dtype).contiguous(), emb.sin().to(dtype).contiguous()
    qr, _ = tr.apply_rotary_pos_emb(q, q, c, s)
    got = kernels.rope(q.transpose(1, 2), c, s, d, False)
    assert torch.equal(got, qr.transpose(1, 2))


def test_rope_autograd_equals_torch_autograd(dev):
    """rope_rows' backward (the kernel's transpose) equals torch's autograd of the
    reference op sequence, bit for bit in fp32."""
    from ssa_amd import precompute_rope_freqs
    from ssa_amd.ssa_layer import head_rope_tables, rope_rows
    from ssa_amd.utils import apply_rope

    _say("rope autograd")
    B, n, h, d = 2, 24, 8, 64
    x = randn((B, n, h, d), 16).to(dev).requires_grad_()
    g = randn((B, n, h, d), 17).to(dev)
    freqs = precompute_rope_freqs(d, n, 1e4, device=dev)
    cos, sin = head_rope_tables(freqs, n, h, d)
    rope_rows(x, cos, sin, d // 2, True).backward(g)
    xr = x.detach().clone().requires_grad_()
    torch.stack([apply_rope(xr[b], freqs) for b in range(B)]).backward(g)
    assert torch.equal(x.grad, xr.grad)


def test_rope_rejects(dev):
    from ssa_amd import kernels

    x = torch.zeros(1, 4, 2, 8, device=dev)
    t = torch.zeros(4, 8, device=dev)
    with pytest.raises(Exception, match="rot"):
        kernels.rope(x, t, t, 3, False)
    with pytest.raises(Exception, match="rows"):
        kernels.rope(x, t[:3], t[:3], 8, False)
