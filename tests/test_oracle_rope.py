"""Pins of the oracle's rotary embedding (oracle.rope), CPU only.

The restatement must equal, bit for bit, the two op sequences it stands for:
the reference's apply_rope (ssa/utils.py:7-48, here as this package's torch
restatement, itself pinned by the closed-form tests in test_api_cpu.py) called
on [n, heads, d] as SSAAttention does (ssa/ssa_layer.py:115-117), and
transformers' apply_rotary_pos_emb that the Qwen2 path runs
(training/train_qwen.py:134-135), in fp32 and bf16.  Closed forms pin it
independently of both, and a planted convention mistake must fail.
"""

import numpy as np
import pytest
import torch

import oracle
from ssa_amd.utils import apply_rope, precompute_rope_freqs


def _x(shape, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


@pytest.mark.parametrize("n,h,d", [(16, 8, 64), (5, 4, 40), (33, 32, 128)])
def test_rope_equals_reference_apply_rope_by_head(n, h, d):
    """apply_rope on [n, h, d]: angle row = head, rot = d/2 (fp32)."""
    x = _x((n, h, d), 1)
    freqs = precompute_rope_freqs(d, max(n, h), 1e4)
    ref = apply_rope(x, freqs).numpy()
    ang = freqs[:h, : d // 2]
    got = oracle.rope(x.numpy()[None], ang.cos().numpy(), ang.sin().numpy(), d // 2, by_head=True)[0]
    np.testing.assert_array_equal(got, ref)


def test_rope_bf16_input_fp32_table_promotes():
    """bf16 x with the fp32 table: torch promotes to fp32, one rounding at the end."""
    n, h, d = 12, 8, 64
    x = _x((n, h, d), 2, torch.bfloat16)
    freqs = precompute_rope_freqs(d, n, 1e6)
    ref = apply_rope(x, freqs)
    assert ref.dtype == torch.float32
    ang = freqs[:h, : d // 2]
    got = oracle.rope(x.float().numpy()[None], ang.cos().numpy(), ang.sin().numpy(), d // 2, True)[0]
    np.testing.assert_array_equal(got, ref.numpy())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rope_equals_transformers_apply_rotary_pos_emb(dtype):
    """Hugging Face Qwen2 RoPE: angle row = position, rot = d; bf16 q with bf16
    tables rounds every op to bf16."""
    tr = pytest.importorskip("transformers.models.qwen2.modeling_qwen2")
    B, h, n, d = 2, 4, 24, 64
    q = _x((B, h, n, d), 3, dtype)
    inv = 1.0 / (1e6 ** (torch.arange(0, d, 2).float() / d))
    pos = torch.stack([torch.arange(n), torch.arange(n) + 7]).float()
    f = pos[..., None] * inv
    emb = torch.cat([f, f], -1)
    cos, sin = emb.cos().to(dtype), emb.sin().to(dtype)
    ref, _ = tr.apply_rotary_pos_emb(q, q, cos, sin)
    got = oracle.rope(q.transpose(1, 2).float().numpy(), cos.float().numpy(), sin.float().numpy(),
                      d, by_head=False, round_bf16=dtype == torch.bfloat16)
    np.testing.assert_array_equal(got, ref.transpose(1, 2).float().numpy())


def test_rope_closed_forms():
    """Zero angle is the identity, a quarter turn is rotate_half, pair norms are
    kept, features past rot pass through, and the inverse undoes the rotation."""
    B, n, h, d = 1, 6, 3, 32
    x = _x((B, n, h, d), 4).numpy()
    one, zero = np.ones((n, d), np.float32), np.zeros((n, d), np.float32)
    np.testing.assert_array_equal(oracle.rope(x, one, zero, d, False), x)
    rh = np.concatenate([-x[..., d // 2:], x[..., : d // 2]], -1)
    np.testing.assert_array_equal(oracle.rope(x, zero, one, d, False), rh)
    ang = np.random.default_rng(5).uniform(-3, 3, (n, d // 4)).astype(np.float32)
    ang = np.concatenate([ang, ang], -1)
    y = oracle.rope(x, np.cos(ang), np.sin(ang), d // 2, False)
    r = d // 4
    nx = np.hypot(x[..., :r].astype(np.float64), x[..., r: 2 * r])
    ny = np.hypot(y[..., :r].astype(np.float64), y[..., r: 2 * r])
    np.testing.assert_allclose(ny, nx, rtol=1e-6)
    np.testing.assert_array_equal(y[..., d // 2:], x[..., d // 2:])
    back = oracle.rope(y, np.cos(ang), np.sin(ang), d // 2, False, inverse=True)
    np.testing.assert_allclose(back, x, rtol=1e-5, atol=1e-6)


def test_rope_checks_catch_planted_mistakes():
    """A wrong pairing convention (all d features rotated where the reference
    rotates d/2), or the angle taken by position instead of head, fails the
    comparison with the reference's op sequence."""
    n, h, d = 16, 8, 64
    x = _x((n, h, d), 6)
    freqs = precompute_rope_freqs(d, n, 1e4)
    ref = apply_rope(x, freqs).numpy()
    ang = freqs[:, : d // 2]
    wrong_rot = oracle.rope(x.numpy()[None], torch.cat([ang, ang], -1).cos().numpy(),
                            torch.cat([ang, ang], -1).sin().numpy(), d, by_head=True)[0]
    assert not np.array_equal(wrong_rot, ref)
    wrong_axis = oracle.rope(x.numpy()[None], ang.cos().numpy(), ang.sin().numpy(), d // 2,
                             by_head=False)[0]
    assert not np.array_equal(wrong_axis, ref)


def test_bf16_round_matches_torch():
    v = _x((4096,), 7).numpy() * np.float32(1e3)
    v[:4] = [0.0, -0.0, np.inf, -np.inf]
    np.testing.assert_array_equal(oracle.bf16_round(v),
                                  torch.from_numpy(v).to(torch.bfloat16).float().numpy())
