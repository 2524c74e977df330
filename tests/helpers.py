"""Seeded input generators shared by the tests (CPU tensors; move to the GPU as needed)."""

from __future__ import annotations

import numpy as np
import torch


def randn(shape, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


def clustered_qk(n, h_q, h_kv, d, n_clusters, sigma, seed, dtype=torch.float32):
    """Q, K from a per-KV-head Gaussian mixture: centres ~ N(0, I_d), one cluster id
    per (token, kv head) shared by the key and its g query heads, noise sigma."""
    g = torch.Generator().manual_seed(seed)
    grp = h_q // h_kv
    centres = torch.randn(h_kv, n_clusters, d, generator=g)
    z = torch.randint(0, n_clusters, (n, h_kv), generator=g)
    kc = centres[torch.arange(h_kv)[None, :], z]            # [n, h_kv, d]
    k = kc + sigma * torch.randn(n, h_kv, d, generator=g)
    qc = kc.repeat_interleave(grp, dim=1)                     # [n, h_q, d]
    q = qc + sigma * torch.randn(n, h_q, d, generator=g)
    return q.to(dtype), k.to(dtype)


def router_params(d, d_s, h_kv, n_c, seed):
    """W_qr, W_kr, codebook with CodebookRouter's default init under a seed."""
    torch.manual_seed(seed)
    w_qr = torch.nn.Linear(d, d_s, bias=False).weight.detach().clone()
    w_kr = torch.nn.Linear(d, d_s, bias=False).weight.detach().clone()
    cb = torch.randn(h_kv, n_c, d_s) / d_s**0.5
    return w_qr, w_kr, cb


def f32(t):
    return np.ascontiguousarray(t.detach().to("cpu", torch.float32).numpy())
