"""ssa_select_block_noalloc (the selection with its workspace in the library's
static device array) against ssa_select_block with a caller workspace, through
the C ABI: identical indices and stats on two calls in a row, the second with
a smaller input (the array keeps the first call's contents), in both output
orders, plus the host-side rejection of a shape whose minimum workspace does
not fit the array."""

import ctypes

import pytest
import torch

from tests.helpers import clustered_qk, router_params

pytestmark = pytest.mark.gpu


def _inputs(dev, n, h_q, h_kv, d, n_c, a, b, seed):
    from ssa_amd import kernels

    q, k = clustered_qk(n, h_q, h_kv, d, 8, 0.3, seed=seed)
    w_qr, w_kr, cb = router_params(d, 32, h_kv, n_c, seed=seed + 1)
    q = q.to(torch.bfloat16).unsqueeze(0).to(dev)
    k = k.to(torch.bfloat16).unsqueeze(0).to(dev)
    qc, kc = kernels.route_codes(q, k, w_qr.to(dev), w_kr.to(dev), cb.to(dev), a, b)
    off, post = kernels.build_index(kc, n_c)
    return q, k, qc, off, post


def _call(L, name, q, k, qc, off, post, b, top_k, sorted_, ws=None):
    from ssa_amd import _lib

    B, n, h_q, d = q.shape
    h_kv = k.shape[2]
    a = qc.shape[-1]
    n_c = off.shape[-1] - 1
    out = torch.full((B, n, h_kv, top_k), -7, device=q.device, dtype=torch.int32)
    stats = torch.full((B, h_kv, n, 2), -7, device=q.device, dtype=torch.int32)
    prefix = torch.full((B, h_kv, n), -7, device=q.device, dtype=torch.int32)
    args = [_lib.ptr(q), _lib.ptr(k), _lib.DTYPE_BF16, B, n, n, 0, h_q, h_kv, d,
            q.stride(0), q.stride(1), q.stride(2), k.stride(0), k.stride(1), k.stride(2),
            _lib.ptr(qc), a, _lib.ptr(off), _lib.ptr(post), n_c, b, top_k, _lib.MASK_CAUSAL, None,
            0, 0, float(d ** 0.5), int(sorted_), None, _lib.ptr(out), _lib.INDEX_I32,
            _lib.ptr(stats), _lib.ptr(prefix)]
    if ws is not None:
        args += [_lib.ptr(ws), ws.numel()]
    args.append(_lib.stream_of(q))
    st = getattr(L, name)(*args)
    assert st == _lib.SSA_OK, (L.ssa_last_error() or b"").decode()
    return out, stats, prefix


@pytest.mark.parametrize("sorted_", [False, True])
def test_noalloc_select_equals_workspace_select_twice(dev, sorted_):
    from ssa_amd import _lib

    L = _lib.load()
    cases = [dict(n=12000, h_q=16, h_kv=4, d=128, n_c=256, a=16, b=4, top_k=256, seed=3),
             dict(n=2500, h_q=8, h_kv=2, d=64, n_c=128, a=8, b=4, top_k=96, seed=5)]
    for c in cases:
        print(f"no-alloc select sorted={sorted_} {c}", flush=True)
        top_k = c.pop("top_k")
        q, k, qc, off, post = _inputs(dev, **c)
        b = c["b"]
        nbytes = L.ssa_select_workspace_bytes(1, c["n"], c["h_kv"], top_k)
        ws = torch.empty(nbytes, device=dev, dtype=torch.uint8)
        ref, ref_st, ref_x = _call(L, "ssa_select_block", q, k, qc, off, post, b, top_k, sorted_, ws)
        got, got_st, got_x = _call(L, "ssa_select_block_noalloc", q, k, qc, off, post, b, top_k,
                                   sorted_)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
        assert torch.equal(got_st, ref_st)
        assert torch.equal(got_x, ref_x)
        if not sorted_:
            assert int((ref_st[..., 0] > top_k).sum()) > 0, "the case should list heavy rows"


def test_noalloc_select_rejects_oversized_shape(dev):
    from ssa_amd import _lib

    L = _lib.load()
    cap = L.ssa_select_noalloc_scratch_bytes()
    assert cap == 64 << 20
    n = 1 << 21
    assert L.ssa_select_workspace_bytes(1, n, 2, 0) > cap
    fake = ctypes.c_void_p(1 << 20)
    st = L.ssa_select_block_noalloc(fake, fake, _lib.DTYPE_BF16, 1, n, n, 0, 8, 2, 128, 0, 0, 0, 0,
                                    0, 0, fake, 16, fake, fake, 4096, 4, 512, _lib.MASK_CAUSAL,
                                    None, 0, 0, 11.3, 0, None, fake, _lib.INDEX_I32, None, None, None)
    assert st == _lib.SSA_ERR_WORKSPACE
    assert "scratch" in (L.ssa_last_error() or b"").decode()
