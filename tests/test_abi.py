"""C-ABI checks that need no GPU: libssa_hip.so loads, exports every function
include/ssa_hip.h declares with the argument types the ctypes bindings use, and
its host-side argument checks return the documented status before any HIP
call (every call below fails validation or is an empty no-op, so nothing is
launched).  Pointers passed here are never dereferenced on the host."""

import ctypes
import os
import re

import pytest

from ssa_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ssa_hip.h")

_CTYPE = {
    "int": ctypes.c_int,
    "int64_t": ctypes.c_int64,
    "size_t": ctypes.c_size_t,
    "float": ctypes.c_float,
    "const char*": ctypes.c_char_p,
}


def _declarations():
    """name -> (return type, [parameter types]) parsed from the header."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    decls = {}
    for m in re.finditer(r"^([A-Za-z_][\w\s\*]*?)\s*\b(ssa_\w+)\s*\(([^)]*)\);", text, flags=re.M):
        ret, name, params = m.group(1).strip(), m.group(2), m.group(3)
        types = []
        for p in params.split(","):
            p = " ".join(p.split())
            if p in ("void", ""):
                continue
            types.append(re.sub(r"\s*\w+$", "", p).replace(" *", "*"))
        decls[name] = (ret.replace(" *", "*"), types)
    return decls


def _ctype(c: str):
    if c in _CTYPE:
        return _CTYPE[c]
    if c.endswith("*"):
        return ctypes.c_void_p
    raise AssertionError(f"unmapped C type {c!r}")


@pytest.fixture(scope="module")
def L():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libssa_hip.so not built (run __graft_entry__.build())")
    return _lib.load()


def test_header_parses_every_entry_point():
    decls = _declarations()
    assert len(decls) == len(_lib.SIGNATURES) >= 22
    assert set(decls) == set(_lib.SIGNATURES)


@pytest.mark.parametrize("name", sorted(_lib.SIGNATURES))
def test_export_and_signature(L, name):
    ret, params = _declarations()[name]
    assert hasattr(L, name), f"{name} not exported"
    res, args = _lib.SIGNATURES[name]
    assert res is _ctype(ret), f"{name}: return type {ret}"
    assert [_ctype(p) for p in params] == list(args), f"{name}: parameter types"


def test_status_strings(L):
    assert L.ssa_version() >= 1
    names = [L.ssa_status_str(s).decode() for s in range(5)]
    assert len(set(names)) == 5 and all(names)
    assert L.ssa_status_str(99)


FAKE = ctypes.c_void_p(1 << 20)       # non-null, 16-byte aligned, never dereferenced
MISALIGNED = ctypes.c_void_p((1 << 20) + 8)
NULL = None


def _rope(L, **kw):
    a = dict(x=FAKE, dtype=_lib.DTYPE_BF16, batch=1, n=64, h=8, d=128, x_sb=64 * 8 * 128,
             x_sn=8 * 128, x_sh=128, cos=FAKE, sin=FAKE, table_dtype=_lib.DTYPE_F32, t_sb=0,
             t_sr=64, table_rows=64, rot=64, angle_axis=_lib.ROPE_BY_HEAD, inverse=0, out=FAKE,
             out_dtype=_lib.DTYPE_BF16, o_sb=64 * 8 * 128, o_sn=8 * 128, o_sh=128, stream=NULL)
    a.update(kw)
    st = L.ssa_rope(*a.values())
    return st, (L.ssa_last_error() or b"").decode()


@pytest.mark.parametrize("kw,status,text", [
    (dict(dtype=3), _lib.SSA_ERR_UNSUPPORTED, "types"),
    (dict(rot=63), _lib.SSA_ERR_INVALID_ARGUMENT, "rot"),
    (dict(rot=130), _lib.SSA_ERR_INVALID_ARGUMENT, "rot"),
    (dict(angle_axis=2), _lib.SSA_ERR_INVALID_ARGUMENT, "angle_axis"),
    (dict(table_rows=7), _lib.SSA_ERR_INVALID_ARGUMENT, "rows"),
    (dict(angle_axis=_lib.ROPE_BY_POSITION, table_rows=63), _lib.SSA_ERR_INVALID_ARGUMENT, "rows"),
    (dict(cos=NULL), _lib.SSA_ERR_INVALID_ARGUMENT, "null"),
    (dict(out=FAKE, out_dtype=_lib.DTYPE_F32), _lib.SSA_ERR_INVALID_ARGUMENT, "in place"),
])
def test_rope_rejects(L, kw, status, text):
    st, msg = _rope(L, **kw)
    assert st == status, msg
    assert text in msg


def test_rope_empty_is_noop(L):
    assert _rope(L, n=0, x=NULL, out=NULL, cos=NULL, sin=NULL)[0] == _lib.SSA_OK


def _select(L, **kw):
    a = dict(q=FAKE, k=FAKE, dtype=_lib.DTYPE_BF16, batch=1, n=1024, h_q=32, h_kv=8, d=128,
             q_sb=1024 * 32 * 128, q_sn=32 * 128, q_sh=128, k_sb=1024 * 8 * 128, k_sn=8 * 128,
             k_sh=128, q_codes=FAKE, a=16, offsets=FAKE, postings=FAKE, n_c=4096, b=4, top_k=512,
             mask_mode=_lib.MASK_CAUSAL, mask=NULL, mask_sb=0, mask_si=0, score_div=11.3137,
             sorted=0, row_order=NULL, out=FAKE, out_index_dtype=_lib.INDEX_I64, stats=NULL,
             row_prefix=NULL, workspace=NULL,
             workspace_bytes=0, stream=NULL)
    a.update(kw)
    st = L.ssa_select(*a.values())
    return st, (L.ssa_last_error() or b"").decode()


@pytest.mark.parametrize("kw,status,text", [
    (dict(dtype=7), _lib.SSA_ERR_UNSUPPORTED, "dtype"),
    (dict(h_q=30), _lib.SSA_ERR_INVALID_ARGUMENT, "divisible"),
    (dict(h_q=8 * 17), _lib.SSA_ERR_UNSUPPORTED, "group size"),
    (dict(a=65), _lib.SSA_ERR_UNSUPPORTED, "codes_per_query"),
    (dict(d=100), _lib.SSA_ERR_UNSUPPORTED, "head_dim"),
    (dict(top_k=4097), _lib.SSA_ERR_UNSUPPORTED, "top_k"),
    (dict(top_k=0), _lib.SSA_ERR_INVALID_ARGUMENT, "shape"),
    (dict(mask_mode=3), _lib.SSA_ERR_INVALID_ARGUMENT, "mask_mode"),
    (dict(mask_mode=_lib.MASK_DENSE), _lib.SSA_ERR_INVALID_ARGUMENT, "mask"),
    (dict(out_index_dtype=5), _lib.SSA_ERR_INVALID_ARGUMENT, "out_index_dtype"),
    (dict(score_div=0.0), _lib.SSA_ERR_INVALID_ARGUMENT, "score_div"),
    (dict(q=MISALIGNED), _lib.SSA_ERR_UNSUPPORTED, "aligned"),
    (dict(k_sn=8 * 128 + 4), _lib.SSA_ERR_UNSUPPORTED, "aligned"),
    (dict(postings=NULL), _lib.SSA_ERR_INVALID_ARGUMENT, "null"),
    (dict(n=1 << 29, b=4), _lib.SSA_ERR_UNSUPPORTED, "2^31"),
    (dict(n=1 << 26, b=4), _lib.SSA_ERR_UNSUPPORTED, "LDS"),
    (dict(workspace=FAKE, workspace_bytes=1024), _lib.SSA_ERR_WORKSPACE, "workspace"),
])
def test_select_rejects(L, kw, status, text):
    st, msg = _select(L, **kw)
    assert st == status, msg
    assert text in msg


def test_select_workspace_size(L):
    # counters and per-row lists (at least 16 bytes per row), then 8 bytes per
    # output slot for candidate lists and their scores
    rows = 2 * 8 * 1000
    fixed = L.ssa_select_workspace_bytes(2, 1000, 8, 0)
    assert fixed >= rows * 16
    assert L.ssa_select_workspace_bytes(2, 1000, 8, 64) == fixed + rows * 64 * 8
    assert L.ssa_select_workspace_bytes(2, 1000, 8, 5000) == fixed + rows * 1000 * 8  # k <= n
    assert _select(L, workspace=FAKE, workspace_bytes=L.ssa_select_workspace_bytes(1, 1024, 8, 0),
                   postings=NULL)[0] == _lib.SSA_ERR_INVALID_ARGUMENT


def test_select_empty_is_noop(L):
    assert _select(L, n=0, q=NULL, k=NULL, out=NULL)[0] == _lib.SSA_OK
    assert _select(L, batch=0)[0] == _lib.SSA_OK


def _attention(L, **kw):
    a = dict(q=FAKE, k=FAKE, v=FAKE, dtype=_lib.DTYPE_BF16, batch=1, n=1024, h_q=32, h_kv=8,
             d=128, q_sb=1024 * 32 * 128, q_sn=32 * 128, q_sh=128, k_sb=1024 * 8 * 128,
             k_sn=8 * 128, k_sh=128, v_sb=1024 * 8 * 128, v_sn=8 * 128, v_sh=128, idx=FAKE,
             idx_dtype=_lib.INDEX_I64, top_k=512, idx_sb=1024 * 8 * 512, idx_sn=8 * 512,
             idx_sh=512, scale_div=11.3137, causal=1, row_order=NULL, row_prefix=NULL, out=FAKE,
             out_dtype=_lib.DTYPE_BF16,
             o_sb=1024 * 32 * 128, o_sn=32 * 128, o_sh=128, error_flag=NULL, row_stats=NULL,
             workspace=NULL, workspace_bytes=0, stream=NULL)
    a.update(kw)
    st = L.ssa_sparse_attention(*a.values())
    return st, (L.ssa_last_error() or b"").decode()


@pytest.mark.parametrize("kw,status,text", [
    (dict(dtype=2), _lib.SSA_ERR_UNSUPPORTED, "dtype"),
    (dict(out_dtype=9), _lib.SSA_ERR_UNSUPPORTED, "out dtype"),
    (dict(idx_dtype=3), _lib.SSA_ERR_INVALID_ARGUMENT, "idx dtype"),
    (dict(h_kv=7), _lib.SSA_ERR_INVALID_ARGUMENT, "divisible"),
    (dict(h_q=8 * 32), _lib.SSA_ERR_UNSUPPORTED, "group size"),
    (dict(d=260), _lib.SSA_ERR_UNSUPPORTED, "head_dim"),
    (dict(d=20), _lib.SSA_ERR_UNSUPPORTED, "head_dim"),
    (dict(scale_div=0.0), _lib.SSA_ERR_INVALID_ARGUMENT, "scale"),
    (dict(v=MISALIGNED), _lib.SSA_ERR_UNSUPPORTED, "aligned"),
    (dict(o_sn=32 * 128 + 2), _lib.SSA_ERR_UNSUPPORTED, "output"),
    (dict(idx=NULL), _lib.SSA_ERR_INVALID_ARGUMENT, "null"),
])
def test_attention_rejects(L, kw, status, text):
    st, msg = _attention(L, **kw)
    assert st == status, msg
    assert text in msg


def test_attention_workspace_bytes(L):
    """The dense-prefix workspace: X per row (256-byte aligned), then the state
    of each (row, head), d + 4 floats; none where the pass does not run."""
    rows, g = 1 * 8 * 1024, 4
    need = L.ssa_sparse_attention_workspace_bytes(_lib.DTYPE_BF16, 1, 1024, 32, 8, 128, 512)
    assert need == rows * 4 + rows * g * (128 + 4) * 4
    assert L.ssa_sparse_attention_workspace_bytes(_lib.DTYPE_F32, 1, 1024, 32, 8, 128, 512) == 0
    assert L.ssa_sparse_attention_workspace_bytes(_lib.DTYPE_BF16, 1, 1024, 32, 8, 96, 512) == 0
    assert L.ssa_sparse_attention_workspace_bytes(_lib.DTYPE_BF16, 1, 1024, 32, 2, 128, 512) == 0
    assert L.ssa_sparse_attention_workspace_bytes(_lib.DTYPE_BF16, 1, 1024, 32, 8, 128, 32) == 0
    st, msg = _attention(L, workspace=FAKE, workspace_bytes=need - 1)
    assert st == _lib.SSA_ERR_WORKSPACE and "workspace" in msg


def test_index_rejects(L):
    ws = L.ssa_index_workspace_bytes(1, 1024, 8, 4, 4096)
    assert ws > 0
    st = L.ssa_build_index(FAKE, 1, 1024, 8, 4, 16385, FAKE, FAKE, FAKE, 1 << 30, NULL)
    assert st == _lib.SSA_ERR_UNSUPPORTED and b"16384" in L.ssa_last_error()
    st = L.ssa_build_index(FAKE, 1, 1024, 8, 4, 4096, FAKE, FAKE, FAKE, ws - 1, NULL)
    assert st == _lib.SSA_ERR_WORKSPACE and b"workspace" in L.ssa_last_error()
    st = L.ssa_build_index(FAKE, 1, 1024, 8, 0, 4096, FAKE, FAKE, FAKE, ws, NULL)
    assert st == _lib.SSA_ERR_INVALID_ARGUMENT
    st = L.ssa_build_index(NULL, 1, 1024, 8, 4, 4096, FAKE, FAKE, FAKE, ws, NULL)
    assert st == _lib.SSA_ERR_INVALID_ARGUMENT and b"null" in L.ssa_last_error()


def test_query_order_rejects(L):
    ws = L.ssa_query_order_workspace_bytes(1, 1024, 8, 4096)
    assert ws > L.ssa_index_workspace_bytes(1, 1024, 8, 1, 4096)  # histogram + bucket starts
    st = L.ssa_query_order(FAKE, 1, 1024, 8, 16, 16385, FAKE, FAKE, 1 << 30, NULL)
    assert st == _lib.SSA_ERR_UNSUPPORTED and b"16384" in L.ssa_last_error()
    st = L.ssa_query_order(FAKE, 1, 1024, 8, 16, 4096, FAKE, FAKE, ws - 1, NULL)
    assert st == _lib.SSA_ERR_WORKSPACE and b"workspace" in L.ssa_last_error()
    st = L.ssa_query_order(FAKE, 1, 1024, 8, 0, 4096, FAKE, FAKE, ws, NULL)
    assert st == _lib.SSA_ERR_INVALID_ARGUMENT
    st = L.ssa_query_order(FAKE, 1, 1024, 8, 16, 4096, NULL, FAKE, ws, NULL)
    assert st == _lib.SSA_ERR_INVALID_ARGUMENT and b"null" in L.ssa_last_error()
    st = L.ssa_query_order(FAKE, 1, 1 << 27, 8, 16, 4096, FAKE, FAKE, 1 << 62, NULL)
    assert st == _lib.SSA_ERR_UNSUPPORTED and b"2^31" in L.ssa_last_error()


def test_route_rejects(L):
    st = L.ssa_route_vectors(FAKE, 5, 1, 1024, 32, 4, 128, 0, 4096, 128, FAKE, 32, FAKE, NULL)
    assert st == _lib.SSA_ERR_UNSUPPORTED
    st = L.ssa_route_vectors(FAKE, _lib.DTYPE_F32, 1, 1024, 30, 4, 128, 0, 4096, 128, FAKE, 32,
                             FAKE, NULL)
    assert st == _lib.SSA_ERR_INVALID_ARGUMENT
    ws = L.ssa_code_topk_workspace_bytes(1, 8, 1024, 4096)
    # top > num_codebook, top > 64, temperature <= 0, workspace too small
    assert L.ssa_code_topk(FAKE, 1, 8, 1024, FAKE, 16, 32, 1.0, 17, FAKE, FAKE, ws, NULL) == \
        _lib.SSA_ERR_INVALID_ARGUMENT
    assert L.ssa_code_topk(FAKE, 1, 8, 1024, FAKE, 4096, 32, 1.0, 65, FAKE, FAKE, ws, NULL) == \
        _lib.SSA_ERR_UNSUPPORTED
    assert L.ssa_code_topk(FAKE, 1, 8, 1024, FAKE, 4096, 32, 0.0, 4, FAKE, FAKE, ws, NULL) == \
        _lib.SSA_ERR_INVALID_ARGUMENT
    assert L.ssa_code_topk(FAKE, 1, 8, 1024, FAKE, 4096, 32, 1.0, 4, FAKE, FAKE, ws - 1, NULL) == \
        _lib.SSA_ERR_WORKSPACE
    rws = L.ssa_route_workspace_bytes(1, 1024, 8, 4096, 32)
    st = L.ssa_route_codes(FAKE, FAKE, _lib.DTYPE_BF16, 1, 1024, 32, 8, 128, 0, 4096, 128, 0, 1024,
                           128, FAKE, FAKE, FAKE, 32, 4096, 16, 4, 1.0, FAKE, FAKE, FAKE, rws - 1,
                           NULL)
    assert st == _lib.SSA_ERR_WORKSPACE
    assert L.ssa_normalize_rows(NULL, 4, 32, FAKE, NULL) == _lib.SSA_ERR_INVALID_ARGUMENT


def test_workspace_sizes_grow(L):
    f = L.ssa_route_workspace_bytes
    assert f(1, 2048, 8, 4096, 32) > f(1, 1024, 8, 4096, 32) > 0
    assert f(2, 1024, 8, 4096, 32) > f(1, 1024, 8, 4096, 32)
    g = L.ssa_index_workspace_bytes
    assert g(1, 65536, 8, 4, 4096) >= g(1, 1024, 8, 4, 4096) > 0
    for ws in (f(1, 1024, 8, 4096, 32), g(1, 1024, 8, 4, 4096),
               L.ssa_code_topk_workspace_bytes(1, 8, 1024, 4096)):
        assert ws % 256 == 0, "workspace sub-buffers are 256-byte aligned"


def test_block_entry_points_reject_rows_past_the_keys(L):
    """ssa_select_block / ssa_sparse_attention_block: query rows
    [q_pos0, q_pos0 + n_q) must lie inside the n keys (checked before any launch)."""
    null = ctypes.c_void_p(0)
    st = L.ssa_sparse_attention_block(null, null, null, 0, 1, 32, 4, 30, 4, 2, 64, 0, 256, 64, 0, 128,
                                      64, 0, 128, 64, null, 0, 8, 0, 16, 8, 8.0, 1, null, null, null,
                                      0, 0, 256, 64, null, null, null, 0, null)
    assert st == _lib.SSA_ERR_INVALID_ARGUMENT
    assert b"outside" in L.ssa_last_error()
    st = L.ssa_select_block(null, null, 0, 1, 32, 4, -1, 4, 2, 64, 0, 256, 64, 0, 128, 64, null, 8,
                            null, null, 16, 4, 8, 1, null, 0, 0, 8.0, 0, null, null, 0, null, null, null,
                            0, null)
    assert st == _lib.SSA_ERR_INVALID_ARGUMENT


@pytest.mark.parametrize("batch,n,h_kv,top_k", [
    (1, 32768, 8, 512), (1, 131072, 2, 1024), (2, 300, 2, 32), (4, 8192, 8, 512), (1, 1, 1, 1),
    (3, 1000, 3, 4096), (1, 64 * 5 + 1, 1, 7), (2, 70000, 2, 512),
])
def test_select_workspace_regions_do_not_overlap(L, batch, n, h_kv, top_k):
    """The select workspace's regions (carve_sel_ws) are disjoint, in order, as
    large as the kernels index them, and inside the workspace: the counter
    block holds 16 + 4 ints per shard, the exact list one int per row, the
    screened-row entries 3 ints and the error bounds one float per shard slot,
    the candidate counts one int per row, the candidate lists and scores cap
    entries per shard.  Swept over shapes and
    workspace sizes from the minimum to past the recommended size (a too-small
    counter block once let a garbage counter drive an out-of-bounds write)."""
    rows = batch * n * h_kv
    lo = L.ssa_select_workspace_bytes(batch, n, h_kv, 0)
    hi = L.ssa_select_workspace_bytes(batch, n, h_kv, top_k)
    assert hi >= lo > 0
    for bytes_ in sorted({lo, lo + 255, (lo + hi) // 2, hi, 2 * hi + 77}):
        for screen in (0, 1):
            lay = (ctypes.c_int64 * 11)()
            assert L.ssa_select_workspace_layout(batch, n, h_kv, bytes_, screen, lay) == _lib.SSA_OK
            ctr, exact, scr, emax, cand, approx, shard_rows, cap, shards, ctr_bytes, cnt = list(lay)
            assert shard_rows * shards >= rows
            assert 4 * (16 + 4 * shards) <= ctr_bytes
            ends = [(ctr, ctr + ctr_bytes), (exact, exact + 4 * rows),
                    (scr, scr + 12 * shards * shard_rows), (emax, emax + 4 * shards * shard_rows),
                    (cnt, cnt + 4 * rows), (cand, cand + 4 * shards * cap),
                    (approx, approx + 4 * shards * cap)]
            assert ctr == 0
            for (s0, e0), (s1, _) in zip(ends, ends[1:]):
                assert s0 <= e0 <= s1, (ends, bytes_)
            assert ends[-1][1] <= bytes_
            assert all(o % 256 == 0 for o in (exact, scr, emax, cnt, cand, approx))
            assert cap % 32 == 0 and cap >= 0
            if not screen or bytes_ == lo:
                assert cap == 0
    assert L.ssa_select_workspace_layout(batch, n, h_kv, lo - 1, 1, (ctypes.c_int64 * 11)()) \
        == _lib.SSA_ERR_WORKSPACE


def _decode(L, **kw):
    a = dict(q=FAKE, k=FAKE, v=FAKE, dtype=_lib.DTYPE_BF16, batch=1, m=1, h_q=32, h_kv=8, d=128,
             q_sb=4096, q_sn=4096, q_sh=128, k_sb=1024, k_sn=1024, k_sh=128, v_sb=1024, v_sn=1024,
             v_sh=128, k_cache=FAKE, v_cache=FAKE, max_len=1024, kc_sb=1024 * 1024, kc_sn=1024,
             kc_sh=128, vc_sb=1024 * 1024, vc_sn=1024, vc_sh=128, n0=100, w_qr=FAKE, w_kr=FAKE,
             prep=FAKE, d_s=32, n_c=4096, a=16, b=4, temperature=1.0, k_codes=FAKE, offsets=FAKE,
             postings=FAKE, n_base=90, tail_offsets=FAKE, tail_postings=FAKE, tail_cap=2048,
             top_k=512, score_div=11.3137, scale_div=11.3137, causal=1, indices=NULL, out=FAKE,
             out_dtype=_lib.DTYPE_BF16, o_sb=4096, o_sn=4096, o_sh=128, workspace=FAKE,
             workspace_bytes=1 << 30, stream=NULL)
    a.update(kw)
    st = L.ssa_decode_step(*a.values())
    return st, (L.ssa_last_error() or b"").decode()


@pytest.mark.parametrize("kw,status,text", [
    (dict(dtype=5), _lib.SSA_ERR_UNSUPPORTED, "dtype"),
    (dict(n0=1024), _lib.SSA_ERR_INVALID_ARGUMENT, "exceed"),
    (dict(n_base=101), _lib.SSA_ERR_INVALID_ARGUMENT, "main index"),
    (dict(n_base=0, tail_cap=100), _lib.SSA_ERR_WORKSPACE, "tail"),
    (dict(workspace_bytes=16), _lib.SSA_ERR_WORKSPACE, "workspace"),
    (dict(n_c=20000), _lib.SSA_ERR_UNSUPPORTED, "16384"),
    (dict(k_sn=1028), _lib.SSA_ERR_UNSUPPORTED, "aligned"),
    (dict(h_q=30), _lib.SSA_ERR_INVALID_ARGUMENT, "shape"),
])
def test_decode_step_rejects(L, kw, status, text):
    st, msg = _decode(L, **kw)
    assert st == status, msg
    assert text in msg


def test_decode_empty_step_is_noop(L):
    assert _decode(L, m=0, q=NULL, k=NULL, v=NULL)[0] == _lib.SSA_OK
