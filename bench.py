"""SSA forward benchmark on one MI355X.

One step = one full SSA forward over resident inputs: routing vectors and
codebook top-codes (stage a), inverted index (b), candidate selection (c) and
gathered-KV attention (d), exactly as CodebookRouter + sparse_exact_attention
run them.  Workload (default): BASELINE config 3 -- 1 x 32768 tokens, bf16,
GQA 32/8, d 128, d_s 32, N_c 4096, a 16, b 4, k 512, causal, RoPE theta 1e6 on
a seeded 64-cluster Gaussian mixture (sigma 0.3), V ~ N(0, 1).  --config c5 is
the 128K-token layer; --config c4 times the whole decoder attention block
(RMSNorm + SSAAttention with its projections) at B 4, n 8192, d_model 4096.

Prints ONE JSON line (rank 0) with the metric, per-stage times, the roofline
of the dominant kernel (stage d: compulsory HBM bytes per launch over its
HIP-event time on the launch stream, next to the counter-measured traffic and
the scope table's logical gather rate) and two bounded CPU baselines: the
reference's dense algorithm restated in torch, and the linear C oracle.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "SSA fwd tokens/s at n=32K,k=512 bf16; % HBM/MFMA roofline per stage"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0

CONFIGS = {
    "c3": dict(B=1, n=32768, h_q=32, h_kv=8, d=128, d_s=32, n_c=4096, b=4, a=16, k=512,
               clusters=64, sigma=0.3, theta=1e6, dtype="bf16"),
    "c4": dict(B=4, n=8192, h_q=32, h_kv=8, d=128, d_s=32, n_c=4096, b=4, a=16, k=512,
               d_model=4096, theta=1e6, dtype="bf16"),
    "c5": dict(B=1, n=131072, h_q=16, h_kv=2, d=128, d_s=32, n_c=8192, b=4, a=32, k=1024,
               clusters=256, sigma=0.3, theta=1e6, dtype="bf16"),
}


def parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--config", default="c3", choices=sorted(CONFIGS))
    p.add_argument("--n", type=int, default=None, help="override sequence length")
    p.add_argument("--num-codebook", type=int, default=None, help="override the codebook size N_c")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline budget")
    p.add_argument("--copy-probe-gib", type=float, default=0.0,
                   help="also run one device copy of this size (PMC byte calibration)")
    p.add_argument("--backward", action="store_true",
                   help="also time the stage-(d) backward (dq, dk, dv) on the workload's indices")
    p.add_argument("--decode", type=int, default=0,
                   help="also time this many single-token decode steps after a prefill of n minus "
                        "that many tokens (SSADecodeCache)")
    p.add_argument("--decode-lens", default="",
                   help="with --decode: also time the steps at these cache lengths (c3 head "
                        "shapes; codebook fixed at the config's N_c and scaled with n)")
    p.add_argument("--block-sparse", type=int, default=0,
                   help="also time the block-granular variant with this many 64-key blocks per "
                        "query block (block indices from the workload's selections, then attention)")
    p.add_argument("--sweep", default=None,
                   help="comma list of n for a tokens/s vs n sweep at the config's head shapes "
                        "(default for c3: 4K..128K, both codebook policies); '' for none")
    p.add_argument("--sweep-nc", default="both", choices=("scaled", "fixed", "both"),
                   help="codebook size in the sweep: scaled with n (constant bucket size; the "
                        "config's N_c at its own n), fixed at the config's N_c, or both")
    p.add_argument("--no-extras", action="store_true",
                   help="skip the default n-sweep and the c5 stage times (profiling runs)")
    return p.parse_args()


def make_workload(cfg, seed, device):
    """Seeded synthetic inputs of the config's shape, resident on `device`."""
    import torch

    from ssa_amd import CodebookRouter
    from ssa_amd.utils import apply_rope, precompute_rope_freqs

    B, n, h_q, h_kv, d = cfg["B"], cfg["n"], cfg["h_q"], cfg["h_kv"], cfg["d"]
    g = h_q // h_kv
    gen = torch.Generator(device=device).manual_seed(seed)
    centres = torch.randn(B, h_kv, cfg["clusters"], d, generator=gen, device=device)
    z = torch.randint(0, cfg["clusters"], (B, n, h_kv), generator=gen, device=device)
    bi = torch.arange(B, device=device)[:, None, None]
    hi = torch.arange(h_kv, device=device)[None, None, :]
    kc = centres[bi, hi, z]                                      # [B, n, h_kv, d]
    k = kc + cfg["sigma"] * torch.randn(B, n, h_kv, d, generator=gen, device=device)
    q = kc.repeat_interleave(g, dim=2) + cfg["sigma"] * torch.randn(B, n, h_q, d, generator=gen,
                                                                    device=device)
    v = torch.randn(B, n, h_kv, d, generator=gen, device=device)
    # Positional RoPE: ssa/utils.py math on a [.., heads, n, d] layout (angle by position).
    freqs = precompute_rope_freqs(d, n, cfg["theta"], device=device)
    q = apply_rope(q.transpose(1, 2), freqs).transpose(1, 2)
    k = apply_rope(k.transpose(1, 2), freqs).transpose(1, 2)
    dt = torch.bfloat16 if cfg["dtype"] == "bf16" else torch.float32
    q, k, v = q.to(dt).contiguous(), k.to(dt).contiguous(), v.to(dt).contiguous()
    torch.manual_seed(seed + 1)
    router = CodebookRouter(head_dim=d, route_dim=cfg["d_s"], num_kv_heads=h_kv,
                            num_codebook=cfg["n_c"], codes_per_key=cfg["b"],
                            codes_per_query=cfg["a"], top_k=cfg["k"]).to(device)
    return q, k, v, router


def make_block(cfg, seed, device):
    """Config 4: RMSNorm, then one full SSAAttention forward (q/k/v projections,
    RoPE as the reference layer applies it (ssa/ssa_layer.py:115-117), routing,
    attention, o_proj) with the default random init from a fixed seed; hidden
    states x ~ N(0, 1) of shape [B, n, d_model], bf16."""
    import torch

    from ssa_amd import SSAAttention
    from ssa_amd.utils import precompute_rope_freqs

    torch.manual_seed(seed + 1)
    layer = SSAAttention(hidden_size=cfg["d_model"], num_q_heads=cfg["h_q"],
                         num_kv_heads=cfg["h_kv"], head_dim=cfg["d"], route_dim=cfg["d_s"],
                         num_codebook=cfg["n_c"], codes_per_key=cfg["b"],
                         codes_per_query=cfg["a"], top_k=cfg["k"])
    norm = torch.nn.RMSNorm(cfg["d_model"], eps=1e-6)
    layer = layer.to(device, torch.bfloat16).eval()
    norm = norm.to(device, torch.bfloat16)
    gen = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(cfg["B"], cfg["n"], cfg["d_model"], generator=gen, device=device).to(torch.bfloat16)
    freqs = precompute_rope_freqs(cfg["d"], cfg["n"], cfg["theta"], device=device)
    return {"layer": layer, "norm": norm, "x": x, "freqs": freqs}


def block_step(blk):
    """One c4 step: exactly the module calls a user makes."""
    return blk["layer"](blk["norm"](blk["x"]), freqs=blk["freqs"])


def block_stages(blk, reps=5):
    """Per-phase times of the c4 forward: the same calls SSAAttention.forward
    makes, with HIP events between them (median of `reps`)."""
    import torch

    from ssa_amd import kernels

    layer, r = blk["layer"], blk["layer"].router
    names = ["norm", "projections+rope", "a", "b", "c", "d", "o_proj"]
    ts = {k_: [] for k_ in names}
    with torch.no_grad():
        for _ in range(reps):
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)]
            ev[0].record()
            h = blk["norm"](blk["x"])
            ev[1].record()
            q, k, v = layer.project(h, None, blk["freqs"])
            ev[2].record()
            qc, kc = kernels.route_codes(q, k, r.W_qr.weight, r.W_kr.weight, r.codebook,
                                         r.codes_per_query, r.codes_per_key, r.temperature)
            ev[3].record()
            off, post = kernels.build_index(kc, r.num_codebook)
            order = kernels.query_order(qc, r.num_codebook)
            ev[4].record()
            pfx = torch.empty(order.shape, device=q.device, dtype=torch.int32)
            idx = kernels.select(q, k, qc, off, post, r.codes_per_key, r.top_k, sorted=False,
                                 index_dtype=torch.int32, row_order=order, row_prefix=pfx)
            ev[5].record()
            out = kernels.sparse_attention(q, k, v, idx, None, layer.causal_attention,
                                           row_order=order, row_prefix=pfx)
            ev[6].record()
            layer.o_proj(out.reshape(h.shape[0], h.shape[1], -1))
            ev[7].record()
            torch.cuda.synchronize()
            for i, k_ in enumerate(names):
                ts[k_].append(ev[i].elapsed_time(ev[i + 1]))
    return {k_: sorted(v_)[len(v_) // 2] for k_, v_ in ts.items()}


def algorithmic(cfg, n, stats_sum=None, distinct_kv=None):
    """Algorithmic bytes / flops per stage for one forward (B*n*h_kv rows).

    stats_sum = (R postings read, C all candidates, C_r candidates of the rows
    that are rescored, heavy rows) from the select kernels' counters;
    distinct_kv = number of distinct (batch, kv head, key) rows stage (d) reads."""
    B, h_q, h_kv, d = cfg["B"], cfg["h_q"], cfg["h_kv"], cfg["d"]
    s = 2 if cfg["dtype"] == "bf16" else 4
    g = h_q // h_kv
    rows = B * n * h_kv
    a, b, k, n_c, d_s = cfg["a"], cfg["b"], cfg["k"], cfg["n_c"], cfg["d_s"]
    out = {}
    out["a_flops"] = 2 * B * n * (h_q + h_kv) * d * d_s + 4 * rows * n_c * d_s
    out["a_flops_projection"] = 2 * B * n * (h_q + h_kv) * d * d_s
    out["a_bytes"] = B * n * (h_q + h_kv) * d * s + h_kv * n_c * d_s * 4 + rows * (a + b) * 4
    out["b_bytes"] = 3 * rows * b * 4 + h_kv * B * (n_c + 1) * 4
    if stats_sum is not None:
        R, C, C_r, heavy = stats_sum
        # the scope table's formula: every candidate's K row, each row's q group
        out["c_bytes_survey"] = R * 4 + C * d * s + rows * (g * d * s + 3 * a * 4 + k * 4)
        # what the index-order kernels read: postings, the K rows of the rescored
        # rows' candidates and their q groups, q_codes and bucket bounds, the output
        out["c_bytes"] = R * 4 + C_r * d * s + heavy * g * d * s + rows * (3 * a * 4 + k * 4)
        out["c_flops"] = C_r * 2 * d * g
    # the scope table's logical gather: each selected K/V row once per (query, kv head)
    out["d_bytes_logical"] = rows * (k * 4 + 2 * k * d * s + 2 * g * d * s)
    out["d_flops"] = 4 * rows * g * k * d
    if distinct_kv is not None:
        # compulsory: q and the output once, the int32 indices once, every distinct
        # K/V row once -- what a kernel with a perfect cache moves to and from HBM
        out["d_bytes_compulsory"] = (2 * B * n * h_q * d * s + rows * k * 4
                                     + distinct_kv * 2 * d * s)
    return out


def run_step(q, k, v, router, events=None):
    import torch

    from ssa_amd import kernels

    if events:
        events[0].record()
    qc, kc = kernels.route_codes(q, k, router.W_qr.weight, router.W_kr.weight, router.codebook,
                                 router.codes_per_query, router.codes_per_key, router.temperature)
    if events:
        events[1].record()
    off, post = kernels.build_index(kc, router.num_codebook)
    order = kernels.query_order(qc, router.num_codebook)
    if events:
        events[2].record()
    # Same calls as SSAAttention: stage (d) does not depend on the order of the
    # selected keys, so the router lists them by index (same set as sorted),
    # the indices pass to stage (d) as int32, and stages (c) and (d) process the
    # rows of each head grouped by best code (results do not depend on the order);
    # the selection also names each row's key prefix [0, X) (its lowest-key
    # filler), which stage (d) attends in blocks of neighbouring rows.
    pfx = torch.empty(order.shape, device=q.device, dtype=torch.int32)
    idx = kernels.select(q, k, qc, off, post, router.codes_per_key, router.top_k, sorted=False,
                         index_dtype=torch.int32, row_order=order, row_prefix=pfx)
    if events:
        events[3].record()
    out = kernels.sparse_attention(q, k, v, idx, None, True, row_order=order, row_prefix=pfx)
    if events:
        events[4].record()
    return out


def time_gpu(cfg, q, k, v, router, steps, warmup):
    import torch

    for _ in range(warmup):
        run_step(q, k, v, router)
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(steps):
        run_step(q, k, v, router, evs[s])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    stage = {"a": [], "b": [], "c": [], "d": []}
    for e in evs:
        for i, key in enumerate("abcd"):
            stage[key].append(e[i].elapsed_time(e[i + 1]))
    return wall, {key: sum(v_) / len(v_) for key, v_ in stage.items()}


def time_code_scoring(cfg, q, k, router, reps=5):
    """Stage (a)'s codebook scoring alone (the matrix-core screen and its exact
    rescoring, ssa/router.py:121-141) on the forward's routing vectors: the query
    side (top a) and the key side (top b) as two ssa_code_topk calls, each with
    its codebook preparation; the forward runs both screens as one launch."""
    import torch

    from ssa_amd import kernels

    g = cfg["h_q"] // cfg["h_kv"]
    qhat = kernels.route_vectors(q, router.W_qr.weight, g)
    khat = kernels.route_vectors(k, router.W_kr.weight, 1)
    chat = kernels.normalize_rows(router.codebook.float())
    kernels.code_topk(qhat, chat, cfg["a"], router.temperature)
    kernels.code_topk(khat, chat, cfg["b"], router.temperature)
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        kernels.code_topk(qhat, chat, cfg["a"], router.temperature)
        kernels.code_topk(khat, chat, cfg["b"], router.temperature)
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1))
    return sorted(ts)[len(ts) // 2]


def time_sorted_select(q, k, router, reps=5):
    """Stage (c) in reference order (keys by score, as torch.topk returns them)."""
    import torch

    from ssa_amd import kernels

    qc, kc = kernels.route_codes(q, k, router.W_qr.weight, router.W_kr.weight, router.codebook,
                                 router.codes_per_query, router.codes_per_key, router.temperature)
    off, post = kernels.build_index(kc, router.num_codebook)
    kernels.select(q, k, qc, off, post, router.codes_per_key, router.top_k, sorted=True)
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        kernels.select(q, k, qc, off, post, router.codes_per_key, router.top_k, sorted=True)
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1))
    return sorted(ts)[len(ts) // 2]


def time_spread_attention(q, k, v, idx_like, reps=5):
    """Stage (d) on an index set with no filler: every (batch, row, kv head)
    attends k distinct keys spread over the whole sequence (a seeded random
    start and odd stride modulo n, distinct because n is a power of two),
    unmasked, so no slot is a filler key that neighbouring rows share.  int32
    indices, as in the forward's call.  Median ms of `reps` calls (HIP events on
    the launch stream); None when n is not a power of two."""
    import torch

    from ssa_amd import kernels

    B, n, h_kv, kk = idx_like.shape
    if n & (n - 1) or kk > n:
        return None
    gen = torch.Generator(device=idx_like.device).manual_seed(7)
    shape = (B, n, h_kv, 1)
    start = torch.randint(0, n, shape, device=idx_like.device, generator=gen, dtype=torch.int64)
    stride = torch.randint(0, max(n // 2, 1), shape, device=idx_like.device, generator=gen,
                           dtype=torch.int64) * 2 + 1
    j = torch.arange(kk, device=idx_like.device, dtype=torch.int64)
    idx = ((start + j * stride) % n).to(torch.int32)
    del start, stride
    out = kernels.sparse_attention(q, k, v, idx, None, False)
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        kernels.sparse_attention(q, k, v, idx, None, False, out=out)
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1))
    return sorted(ts)[len(ts) // 2]


def stats_sums(q, k, router):
    import torch

    from ssa_amd import kernels

    qc, kc = kernels.route_codes(q, k, router.W_qr.weight, router.W_kr.weight, router.codebook,
                                 router.codes_per_query, router.codes_per_key, router.temperature)
    off, post = kernels.build_index(kc, router.num_codebook)
    pfx = torch.empty(qc.shape[:3], device=q.device, dtype=torch.int32)
    idx, st = kernels.select(q, k, qc, off, post, router.codes_per_key, router.top_k,
                             with_stats=True, sorted=False, row_prefix=pfx)
    prefix_slots = int(pfx.to(torch.int64).sum())
    st = st.to(torch.int64)
    C = int(st[..., 0].sum())
    R = int(st[..., 1].sum())
    heavy = st[..., 0] > router.top_k      # index order rescores only these rows
    C_r = int(st[..., 0][heavy].sum())
    # distinct (batch, kv head, key) rows that stage (d) reads
    B, n, h_kv, _ = idx.shape
    base = (torch.arange(B, device=idx.device)[:, None, None, None] * h_kv
            + torch.arange(h_kv, device=idx.device)[None, None, :, None]) * n
    seen = torch.zeros(B * h_kv * n, dtype=torch.bool, device=idx.device)
    seen[(idx + base).reshape(-1)] = True
    distinct = int(seen.sum())
    return (R, C, int(heavy.sum()), C_r, st[..., 0].numel(), distinct, (qc, kc, off, post, idx),
            prefix_slots)


def time_backward(cfg, q, k, v, inter, reps=3):
    """Stage (d) backward on the forward's indices and query order, with an fp32
    forward output and a seeded bf16 output gradient, as SSAAttention trains:
    ssa_sparse_attention_backward_routed (candidate and prefix keys by codebook
    bucket / prefix tile) with the forward's row stats, and, for comparison,
    the plain ssa_sparse_attention_backward without either; median of `reps`
    launches each (HIP events on the launch stream)."""
    import torch

    from ssa_amd import kernels

    qc, kc, off, post, _ = inter
    order = kernels.query_order(qc, cfg["n_c"])
    pfx = torch.empty(order.shape, device=q.device, dtype=torch.int32)
    idx = kernels.select(q, k, qc, off, post, cfg["b"], cfg["k"], sorted=False,
                         index_dtype=torch.int32, row_order=order, row_prefix=pfx)
    out32 = torch.empty(q.shape, device=q.device, dtype=torch.float32)
    stats = kernels.row_stats_buffer(q, cfg["h_kv"])  # the forward's softmax stats, as in training
    kernels.sparse_attention(q, k, v, idx, None, True, out=out32, row_order=order, row_prefix=pfx,
                             row_stats=stats)
    gen = torch.Generator(device=q.device).manual_seed(7)
    dout = torch.randn(q.shape, generator=gen, device=q.device).to(q.dtype)
    routing = kernels.Routing(qc, kc, off, post, True)

    def median_ms(rt, st):
        ts = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            kernels.sparse_attention_backward(q, k, v, idx, out32, dout, None, True, row_order=order,
                                              row_prefix=pfx, routing=rt, row_stats=st)
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1))
        return sorted(ts)[len(ts) // 2]

    ms = median_ms(routing, stats)
    ms_plain = median_ms(None, None)
    B, n, h_q, h_kv, d, kk = cfg["B"], cfg["n"], cfg["h_q"], cfg["h_kv"], cfg["d"], cfg["k"]
    s = 2 if cfg["dtype"] == "bf16" else 4
    rows = B * n * h_kv
    g = h_q // h_kv
    # per row: K and V of each slot once, its indices, q / dO (input type) and
    # o (fp32) read, dq written; dk and dv written once per key
    byt = rows * (2 * kk * d * s + kk * 4 + g * d * (2 * s + 4) + g * d * 4) + B * n * h_kv * d * 8
    return {"ms": ms, "tokens_per_s": B * n / (ms / 1000),
            "kernel": "sparse_attention_bwd_mfma_kernel + prefix_attention_bwd_kernel + bucket_attention_bwd_kernel",
            "ms_plain_without_buckets_or_stats": ms_plain,
            "algorithmic_gb": byt / 1e9, "gbs": byt / (ms / 1000) / 1e9}


def time_blocks(cfg, q, k, v, inter, n_k_blocks, block_size=64, reps=3):
    """Block-granular variant: ssa_block_indices on the workload's token
    selections, then ssa_block_sparse_attention; median of `reps` (HIP events)."""
    import torch

    from ssa_amd import kernels

    qc, kc, off, post, _ = inter
    idx = kernels.select(q, k, qc, off, post, cfg["b"], cfg["k"], sorted=False, index_dtype=torch.int32)
    ts = {"indices": [], "attention": []}
    for _ in range(reps):
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record()
        blocks = kernels.block_indices(idx, block_size, n_k_blocks)
        e[1].record()
        kernels.block_sparse_attention(q, k, v, blocks, block_size)
        e[2].record()
        torch.cuda.synchronize()
        ts["indices"].append(e[0].elapsed_time(e[1]))
        ts["attention"].append(e[1].elapsed_time(e[2]))
    med = {key: sorted(v)[len(v) // 2] for key, v in ts.items()}
    return {"block_size": block_size, "n_k_blocks": n_k_blocks, "ms_indices": med["indices"],
            "ms_attention": med["attention"],
            "tokens_per_s": cfg["B"] * cfg["n"] / ((med["indices"] + med["attention"]) / 1000.0)}


def time_decode(cfg, q, k, v, router, steps, tail_tokens=512):
    """Single-token decode steps (ssa_amd.decode.SSADecodeCache: one native call
    per step, a tail index over the newest keys, the main index rebuilt every
    tail_tokens keys) for the last `steps` tokens of the workload after a
    prefill of the rest; host wall time per step, including the rebuilds that
    fall inside the timed steps, and HIP-event time of the steps."""
    import torch

    from ssa_amd.decode import SSADecodeCache

    n = cfg["n"]
    cache = SSADecodeCache(router, cfg["B"], n, cfg["d"], dtype=q.dtype, tail_tokens=tail_tokens)
    n0 = n - steps
    cache.step(q[:, :n0], k[:, :n0], v[:, :n0])
    torch.cuda.synchronize()
    rebuilds0 = cache.rebuilds
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for t in range(n0, n):
        cache.step(q[:, t:t + 1], k[:, t:t + 1], v[:, t:t + 1])
    e1.record()
    torch.cuda.synchronize()
    ms = 1000 * (time.perf_counter() - t0) / steps
    return {"ms_per_token": ms, "gpu_ms_per_token": e0.elapsed_time(e1) / steps,
            "tokens_per_s": cfg["B"] / (ms / 1000), "cache_len": n, "steps": steps,
            "prefill_tokens": n0, "tail_tokens": tail_tokens,
            "rebuilds_in_timed_steps": cache.rebuilds - rebuilds0}


DEFAULT_SWEEP = (4096, 8192, 16384, 32768, 65536, 131072)


def run_sweep(cfg, ns, policy, seed, dev, steps):
    """tokens/s of the full forward at each n (the config's head shapes), the
    codebook scaled with n (N_c = cfg N_c * n / cfg n, constant expected bucket
    size) or fixed; least-squares t = alpha * n + beta and its R^2 (the
    reference's linearity check, benchmark/profile_scaling.py:39-54)."""
    points = {}
    for n_ in ns:
        c2 = dict(cfg, n=n_)
        if policy == "scaled":
            c2["n_c"] = max(16, cfg["n_c"] * n_ // cfg["n"])
        q2, k2, v2, r2 = make_workload(c2, seed, dev)
        w2, s2 = time_gpu(c2, q2, k2, v2, r2, steps, 2)
        ms2 = 1000 * w2 / steps
        points[n_] = {"ms": ms2, "tokens_per_s": c2["B"] * n_ / (ms2 / 1000), "num_codebook": c2["n_c"],
                      "stages_ms": s2}
        print(f"sweep ({policy} N_c) n={n_}: {ms2:.3f} ms", file=sys.stderr, flush=True)
        del q2, k2, v2, r2
    out = {"num_codebook_policy": (f"scaled: N_c = {cfg['n_c']} * n / {cfg['n']}" if policy == "scaled"
                                   else f"fixed: N_c = {cfg['n_c']}"),
           "points": points}
    xs = sorted(points)
    ts = [points[x]["ms"] for x in xs]
    if len(xs) >= 3:
        mn, mt = sum(xs) / len(xs), sum(ts) / len(ts)
        sxx = sum((x - mn) ** 2 for x in xs)
        alpha = sum((x - mn) * (t_ - mt) for x, t_ in zip(xs, ts)) / sxx
        beta = mt - alpha * mn
        ss_res = sum((t_ - (alpha * x + beta)) ** 2 for x, t_ in zip(xs, ts))
        ss_tot = sum((t_ - mt) ** 2 for t_ in ts)
        out["fit"] = {"ms_per_token": alpha, "ms_offset": beta,
                      "r2": 1.0 - ss_res / ss_tot if ss_tot > 0 else 1.0}
    return out


def run_c5(seed, dev, steps, warmup):
    """Config 5 (n = 131072, GQA 16/2, N_c 8192, a 32, k 1024): whole-forward
    ms and tokens/s and per-stage ms (HIP events on the launch stream)."""
    cfg = dict(CONFIGS["c5"])
    q, k, v, router = make_workload(cfg, seed, dev)
    wall, st = time_gpu(cfg, q, k, v, router, steps, warmup)
    ms = 1000 * wall / steps
    print(f"c5: {ms:.3f} ms", file=sys.stderr, flush=True)
    return {"workload": "c5: SSA forward (stages a-d), causal, n=131072, GQA 16/2, N_c 8192, a 32, k 1024",
            "ms": ms, "tokens_per_s": cfg["B"] * cfg["n"] / (ms / 1000), "stages_ms": st, "steps": steps}


def run_c4(seed, dev, steps, warmup):
    """Config 4 (the decoder block: RMSNorm, projections, RoPE, SSA, o_proj;
    B 4, n 8192, d_model 4096): whole-block ms and tokens/s and per-phase ms."""
    import torch

    cfg = dict(CONFIGS["c4"])
    blk = make_block(cfg, seed, dev)
    with torch.no_grad():
        for _ in range(warmup):
            block_step(blk)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            block_step(blk)
        torch.cuda.synchronize()
        ms = 1000 * (time.perf_counter() - t0) / steps
        phases = block_stages(blk)
    print(f"c4: {ms:.3f} ms", file=sys.stderr, flush=True)
    del blk
    return {"workload": "c4: RMSNorm + SSAAttention forward (projections, RoPE, stages a-d, o_proj), "
                        "B 4, n 8192, d_model 4096, causal routing",
            "ms": ms, "tokens_per_s": cfg["B"] * cfg["n"] / (ms / 1000), "phases_ms": phases, "steps": steps}


def _cpu_model():
    cpu = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return cpu


def cpu_share():
    """Threads for the CPU baselines: the job's share of the host (16 per GPU on
    the GPU boxes, which set OMP_NUM_THREADS to it), at most the CPUs present."""
    share = int(os.environ.get("OMP_NUM_THREADS", "16") or 16)
    return max(1, min(share, os.cpu_count() or 1))


def cpu_reference(cfg, q, k, v, router, budget_s, blk=None):
    """The reference's own dense algorithm (oracle/dense_ref.py: torch on the host
    cores) on batch element 0.  Its memory grows as rows * n (about 280 GB with
    every row at n = 32768), so routing runs in full, selection and attention on
    sampled query rows against all n keys (each sampled row does the full
    per-row work: all keys scored, masked and ranked), scaled to n rows and to
    the batch.  With a block (config 4) the q/k/v/o projections of sampled
    tokens are timed too (fp32 GEMMs) and scaled."""
    import torch

    from oracle import dense_ref

    threads = cpu_share()
    torch.set_num_threads(threads)
    n, B = cfg["n"], cfg["B"]
    qf, kf, vf = q[0].float().cpu(), k[0].float().cpu(), v[0].float().cpu()
    w_qr, w_kr = router.W_qr.weight.float().cpu(), router.W_kr.weight.float().cpu()
    cb = router.codebook.float().cpu()
    with torch.no_grad():
        t0 = time.perf_counter()
        qc, ka = dense_ref.route_codes(qf, kf, w_qr, w_kr, cb, cfg["a"], cfg["b"])
        t_a = time.perf_counter() - t0
        sc = 4
        while True:
            rows = torch.linspace(0, n - 1, sc).long()
            t0 = time.perf_counter()
            idx = dense_ref.select(qf, kf, qc, ka, cfg["k"], rows, causal=True)
            t_c1 = time.perf_counter() - t0
            t0 = time.perf_counter()
            dense_ref.sparse_attention(qf, kf, vf, idx, rows)
            t_d1 = time.perf_counter() - t0
            if t_a + t_c1 + t_d1 > budget_s / 2 or sc >= min(n, 256):
                break
            sc = min(n, sc * 2)
        t_proj = 0.0
        if blk is not None:
            layer = blk["layer"]
            tok = min(512, n)
            xs = blk["x"][0, :tok].float().cpu()
            ws = [getattr(layer, m).weight.float().cpu() for m in ("q_proj", "k_proj", "v_proj", "o_proj")]
            t0 = time.perf_counter()
            for w in ws:            # every projection's input width is d_model = h_q * d here
                xs @ w.T
            t_proj = (time.perf_counter() - t0) * n / tok
    t_c, t_d = t_c1 * n / sc, t_d1 * n / sc
    total = t_a + t_c + t_d + t_proj                  # one batch element
    return {
        "value": n / total,
        "unit": "tokens/s",
        "cores": threads,
        "host_cpus": os.cpu_count(),
        "kind": "port",
        "sample": (f"the reference's dense algorithm (ssa/router.py:102-259, ssa/attention.py:64-113) "
                   f"restated in torch on the CPU (oracle/dense_ref.py; {threads} threads, the job's "
                   f"share of {os.cpu_count()} host CPUs, {_cpu_model()}): routing of all {n} tokens in full, dense rescoring + candidate "
                   f"mask + top-k + attention for {sc} sampled query rows against all {n} keys, scaled "
                   f"to {n} rows" + (f" and {B} batch elements" if B > 1 else "")
                   + ("; q/k/v/o projections timed on 512 tokens, scaled" if blk is not None else "")
                   + f"; all rows at once would need about {dense_bytes(cfg) / 1e9:.0f} GB"),
        "stage_s": {"a": t_a, "c": t_c, "d": t_d, "projections": t_proj},
    }


def dense_bytes(cfg):
    """Host memory the reference's dense algorithm needs for one batch element with
    every row at once: fp32 scores [n, h_kv, g, n], their masked copy and group
    mean, the candidate mask, the gathered K and V."""
    n, h_q, h_kv, d, k = cfg["n"], cfg["h_q"], cfg["h_kv"], cfg["d"], cfg["k"]
    s = 2 if cfg["dtype"] == "bf16" else 4
    return 4 * n * n * h_q * 2 + 4 * n * n * h_kv + n * n * h_kv + 2 * n * h_kv * k * d * s


def cpu_oracle(cfg, q, k, v, router, inter, budget_s):
    """Times the linear-memory CPU oracle (oracle/ssa_oracle.c, OpenMP) on sampled
    rows of batch element 0 and extrapolates each stage to the full forward (all
    batch elements).  Its outputs on the sample are checked equal to the GPU's."""
    import numpy as np
    import torch

    import oracle

    threads = cpu_share()
    oracle.set_threads(threads)
    n, h_q, h_kv, d = cfg["n"], cfg["h_q"], cfg["h_kv"], cfg["d"]
    g = h_q // h_kv
    qf = oracle.to_f32(q[0])
    kf = oracle.to_f32(k[0])
    vf = oracle.to_f32(v[0])
    w_qr = oracle.to_f32(router.W_qr.weight)
    w_kr = oracle.to_f32(router.W_kr.weight)
    cb = oracle.to_f32(router.codebook)
    qc, kc, off, post, idx = (t[0].cpu().numpy() for t in inter)
    # Stage (a) on a sample of token rows (queries and keys), scaled by n / sample.
    sa = max(64, min(n, 2048))
    rows_a = np.linspace(0, n - 1, sa).astype(np.int64)
    t0 = time.perf_counter()
    chat = oracle.normalize(cb)
    qh = oracle.route_vectors(qf[rows_a], w_qr, g)
    kh = oracle.route_vectors(kf[rows_a], w_kr, 1)
    qcs = oracle.code_topk(qh, chat, cfg["a"])
    kcs = oracle.code_topk(kh, chat, cfg["b"])
    t_a = (time.perf_counter() - t0) * n / sa
    assert np.array_equal(qcs, qc[:, rows_a]) and np.array_equal(kcs, kc[:, rows_a]), \
        "CPU baseline: stage (a) sample disagrees with the GPU codes"
    # Stage (b) in full.
    t0 = time.perf_counter()
    roff, rpost = oracle.build_index(kc, cfg["n_c"])
    t_b = time.perf_counter() - t0
    # Stages (c), (d) on query rows spread over all positions, grown until the budget.
    sc = 64
    while True:
        rows = np.linspace(0, n - 1, sc).astype(np.int64)
        t0 = time.perf_counter()
        sel = oracle.select(qf, kf, qc, roff, rpost, cfg["b"], cfg["k"], oracle.MASK_CAUSAL,
                            rows=rows, sorted=False)
        t_c1 = time.perf_counter() - t0
        t0 = time.perf_counter()
        oracle.sparse_attention(qf, kf, vf, sel, causal=True, rows=rows)
        t_d1 = time.perf_counter() - t0
        spent = t_a * sa / n + t_b + t_c1 + t_d1
        if spent > budget_s / 2 or sc >= n:
            break
        sc = min(n, sc * 4)
    assert np.array_equal(sel, idx[rows]), "CPU baseline: stage (c) sample disagrees with the GPU"
    t_c = t_c1 * n / sc
    t_d = t_d1 * n / sc
    total = t_a + t_b + t_c + t_d
    cpu = _cpu_model()
    return {
        "value": n / total,
        "unit": "tokens/s",
        "cores": threads,
        "host_cpus": os.cpu_count(),
        "kind": "port",
        "sample": (f"linear CPU oracle (oracle/ssa_oracle.c, OpenMP {threads} threads of {os.cpu_count()} "
                   f"host CPUs, {cpu}): stage a on "
                   f"{sa} of {n} token rows, stage b in full, stages c+d on {sc} of {n} query "
                   f"positions (all {h_kv} kv heads), each scaled to n; outputs checked equal to "
                   f"the GPU's on the sample"),
        "stage_s": {"a": t_a, "b": t_b, "c": t_c, "d": t_d},
    }


def measured_traffic(workload, kernel="stage_d"):
    """Bytes between L2 and the fabric per stage-(d) call (its two kernels) at
    `workload`, from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
    (profiles/sparse_attention_<workload>_traffic.md, line ``traffic_bytes
    stage_d <workload> <bytes>``); None when no such profile exists."""
    path = os.path.join(ROOT, "profiles", f"sparse_attention_{workload}_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 4 and parts[:3] == ["traffic_bytes", kernel, workload]:
                    return float(parts[3]), os.path.relpath(path, ROOT)
    except OSError:
        pass
    return None, None


def copy_probe(gib):
    import torch

    nbytes = int(gib * (1 << 30))
    x = torch.empty(nbytes // 4, device="cuda", dtype=torch.float32).fill_(1.0)
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    y.copy_(x)
    torch.cuda.synchronize()
    return nbytes


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 (the sharded path "
                                   "is designed, not built)"}))
        sys.exit(2)
    import torch

    import ssa_amd

    ssa_amd._lib.load()
    dev = torch.device("cuda:0")
    cfg = dict(CONFIGS[args.config])
    if args.n:
        cfg["n"] = args.n
    if args.num_codebook:
        cfg["n_c"] = args.num_codebook
    if args.copy_probe_gib > 0:
        nb = copy_probe(args.copy_probe_gib)
        print(f"copy probe: {nb} bytes read, {nb} bytes written", file=sys.stderr, flush=True)

    is_block = "d_model" in cfg
    blk = None
    if is_block:
        blk = make_block(cfg, args.seed, dev)
        torch.cuda.synchronize()
        print(f"block ready: {args.config} B={cfg['B']} n={cfg['n']}", file=sys.stderr, flush=True)
        with torch.no_grad():
            for _ in range(args.warmup):
                block_step(blk)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(args.steps):
                block_step(blk)
            torch.cuda.synchronize()
            wall = time.perf_counter() - t0
            phases = block_stages(blk)
            q, k, v = blk["layer"].project(blk["norm"](blk["x"]), None, blk["freqs"])
        router = blk["layer"].router
        st = {key: phases[key] for key in "abcd"}
    else:
        q, k, v, router = make_workload(cfg, args.seed, dev)
        torch.cuda.synchronize()
        print(f"workload ready: {args.config} n={cfg['n']}", file=sys.stderr, flush=True)
        wall, st = time_gpu(cfg, q, k, v, router, args.steps, args.warmup)
    ms_step = 1000.0 * wall / args.steps
    R, C, heavy_rows, C_r, nrows, distinct, inter, prefix_slots = stats_sums(q, k, router)
    alg = algorithmic(cfg, cfg["n"], (R, C, C_r, heavy_rows), distinct)
    tokens = cfg["B"] * cfg["n"]
    t = {key: st[key] / 1000.0 for key in "abcd"}
    d_comp_gbs = alg["d_bytes_compulsory"] / t["d"] / 1e9
    # Counter-measured traffic applies only to the profiled workload shape.
    traffic, traffic_src = (measured_traffic(args.config) if args.n is None and args.num_codebook is None and args.seed == 0
                            else (None, None))
    scoring_gflop = (alg["a_flops"] - alg["a_flops_projection"]) / 1e9
    scoring_ms = None if is_block else time_code_scoring(cfg, q, k, router)
    stages = {
        "a": {"ms": st["a"], "gflop": alg["a_flops"] / 1e9,
              "gflop_fp32_projection": alg["a_flops_projection"] / 1e9,
              "tflops": alg["a_flops"] / t["a"] / 1e12,
              "frac_mfma_bf16": alg["a_flops"] / t["a"] / 1e12 / MFMA_BF16_PEAK_TFLOPS},
        "b": {"ms": st["b"], "gb": alg["b_bytes"] / 1e9,
              "frac_hbm": alg["b_bytes"] / t["b"] / 1e9 / HBM_PEAK_GBS},
        "c": {"ms": st["c"], "order": "index (same set as by score)",
              "gb_read": alg["c_bytes"] / 1e9,
              "frac_hbm_read": alg["c_bytes"] / t["c"] / 1e9 / HBM_PEAK_GBS,
              "gb_scope_formula": alg["c_bytes_survey"] / 1e9,
              "gbs_scope_formula": alg["c_bytes_survey"] / t["c"] / 1e9,
              "ms_sorted_by_score": time_sorted_select(q, k, router),
              "postings_read": R, "candidates": C, "rows": nrows,
              "rows_rescored": heavy_rows, "candidates_rescored": C_r},
        "d": {"ms": st["d"], "gb_compulsory": alg["d_bytes_compulsory"] / 1e9,
              "frac_hbm_compulsory": d_comp_gbs / HBM_PEAK_GBS,
              "distinct_kv_rows": distinct,
              "slots": nrows * cfg["k"], "slots_in_dense_prefixes": prefix_slots,
              "gb_logical_gather": alg["d_bytes_logical"] / 1e9,
              "gbs_logical_gather": alg["d_bytes_logical"] / t["d"] / 1e9,
              "tflops": alg["d_flops"] / t["d"] / 1e12},
    }
    if scoring_ms is not None:
        stages["a"]["scoring"] = {
            "ms": scoring_ms, "gflop": scoring_gflop,
            "tflops": scoring_gflop / scoring_ms, "frac_mfma_bf16": scoring_gflop / scoring_ms / MFMA_BF16_PEAK_TFLOPS,
            "calls": "ssa_code_topk for the query codes (top a) and the key codes (top b): codebook "
                     "preparation, bf16 matrix-core screen, exact fp32 rescoring"}
    spread_ms = time_spread_attention(q, k, v, inter[4])
    if spread_ms is not None:
        stages["d"]["spread_keys"] = {
            "ms": spread_ms,
            "index_set": "k distinct keys per row spread over the sequence (no filler, unmasked)",
            "gbs_logical_gather": alg["d_bytes_logical"] / (spread_ms / 1000.0) / 1e9}
    workload = (f"{args.config}: RMSNorm + SSAAttention forward (projections, RoPE, stages a-d, "
                f"o_proj), causal routing" if is_block else
                f"{args.config}: SSA forward (stages a-d), causal")
    if is_block:
        data = "synthetic: hidden states ~ N(0,1); layer, RMSNorm and router default init from a fixed seed"
    else:
        data = ("synthetic: seeded Gaussian-mixture Q/K (%d clusters, sigma %.1f, RoPE theta %g), "
                "V ~ N(0,1); router default init from a fixed seed" %
                (cfg["clusters"], cfg["sigma"], cfg["theta"]))
    config = {"workload": workload, "batch": cfg["B"], "seq_len": cfg["n"], "h_q": cfg["h_q"],
              "h_kv": cfg["h_kv"], "head_dim": cfg["d"], "route_dim": cfg["d_s"],
              "num_codebook": cfg["n_c"], "codes_per_query": cfg["a"], "codes_per_key": cfg["b"],
              "top_k": cfg["k"]}
    if is_block:
        config["d_model"] = cfg["d_model"]
        stages["block_phases_ms"] = phases
    line = {
        "metric": METRIC,
        "value": tokens / (wall / args.steps),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": data,
        "config": config,
        "roofline": {"bound": "hbm",
                     "kernel": "stage d: prefix_attention_kernel + sparse_attention_mfma_kernel",
                     "achieved": d_comp_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": d_comp_gbs / HBM_PEAK_GBS, "traffic": traffic,
                     "traffic_counter": "FETCH_SIZE + WRITE_SIZE (bytes between L2 and the fabric; "
                                        "the 256 MB Infinity Cache serves part of them)",
                     "traffic_source": traffic_src,
                     "algorithmic_bytes": alg["d_bytes_compulsory"],
                     "algorithmic_basis": "compulsory: q and output once, int32 indices once, each "
                                          "distinct K/V row once",
                     "logical_gather_bytes": alg["d_bytes_logical"],
                     "logical_gather_gbs": alg["d_bytes_logical"] / t["d"] / 1e9},
        "stages": stages,
    }
    # The default c3 run also records the backward, single-token decoding at
    # the full cache and config 4 (the flags set other sizes).
    extras = args.config == "c3" and not args.no_extras and args.n is None and args.num_codebook is None
    if args.backward or extras:
        line["backward"] = time_backward(cfg, q, k, v, inter)
        print(f"backward: {line['backward']['ms']:.3f} ms", file=sys.stderr, flush=True)
    if args.decode > 0 or extras:
        line["decode"] = time_decode(cfg, q, k, v, router, args.decode if args.decode > 0 else 128)
        print(f"decode: {line['decode']['ms_per_token']:.3f} ms per token", file=sys.stderr, flush=True)
        if args.decode_lens:
            by_len = {}
            for n_ in [int(x) for x in args.decode_lens.split(",")]:
                for policy in ("fixed", "scaled"):
                    c2 = dict(cfg, n=n_)
                    if policy == "scaled":
                        c2["n_c"] = max(16, cfg["n_c"] * n_ // cfg["n"])
                    q2, k2, v2, r2 = make_workload(c2, args.seed, dev)
                    by_len[f"{n_}_{policy}"] = dict(time_decode(c2, q2, k2, v2, r2, args.decode),
                                                    num_codebook=c2["n_c"])
                    print(f"decode n={n_} N_c={c2['n_c']}: "
                          f"{by_len[f'{n_}_{policy}']['ms_per_token']:.3f} ms", file=sys.stderr, flush=True)
                    del q2, k2, v2, r2
            line["decode_by_cache_len"] = by_len
    if args.block_sparse > 0:
        line["block_sparse"] = time_blocks(cfg, q, k, v, inter, args.block_sparse)
    if not args.no_cpu_baseline:
        print("cpu baseline: reference algorithm", file=sys.stderr, flush=True)
        line["cpu_baseline"] = cpu_reference(cfg, q, k, v, router, args.cpu_seconds, blk)
        print("cpu baseline: linear oracle", file=sys.stderr, flush=True)
        line["cpu_oracle"] = cpu_oracle(cfg, q, k, v, router, inter, args.cpu_seconds)
    sweep_ns = args.sweep
    if sweep_ns is None:
        default_shape = args.config == "c3" and args.n is None and args.num_codebook is None
        sweep_ns = ",".join(str(x) for x in DEFAULT_SWEEP) if default_shape and not args.no_extras else ""
    if sweep_ns:
        ns = [int(x) for x in sweep_ns.split(",")]
        policies = ("scaled", "fixed") if args.sweep_nc == "both" else (args.sweep_nc,)
        steps = max(3, args.steps // 4)
        line["sweep"] = {pol: run_sweep(cfg, ns, pol, args.seed, dev, steps) for pol in policies}
    if extras:
        del q, k, v, inter
        line["c5"] = run_c5(args.seed, dev, max(3, args.steps // 4), 2)
        line["c4"] = run_c4(args.seed, dev, max(3, args.steps // 4), 2)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
