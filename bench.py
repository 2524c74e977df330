"""SSA forward benchmark on one MI355X.

One step = one full SSA forward over resident inputs: routing vectors and
codebook top-codes (stage a), inverted index (b), candidate selection (c) and
gathered-KV attention (d), exactly as CodebookRouter + sparse_exact_attention
run them.  Workload (default): BASELINE config 3 -- 1 x 32768 tokens, bf16,
GQA 32/8, d 128, d_s 32, N_c 4096, a 16, b 4, k 512, causal, RoPE theta 1e6 on
a seeded 64-cluster Gaussian mixture (sigma 0.3), V ~ N(0, 1).

Prints ONE JSON line (rank 0) with the metric, per-stage times, the roofline
of the dominant kernel (stage d, HIP events on the launch stream) and a
bounded CPU-oracle baseline.
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
FP32_PEAK_TFLOPS = 157.3

CONFIGS = {
    "c3": dict(B=1, n=32768, h_q=32, h_kv=8, d=128, d_s=32, n_c=4096, b=4, a=16, k=512,
               clusters=64, sigma=0.3, theta=1e6, dtype="bf16"),
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
    p.add_argument("--block-sparse", type=int, default=0,
                   help="also time the block-granular variant with this many 64-key blocks per "
                        "query block (block indices from the workload's selections, then attention)")
    p.add_argument("--sweep", default="", help="comma list of n for a tokens/s vs n sweep")
    p.add_argument("--sweep-nc", default="scaled", choices=("scaled", "fixed"),
                   help="codebook size in the sweep: scaled with n (constant bucket size; the "
                        "config's N_c at its own n) or fixed at the config's N_c")
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


def algorithmic(cfg, n, stats_sum=None):
    """Algorithmic bytes / flops per stage for one forward (B*n*h_kv rows)."""
    B, h_q, h_kv, d = cfg["B"], cfg["h_q"], cfg["h_kv"], cfg["d"]
    s = 2 if cfg["dtype"] == "bf16" else 4
    g = h_q // h_kv
    rows = B * n * h_kv
    a, b, k, n_c, d_s = cfg["a"], cfg["b"], cfg["k"], cfg["n_c"], cfg["d_s"]
    out = {}
    out["a_flops"] = 2 * B * n * (h_q + h_kv) * d * d_s + 4 * rows * n_c * d_s
    out["a_bytes"] = B * n * (h_q + h_kv) * d * s + h_kv * n_c * d_s * 4 + rows * (a + b) * 4
    out["b_bytes"] = 3 * rows * b * 4 + h_kv * B * (n_c + 1) * 4
    if stats_sum is not None:
        # index order: postings, the K rows of the rescored rows' candidates and
        # their query rows, q_codes and bucket bounds, the output row
        R, C_r, heavy = stats_sum
        out["c_bytes"] = R * 4 + C_r * d * s + heavy * g * d * s + rows * (3 * a * 4 + k * 4)
        out["c_flops"] = C_r * 2 * d * g
    out["d_bytes"] = rows * (k * 4 + 2 * k * d * s + 2 * g * d * s)
    out["d_flops"] = 4 * rows * g * k * d
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
    # rows of each head grouped by best code (results do not depend on the order).
    idx = kernels.select(q, k, qc, off, post, router.codes_per_key, router.top_k, sorted=False,
                         index_dtype=torch.int32, row_order=order)
    if events:
        events[3].record()
    out = kernels.sparse_attention(q, k, v, idx, None, True, row_order=order)
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


def stats_sums(q, k, router):
    import torch

    from ssa_amd import kernels

    qc, kc = kernels.route_codes(q, k, router.W_qr.weight, router.W_kr.weight, router.codebook,
                                 router.codes_per_query, router.codes_per_key, router.temperature)
    off, post = kernels.build_index(kc, router.num_codebook)
    idx, st = kernels.select(q, k, qc, off, post, router.codes_per_key, router.top_k,
                             with_stats=True, sorted=False)
    st = st.to(torch.int64)
    C = int(st[..., 0].sum())
    R = int(st[..., 1].sum())
    heavy = st[..., 0] > router.top_k      # index order rescores only these rows
    C_r = int(st[..., 0][heavy].sum())
    return R, C, int(heavy.sum()), C_r, st[..., 0].numel(), (qc, kc, off, post, idx)


def time_backward(cfg, q, k, v, inter, reps=3):
    """Stage (d) backward (ssa_sparse_attention_backward) on the forward's indices
    and query order, with an fp32 forward output and a seeded bf16 output
    gradient; median of `reps` launches (HIP events on the launch stream)."""
    import torch

    from ssa_amd import kernels

    qc, kc, off, post, _ = inter
    order = kernels.query_order(qc, cfg["n_c"])
    idx = kernels.select(q, k, qc, off, post, cfg["b"], cfg["k"], sorted=False,
                         index_dtype=torch.int32, row_order=order)
    out32 = torch.empty(q.shape, device=q.device, dtype=torch.float32)
    kernels.sparse_attention(q, k, v, idx, None, True, out=out32, row_order=order)
    gen = torch.Generator(device=q.device).manual_seed(7)
    dout = torch.randn(q.shape, generator=gen, device=q.device).to(q.dtype)
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        kernels.sparse_attention_backward(q, k, v, idx, out32, dout, None, True, row_order=order)
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1))
    ms = sorted(ts)[len(ts) // 2]
    B, n, h_q, h_kv, d, kk = cfg["B"], cfg["n"], cfg["h_q"], cfg["h_kv"], cfg["d"], cfg["k"]
    s = 2 if cfg["dtype"] == "bf16" else 4
    rows = B * n * h_kv
    g = h_q // h_kv
    # per row: K gathered twice (two passes) and V once, indices twice, q/dO
    # (input type) and o (fp32) read, dq written, dk and dv read-modify-written
    byt = rows * (3 * kk * d * s + 2 * kk * 4 + g * d * (2 * s + 4) + g * d * 4 + 2 * kk * d * 8)
    return {"ms": ms, "tokens_per_s": B * n / (ms / 1000), "kernel": "sparse_attention_bwd_kernel",
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


def time_decode(cfg, q, k, v, router, steps):
    """Single-token decode steps (ssa_amd.decode.SSADecodeCache) for the last
    `steps` tokens of the workload after a prefill of the rest; wall time per
    step on the host (each step launches about a dozen kernels)."""
    import torch

    from ssa_amd.decode import SSADecodeCache

    n = cfg["n"]
    cache = SSADecodeCache(router, cfg["B"], n, cfg["d"], dtype=q.dtype)
    n0 = n - steps
    cache.step(q[:, :n0], k[:, :n0], v[:, :n0])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for t in range(n0, n):
        cache.step(q[:, t:t + 1], k[:, t:t + 1], v[:, t:t + 1])
    torch.cuda.synchronize()
    ms = 1000 * (time.perf_counter() - t0) / steps
    return {"ms_per_token": ms, "tokens_per_s": cfg["B"] / (ms / 1000), "cache_len": n,
            "steps": steps, "prefill_tokens": n0}


def cpu_baseline(cfg, q, k, v, router, inter, budget_s):
    """Times the CPU oracle (oracle/ssa_oracle.c, OpenMP) on sampled rows of the same
    workload and extrapolates each stage to the full forward."""
    import numpy as np
    import torch

    import oracle

    threads = min(16, os.cpu_count() or 1)
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
    cpu = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": cfg["B"] * n / total,
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"CPU oracle (oracle/ssa_oracle.c, OpenMP {threads} threads, {cpu}): stage a on "
                   f"{sa} of {n} token rows, stage b in full, stages c+d on {sc} of {n} query "
                   f"positions (all {h_kv} kv heads), each scaled to n; outputs checked equal to "
                   f"the GPU's on the sample"),
        "stage_s": {"a": t_a, "b": t_b, "c": t_c, "d": t_d},
    }


def measured_traffic(workload, kernel="sparse_attention_mfma_kernel"):
    """HBM bytes per launch of `kernel` at `workload`, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (profiles/<kernel>_<workload>_traffic.md, line
    ``traffic_bytes <kernel> <workload> <bytes>``); None when no such profile exists."""
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
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 (sharding design is "
                                   "described in DESIGN.md, not built)"}))
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

    q, k, v, router = make_workload(cfg, args.seed, dev)
    torch.cuda.synchronize()
    print(f"workload ready: {args.config} n={cfg['n']}", file=sys.stderr, flush=True)
    wall, st = time_gpu(cfg, q, k, v, router, args.steps, args.warmup)
    ms_step = 1000.0 * wall / args.steps
    R, C, heavy_rows, C_r, nrows, inter = stats_sums(q, k, router)
    alg = algorithmic(cfg, cfg["n"], (R, C_r, heavy_rows))
    tokens = cfg["B"] * cfg["n"]
    t_d = st["d"] / 1000.0
    d_gbs = alg["d_bytes"] / t_d / 1e9
    # Counter-measured traffic applies only to the profiled workload shape.
    traffic, traffic_src = (measured_traffic(args.config) if args.n is None and args.num_codebook is None and args.seed == 0
                            else (None, None))
    stages = {
        "a": {"ms": st["a"], "gflop": alg["a_flops"] / 1e9,
              "tflops": alg["a_flops"] / (st["a"] / 1000) / 1e12,
              "frac_mfma_bf16": alg["a_flops"] / (st["a"] / 1000) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
              "frac_fp32": alg["a_flops"] / (st["a"] / 1000) / 1e12 / FP32_PEAK_TFLOPS},
        "b": {"ms": st["b"], "gb": alg["b_bytes"] / 1e9,
              "frac_hbm": alg["b_bytes"] / (st["b"] / 1000) / 1e9 / HBM_PEAK_GBS},
        "c": {"ms": st["c"], "gb": alg["c_bytes"] / 1e9,
              "frac_hbm": alg["c_bytes"] / (st["c"] / 1000) / 1e9 / HBM_PEAK_GBS,
              "order": "index (same set as by score)",
              "ms_sorted_by_score": time_sorted_select(q, k, router),
              "postings_read": R, "candidates": C, "rows": nrows,
              "rows_rescored": heavy_rows, "candidates_rescored": C_r},
        "d": {"ms": st["d"], "gb": alg["d_bytes"] / 1e9, "frac_hbm": d_gbs / HBM_PEAK_GBS},
    }
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
        "data": ("synthetic: seeded Gaussian-mixture Q/K (%d clusters, sigma %.1f, RoPE theta %g), "
                 "V ~ N(0,1); router default init from a fixed seed" %
                 (cfg["clusters"], cfg["sigma"], cfg["theta"])),
        "config": {"workload": f"{args.config}: SSA forward (stages a-d), causal",
                   "batch": cfg["B"], "seq_len": cfg["n"], "h_q": cfg["h_q"], "h_kv": cfg["h_kv"],
                   "head_dim": cfg["d"], "route_dim": cfg["d_s"], "num_codebook": cfg["n_c"],
                   "codes_per_query": cfg["a"], "codes_per_key": cfg["b"], "top_k": cfg["k"]},
        "roofline": {"bound": "hbm", "kernel": "sparse_attention_mfma_kernel (stage d)",
                     "achieved": d_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": d_gbs / HBM_PEAK_GBS, "traffic": traffic,
                     "traffic_source": traffic_src,
                     "algorithmic_bytes": alg["d_bytes"]},
        "stages": stages,
    }
    if args.backward:
        line["backward"] = time_backward(cfg, q, k, v, inter)
    if args.decode > 0:
        line["decode"] = time_decode(cfg, q, k, v, router, args.decode)
    if args.block_sparse > 0:
        line["block_sparse"] = time_blocks(cfg, q, k, v, inter, args.block_sparse)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(cfg, q, k, v, router, inter, args.cpu_seconds)
    if args.sweep:
        sweep = {}
        for n_ in [int(x) for x in args.sweep.split(",")]:
            c2 = dict(cfg, n=n_)
            if args.sweep_nc == "scaled":
                c2["n_c"] = max(16, cfg["n_c"] * n_ // cfg["n"])
            q2, k2, v2, r2 = make_workload(c2, args.seed, dev)
            w2, s2 = time_gpu(c2, q2, k2, v2, r2, max(3, args.steps // 2), 1)
            ms2 = 1000 * w2 / max(3, args.steps // 2)
            sweep[n_] = {"ms": ms2, "tokens_per_s": c2["B"] * n_ / (ms2 / 1000), "num_codebook": c2["n_c"],
                         "stages_ms": s2}
            print(f"sweep n={n_}: {sweep[n_]['ms']:.3f} ms", file=sys.stderr, flush=True)
            del q2, k2, v2, r2
        ns = sorted(sweep)
        ts = [sweep[x]["ms"] for x in ns]
        if len(ns) >= 3:  # least-squares t = alpha * n + beta and its R^2
            mn, mt = sum(ns) / len(ns), sum(ts) / len(ts)
            sxx = sum((x - mn) ** 2 for x in ns)
            alpha = sum((x - mn) * (t - mt) for x, t in zip(ns, ts)) / sxx
            beta = mt - alpha * mn
            ss_res = sum((t - (alpha * x + beta)) ** 2 for x, t in zip(ns, ts))
            ss_tot = sum((t - mt) ** 2 for t in ts)
            sweep["fit"] = {"ms_per_token": alpha, "ms_offset": beta,
                            "r2": 1.0 - ss_res / ss_tot if ss_tot > 0 else 1.0}
        sweep["num_codebook_policy"] = args.sweep_nc
        line["sweep"] = sweep
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
