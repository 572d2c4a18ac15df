#!/usr/bin/env python3
"""Benchmark of the int4 sparse-attention KV-retrieval decode step on one MI355X.

A "step" is one decode step of every layer of the workload: per layer, the
fused int4 scoring + block max kernel, the top-k kernel and the GQA sparse
attention (partial + merge).  Inputs (K/V bf16, int4 packed K, subset slab,
q) are generated and quantized before the timed region and stay resident in
HBM; every layer has its own buffers, so a step streams far more than the
256 MB Infinity Cache.  The step is captured once in a HIP graph and
replayed.

Prints ONE JSON line (the driver contract): value = keys scored per second
over the whole step, where a key is one (sequence, KV head, token) row.
"roofline" is the scoring kernel's achieved algorithmic GB/s (HIP events
around graph-replayed launches of that kernel alone) against 8 TB/s.
"cpu_baseline" is the reference's PyTorch CPU op sequence (restated in
oracle/ref_semantics.py) timed on the host cores on a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "int4 partial-QK keys scored/s + HBM GB/s % of peak; sparse decode µs/layer"


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--config", default="cfg2", choices=["cfg1", "cfg2", "cfg3", "cfg4"])
    p.add_argument("--kernel-reps", type=int, default=20, help="graph replays for per-kernel timing")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample budget")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--eager", action="store_true", help="time eager launches instead of a HIP graph")
    p.add_argument("--profile-steps", type=int, default=0,
                   help="extra eager steps after timing, for rocprofv3 kernel statistics")
    p.add_argument("--copy-probe-mb", type=int, default=0,
                   help="also run a plain device copy of this many MiB (HBM counter calibration)")
    return p.parse_args()


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def graph_of(fn):
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def time_replays(replay, reps: int) -> float:
    """Milliseconds per replay, HIP events on the current stream."""
    import torch

    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def cpu_baseline(cfg, budget_s: float) -> dict:
    """The reference's qabs{S}cand{pct}attn op sequence on CPU tensors for one
    sequence of one layer, repeated for about ``budget_s`` seconds."""
    import torch

    from kv_cache_amd.workloads import make_layer
    from oracle import ref_semantics as R

    cores = max(1, min(16, os.cpu_count() or 1))
    torch.set_num_threads(cores)
    q, k, v, _ = make_layer(cfg, 0, device="cpu", batch=1)
    qs = q[:, :, None, :]
    frac = cfg.topk * cfg.block / cfg.tokens
    run = lambda: R.qabs_candidate_attention_cpu(qs, k, v, cfg.selected, frac, cfg.scaling)  # noqa: E731
    run()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 200):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    keys = cfg.kv_heads * cfg.tokens
    cpu_name = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_name = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": keys / med,
        "unit": "keys/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"one sequence x one layer of {cfg.name}: reference op sequence (top-|q| {cfg.selected} "
                   f"dims, fp32 partial scores over GQA-expanded bf16 K, top {frac:.4%} tokens, gather "
                   f"attention) on CPU tensors; {keys} keys/call, median of {len(times)} calls "
                   f"= {med * 1e3:.1f} ms; {cpu_name}"),
    }


def read_traffic(config: str, kernel: str):
    """HBM bytes per launch of ``kernel`` at ``config``, measured by two
    rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) scaled by a device copy
    of known size; recorded in profiles/hbm_traffic.json (None if absent)."""
    p = ROOT / "profiles" / "hbm_traffic.json"
    if not p.exists():
        return None
    try:
        data = json.loads(p.read_text())
        return data.get(config, {}).get(kernel, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        log(f"bench.py measures one GPU only (got --gpus {args.gpus}); this path shards per "
            "(sequence, KV head) without exchange and is not run across GPUs here")
        return 2

    import torch

    from kv_cache_amd import int4 as K
    from kv_cache_amd.workloads import CONFIGS, make_layer

    torch.cuda.set_device(0)
    cfg = CONFIGS[args.config]
    layers, rows, T = cfg.layers, cfg.rows, cfg.tokens
    log(f"[bench] setup {cfg.name}: {layers} layers, rows={rows}, T={T}, S={cfg.selected}, "
        f"block={cfg.block}, top-{cfg.topk}")
    qs, ks, vs, caches = [], [], [], []
    for layer in range(layers):
        q, k, v, _ = make_layer(cfg, layer, device="cuda")
        caches.append(K.Int4KCache.from_prefill(k, cfg.group, cfg.selected))
        qs.append(q)
        ks.append(k)
        vs.append(v)
    torch.cuda.synchronize()
    log(f"[bench] resident: {torch.cuda.memory_allocated() / 2**30:.1f} GiB")

    step = K.SparseDecodeStep(cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.head_dim, T, cfg.block, cfg.topk)

    def run_step():
        for layer in range(layers):
            step(qs[layer], caches[layer], ks[layer], vs[layer], cfg.scaling)

    def run_scores():
        for layer in range(layers):
            c = caches[layer]
            K.decode_scores(qs[layer], c.chan_idx, c.slab, c.slab_scales, T, cfg.block, bmax=step.bmax)

    def run_topk():
        for _ in range(layers):
            K.block_topk(step.bmax, cfg.topk, out=step.sel)

    def run_attn():
        for layer in range(layers):
            K.sparse_attention(qs[layer], ks[layer], vs[layer], step.sel, cfg.block, T, cfg.scaling,
                               workspace=step.workspace, out=step.out)

    dense_sel = torch.arange(cfg.n_blocks, dtype=torch.int32, device="cuda").repeat(rows, 1).contiguous()
    dense_ws = K.attention_workspace(cfg.batch, cfg.q_heads, cfg.kv_heads, cfg.head_dim, cfg.n_blocks,
                                     cfg.block, "cuda")
    dense_out = torch.empty_like(step.out)

    def run_dense():
        for layer in range(layers):
            K.sparse_attention(qs[layer], ks[layer], vs[layer], dense_sel, cfg.block, T, cfg.scaling,
                               workspace=dense_ws, out=dense_out)

    for _ in range(args.warmup):
        run_step()
    torch.cuda.synchronize()
    log("[bench] warmup done")

    replay = run_step if args.eager else graph_of(run_step).replay
    ms_per_step = time_replays(replay, args.steps)
    log(f"[bench] step: {ms_per_step:.3f} ms ({ms_per_step * 1e3 / layers:.1f} us/layer)")

    kernels = {}
    keys_per_layer = rows * T
    sel_tokens = min(T, cfg.topk * cfg.block)
    plan = [
        ("int4_decode_scores", run_scores, keys_per_layer * cfg.slab_bytes_per_key()),
        ("topk", run_topk, rows * cfg.n_blocks * 4),
        ("sparse_attention", run_attn, rows * sel_tokens * cfg.head_dim * 2 * 2),
        ("dense_bf16_attention", run_dense, rows * T * cfg.head_dim * 2 * 2),
    ]
    for name, fn, nbytes in plan:
        g = graph_of(fn)
        ms = time_replays(g.replay, args.kernel_reps) / layers
        kernels[name] = {"us_per_launch": ms * 1e3, "bytes_per_launch": nbytes,
                         "gbs": nbytes / (ms * 1e-3) / 1e9, "frac_hbm_peak": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
        log(f"[bench] {name}: {ms * 1e3:.2f} us/launch, {kernels[name]['gbs']:.0f} GB/s")
        del g

    for _ in range(args.profile_steps):
        run_step()
    if args.copy_probe_mb:
        n = args.copy_probe_mb * 2**20 // 4
        src = torch.ones(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
    torch.cuda.synchronize()

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline ...")
        cpu = cpu_baseline(cfg, args.cpu_seconds)
        log(f"[bench] cpu baseline: {cpu['value']:.3e} keys/s on {cpu['cores']} cores")

    sc = kernels["int4_decode_scores"]
    value = layers * keys_per_layer / (ms_per_step * 1e-3)
    line = {
        "metric": METRIC,
        "value": value,
        "unit": "keys/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i32 (int8 query x int4 K); bf16->f32 attention",
        "data": "synthetic (seeded N(0,1) K/V/q, 4 outlier channels x8)",
        "config": {
            "workload": f"{args.config}: {cfg.name}",
            "batch": cfg.batch, "q_heads": cfg.q_heads, "kv_heads": cfg.kv_heads, "head_dim": cfg.head_dim,
            "context": T, "layers": layers, "int4_group": cfg.group, "channels": cfg.selected,
            "block": cfg.block, "topk_blocks": cfg.topk, "graph": not args.eager,
        },
        "us_per_layer": ms_per_step * 1e3 / layers,
        "dense_bf16_us_per_layer": kernels["dense_bf16_attention"]["us_per_launch"],
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_scores_kernel (int4 scoring + block max)",
            "achieved": sc["gbs"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": sc["gbs"] / HBM_PEAK_GBS,
            "traffic": read_traffic(args.config, "decode_scores_kernel"),
        },
        "kernels": kernels,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
