#!/usr/bin/env python3
"""Benchmark of the int4 sparse-attention KV-retrieval path on one MI355X.

Decode configs (cfg1-cfg4): a "step" is one decode step of every layer of
the workload: per layer, the fused int4 scoring + block max kernel, the
top-k selection and the GQA sparse attention.  The default is cfg3, the
largest configuration that fits one GPU (Qwen3-8B heads, batch 32, context
32768, all 36 layers resident: about 172 GiB), followed in the same run by
cfg2 (Qwen3-0.6B, 28 layers), whose figures go under "secondary".  Inputs (K/V bf16,
int4 packed K, subset slab, q) are generated and quantized before the timed
region and stay resident in HBM; every layer has its own buffers, so a step
streams far more than the 256 MB Infinity Cache.  The step is captured once
in a HIP graph and replayed.  value = keys scored per second over the whole
step, where a key is one (sequence, KV head, token) row; "roofline" is the
scoring kernel's achieved algorithmic GB/s (HIP events around graph-replayed
launches of that kernel alone) against 8 TB/s.  cfg4 also reports the
recall of its planted keys at k = 64, 256, 1024 tokens.

cfg5 (chunked prefill): a step is one layer's block selection for a chunk of
2048 queries against 65536 cached int4 keys (int8 query quantization, int8
MFMA block scores with the causal mask, top-64 blocks per query row), over
rotating per-layer buffers; value = (query head, visible key) pairs scored
per second; "roofline" is the MFMA scoring kernel's algorithmic int8 ops
per second against the 5.0 POP/s dense int8 peak.

reuse (candidate reuse + exact rerank, kv_cache_amd.reuse) and qbb / brep
(block-metadata selectors, kv_cache_amd.blocksel): a step is one decode token
through 8 layers of the qabs8cand5reuse / qbb64q8s3cand3 / brep64r4q8s3cand3
step at Qwen3-8B heads and history 32768; value = history tokens x KV heads x
layers per second.

"cpu_baseline" is timed on the host cores on a bounded sample: for decode
the reference's PyTorch op sequence (restated in oracle/ref_semantics.py),
for prefill the numpy restatement of the scoring (oracle/qkv_oracle.py), for
reuse / qbb / brep the reference's op sequence of that mode
(oracle/ref_semantics.py).
Prints ONE JSON line (the driver contract).
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
INT8_PEAK_TOPS = 5000.0   # dense int8 MFMA, MI355X
METRIC = "int4 partial-QK keys scored/s + HBM GB/s % of peak; sparse decode µs/layer"


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--config", default="cfg3",
                   choices=["cfg1", "cfg2", "cfg3", "cfg4", "cfg5", "reuse", "qbb", "brep", "qabsattn"],
                   help="workload (default cfg3: the largest single-GPU config, all 36 layers resident)")
    p.add_argument("--secondary", default=None,
                   help="a second decode config measured in the same run, reported under 'secondary' "
                        "(default: cfg2 when --config is cfg3; 'none' to skip)")
    p.add_argument("--layers", type=int, default=None,
                   help="layer buffers to rotate through (default: the config's layer count, at least 8)")
    p.add_argument("--kernel-reps", type=int, default=20, help="graph replays for per-kernel timing")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample budget")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--reuse-mode", default=None,
                   help="--config reuse: a qabs{S}cand{pct}reuse[final|2set][blk{bs}] mode (default qabs8cand5reuse)")
    p.add_argument("--qabs-mode", default="qabs8cand3attn",
                   help="--config qabsattn: a qabs{S}cand{pct}[append]attn mode")
    p.add_argument("--candidate-selection", default="topk", choices=["topk", "sample_quantile", "previous_threshold"],
                   help="--config reuse: the reference's --qabs_candidate_selection")
    p.add_argument("--eager", action="store_true", help="time eager launches instead of a HIP graph")
    p.add_argument("--profile-steps", type=int, default=0,
                   help="extra eager steps after timing, for rocprofv3 kernel statistics")
    p.add_argument("--copy-probe-mb", type=int, default=0,
                   help="also run a plain device copy of this many MiB (HBM counter calibration)")
    args = p.parse_args()
    if args.secondary is None:
        args.secondary = "cfg2" if args.config == "cfg3" else None
    elif args.secondary == "none":
        args.secondary = None
    elif args.secondary not in ("cfg1", "cfg2", "cfg3", "cfg4"):
        p.error("--secondary must be a decode config (cfg1-cfg4) or 'none'")
    return args


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


def host_threads() -> int:
    """Threads of the CPU baselines: every core this process may run on (its
    affinity set), capped by OMP_NUM_THREADS where the host sets it -- the GPU
    box sets it to the CPU share of its one GPU, which the whole host's
    os.cpu_count() does not reflect."""
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count() or 1
    try:
        cap = int(os.environ.get("OMP_NUM_THREADS", "0"))
    except ValueError:
        cap = 0
    return max(1, min(avail, cap) if cap > 0 else avail)


def cpu_name() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def host_note(threads: int) -> str:
    return f"{threads} threads on {cpu_name() or 'unknown CPU'} (os.cpu_count() = {os.cpu_count()})"


def cpu_baseline(cfg, budget_s: float) -> dict:
    """The reference's qabs{S}cand{pct}attn op sequence on CPU tensors for one
    sequence of one layer, repeated for about ``budget_s`` seconds.  Rows are
    independent, so the keys/s of one sequence is the rate of the full batch."""
    import torch

    from kv_cache_amd.workloads import make_layer
    from oracle import ref_semantics as R

    torch.set_num_threads(host_threads())
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
    return {
        "value": keys / med,
        "unit": "keys/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"one sequence (of {cfg.batch}) x one layer of {cfg.name}: reference op sequence (top-|q| "
                   f"{cfg.selected} dims, fp32 partial scores over GQA-expanded bf16 K, top {frac:.4%} tokens, "
                   f"gather attention) on CPU tensors; {keys} keys/call, median of {len(times)} calls "
                   f"= {med * 1e3:.1f} ms, keys/s scales linearly to the batch (rows are independent); "
                   f"{host_note(torch.get_num_threads())}"),
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

    torch.cuda.set_device(0)
    if args.config == "cfg5":
        line = run_prefill(args)
    elif args.config == "reuse":
        line = run_reuse(args)
    elif args.config in ("qbb", "brep"):
        line = run_blocksel(args)
    elif args.config == "qabsattn":
        line = run_qabs_attn(args)
    else:
        line = run_decode(args, args.config, args.layers)
        if args.secondary and args.secondary != args.config:
            # A second decode workload in the same run (default: cfg2 after the
            # cfg3 headline); its own buffers are built after the first's are freed.
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
            try:
                sec = run_decode(args, args.secondary, with_cpu=True)
                line["secondary"] = {k: sec[k] for k in ("config", "value", "unit", "ms_per_step", "us_per_layer",
                                                         "dense_bf16_us_per_layer", "roofline", "kernels",
                                                         "hbm_read_probe", "cpu_baseline")}
            except Exception as exc:   # the headline line is still printed
                log(f"[bench] secondary workload {args.secondary} failed: {exc!r}")
                line["secondary"] = {"config": {"workload": args.secondary}, "error": repr(exc)}
    print(json.dumps(line), flush=True)
    return 0


def copy_probe(mb: int) -> None:
    """Plain device copies of a known size (HBM counter calibration)."""
    import torch

    if mb:
        n = mb * 2**20 // 4
        src = torch.ones(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()


def hbm_read_probe(nbytes: int, reps: int = 20, min_total: int = 1 << 30) -> dict:
    """The read ceiling of one launch of ``nbytes``: libqkv's streaming-read
    probe (the scoring kernel's access shape, no arithmetic) over rotating
    buffers of that size (>= 1 GiB in all, so no launch finds its buffer in
    the 256 MB Infinity Cache), graph-replayed; HIP events on the stream the
    probe runs on."""
    import torch

    from kv_cache_amd import _lib

    lib = _lib.load()
    n_buf = max(2, -(-min_total // nbytes))
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(b % 251) for b in range(n_buf)]
    words = lib.qkv_hbm_read_probe_sink_words(nbytes)
    sink = torch.empty(words, dtype=torch.int32, device="cuda")

    def run():
        for b in bufs:
            _lib.check(lib.qkv_hbm_read_probe(b.data_ptr(), nbytes, sink.data_ptr(), words,
                                              torch.cuda.current_stream().cuda_stream))

    g = graph_of(run)
    ms = time_replays(g.replay, reps) / n_buf
    del g, bufs
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"bytes": nbytes, "us_per_launch": ms * 1e3, "gbs": gbs, "frac_hbm_peak": gbs / HBM_PEAK_GBS}


def planted_recall(cfg, qs, caches, planted, ks=(64, 256, 1024)) -> dict:
    """Fraction of (layer, row) planted keys inside the top-k tokens of the
    decode scoring, per k (OV:260-322's hits / true-count, one planted key)."""
    import torch

    from kv_cache_amd import int4 as K

    hits = {k: 0 for k in ks}
    total = 0
    for q, c, pl in zip(qs, caches, planted):
        bmax = K.decode_scores(q, c.chan_idx, c.slab, c.slab_scales, cfg.tokens, cfg.block)
        for k in ks:
            sel = K.block_topk(bmax, k // cfg.block)                        # [B, Hkv, k/block] block ids
            first = sel.to(torch.int64) * cfg.block
            inside = (pl[..., None] >= first) & (pl[..., None] < first + cfg.block)
            hits[k] += int(inside.any(dim=-1).sum())
        total += pl.numel()
    return {str(k): hits[k] / total for k in ks}


def run_decode(args, name: str, layers: int | None = None, with_cpu: bool = True) -> dict:
    import torch

    from kv_cache_amd import int4 as K
    from kv_cache_amd.workloads import CONFIGS, make_layer

    cfg = CONFIGS[name]
    # Single-layer configs rotate 8 distinct layer buffers (seeds seed..seed+7)
    # so that repeated steps do not run out of the 256 MB Infinity Cache.
    layers, rows, T = (layers or max(cfg.layers, 8)), cfg.rows, cfg.tokens
    log(f"[bench] setup {cfg.name}: {layers} layers, rows={rows}, T={T}, S={cfg.selected}, "
        f"block={cfg.block}, top-{cfg.topk}")
    qs, ks, vs, caches, planted = [], [], [], [], []
    for layer in range(layers):
        q, k, v, pl = make_layer(cfg, layer, device="cuda")
        caches.append(K.Int4KCache.from_prefill(k, cfg.group, cfg.selected))
        qs.append(q)
        ks.append(k)
        vs.append(v)
        planted.append(pl)
        if (layer + 1) % 8 == 0 and layer + 1 < layers:
            torch.cuda.synchronize()
            log(f"[bench] {layer + 1} layers built, {torch.cuda.memory_allocated() / 2**30:.1f} GiB")
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
            K.block_topk(step.bmax, cfg.topk, out=step.sel, workspace=step.topk_ws)

    def run_decode_topk():   # the step's token selection: scoring that also builds the top-k's chunk windows
        for layer in range(layers):
            c = caches[layer]
            K.decode_topk(qs[layer], c.chan_idx, c.slab, c.slab_scales, T, cfg.topk, scores=step.bmax,
                          out=step.sel, workspace=step.topk_ws)

    def run_attn():
        for layer in range(layers):
            K.sparse_attention(qs[layer], ks[layer], vs[layer], step.sel, cfg.block, T, cfg.scaling,
                               workspace=step.workspace, out=step.out)

    def run_select_attn():
        for layer in range(layers):
            K.sparse_attention_select(qs[layer], ks[layer], vs[layer], step.bmax, cfg.topk, cfg.block, T,
                                      cfg.scaling, workspace=step.workspace, sel_out=step.sel, out=step.out)

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

    # A graph of a few launches would time the host's graph launch, not the
    # GPU: short workloads are repeated inside the graph (>= 28 layer steps).
    reps = max(1, -(-28 // layers))

    def repeated(fn):
        def run():
            for _ in range(reps):
                fn()
        return run

    replay = run_step if args.eager else graph_of(repeated(run_step)).replay
    ms_per_step = time_replays(replay, args.steps) / (1 if args.eager else reps)
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
    if not step.fused and cfg.block == 1:   # scores written and read back once more by the top-k
        plan.insert(2, ("int4_decode_topk", run_decode_topk,
                        keys_per_layer * cfg.slab_bytes_per_key() + rows * cfg.n_blocks * 4 * 2))
    if step.fused:   # the step's own second launch: selection inside the attention kernel
        plan.insert(3, ("select_sparse_attention", run_select_attn,
                        rows * (cfg.n_blocks * 4 + sel_tokens * cfg.head_dim * 2 * 2)))
    for kname, fn, nbytes in plan:
        g = graph_of(repeated(fn))
        ms = time_replays(g.replay, args.kernel_reps) / (layers * reps)
        kernels[kname] = {"us_per_launch": ms * 1e3, "bytes_per_launch": nbytes,
                          "gbs": nbytes / (ms * 1e-3) / 1e9,
                          "frac_hbm_peak": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
        log(f"[bench] {kname}: {ms * 1e3:.2f} us/launch, {kernels[kname]['gbs']:.0f} GB/s")
        del g

    for _ in range(args.profile_steps):
        run_step()
    torch.cuda.synchronize()
    copy_probe(args.copy_probe_mb)
    recall = planted_recall(cfg, qs, caches, planted) if cfg.planted else None
    # the read ceiling of one launch of the scoring kernel's size (layer buffers freed first)
    fused = step.fused
    del qs, ks, vs, caches, planted, step, replay
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    probe = hbm_read_probe(keys_per_layer * cfg.slab_bytes_per_key())
    log(f"[bench] read probe of {probe['bytes'] / 1e6:.1f} MB: {probe['us_per_launch']:.2f} us/launch, "
        f"{probe['gbs']:.0f} GB/s ({probe['frac_hbm_peak']:.1%} of peak)")
    if recall:
        log(f"[bench] planted-key recall at k tokens: {recall}")

    cpu = None
    if with_cpu and not args.no_cpu_baseline:
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
            "workload": f"{name}: {cfg.name}",
            "batch": cfg.batch, "q_heads": cfg.q_heads, "kv_heads": cfg.kv_heads, "head_dim": cfg.head_dim,
            "context": T, "layers": layers, "int4_group": cfg.group, "channels": cfg.selected,
            "block": cfg.block, "topk_blocks": cfg.topk, "graph": not args.eager, "fused_select": fused,
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
            "traffic": read_traffic(name, "decode_scores_kernel"),
        },
        "kernels": kernels,
        "hbm_read_probe": probe,
        "cpu_baseline": cpu,
    }
    if recall:
        line["planted_recall"] = recall
    return line


def cpu_baseline_prefill(cfg, budget_s: float) -> dict:
    """The numpy restatement of prefill block scoring (oracle/qkv_oracle.py)
    on the host cores, for a few query rows of one head against all keys."""
    import numpy as np
    import torch

    from kv_cache_amd.workloads import make_prefill
    from oracle import qkv_oracle as O

    q, k = make_prefill(cfg, device="cpu")
    kp, ks = O.int4_pack_k(k[:, :1].float().numpy(), 128)
    rows = q[:, :1, -4:].float().numpy()                        # the chunk's last 4 queries of head 0
    q8, _ = O.quantize_query_rows(rows)
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        bm = O.prefill_block_scores(q8, kp, ks[..., 0], cfg.block, cfg.tokens - 4)
        O.prefill_block_topk(bm, cfg.topk)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    pairs = sum(min(cfg.tokens, cfg.tokens - 4 + i + 1) for i in range(4))
    return {
        "value": pairs / med,
        "unit": "query-key pairs/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"4 query rows x {cfg.tokens} int4 keys of one head: numpy int64 scoring (einsum, one "
                   f"thread), causal block-64 max, top-{cfg.topk}; median of {len(times)} calls = "
                   f"{med * 1e3:.1f} ms; {cpu_name() or 'unknown CPU'}"),
    }


def run_prefill(args) -> dict:
    import torch

    from kv_cache_amd import int4 as K
    from kv_cache_amd import prefill as P
    from kv_cache_amd.workloads import PREFILL, make_prefill

    cfg = PREFILL
    layers = args.layers or 8
    nb = cfg.n_blocks
    log(f"[bench] setup {cfg.name}: {layers} layer buffers, {cfg.queries} queries x {cfg.tokens} keys, "
        f"{cfg.q_heads}/{cfg.kv_heads} heads, block {cfg.block}, top-{cfg.topk}, q_pos0 {cfg.q_pos0}")
    qs, packs, scs = [], [], []
    for layer in range(layers):
        q, k = make_prefill(cfg, device="cuda")
        q = q + 0.0 * layer   # distinct buffers per layer, same values
        packed, scales = K.int4_pack_k(k, 128)
        del k
        qs.append(q.contiguous())
        packs.append(packed)
        scs.append(scales)
    q8 = torch.empty((cfg.batch, cfg.q_heads, cfg.queries, 128), dtype=torch.int8, device="cuda")
    bmax = torch.empty((cfg.batch, cfg.q_heads, cfg.queries, nb), dtype=torch.float32, device="cuda")
    sel = torch.empty((cfg.batch, cfg.q_heads, cfg.queries, cfg.topk), dtype=torch.int32, device="cuda")
    q8s = [P.quantize_query(qs[layer])[0] for layer in range(layers)]
    torch.cuda.synchronize()

    def run_step():
        for layer in range(layers):
            q8l, _ = P.quantize_query(qs[layer])
            P.block_scores(q8l, packs[layer], scs[layer], cfg.tokens, cfg.q_pos0, bmax=bmax)
            P.block_topk(bmax, cfg.topk, out=sel)

    def run_scores():
        for layer in range(layers):
            P.block_scores(q8s[layer], packs[layer], scs[layer], cfg.tokens, cfg.q_pos0, bmax=bmax)

    def run_topk():
        for _ in range(layers):
            P.block_topk(bmax, cfg.topk, out=sel)

    for _ in range(args.warmup):
        run_step()
    torch.cuda.synchronize()
    replay = run_step if args.eager else graph_of(run_step).replay
    ms_per_step = time_replays(replay, args.steps) / layers
    ops = cfg.int_ops()
    pairs = cfg.batch * cfg.q_heads * cfg.visible_keys()
    kernels = {}
    for name, fn in [("prefill_block_scores", run_scores), ("prefill_block_topk", run_topk)]:
        g = graph_of(fn)
        ms = time_replays(g.replay, args.kernel_reps) / layers
        kernels[name] = {"us_per_launch": ms * 1e3}
        del g
    sc_ms = kernels["prefill_block_scores"]["us_per_launch"] * 1e-3
    kernels["prefill_block_scores"]["tops"] = ops / (sc_ms * 1e-3) / 1e12
    log(f"[bench] layer step {ms_per_step * 1e3:.1f} us; scores {sc_ms * 1e3:.1f} us = "
        f"{kernels['prefill_block_scores']['tops']:.0f} TOP/s; top-k {kernels['prefill_block_topk']['us_per_launch']:.1f} us")
    for _ in range(args.profile_steps):
        run_step()
    torch.cuda.synchronize()
    copy_probe(args.copy_probe_mb)
    cpu = None if args.no_cpu_baseline else cpu_baseline_prefill(cfg, args.cpu_seconds)
    achieved = kernels["prefill_block_scores"]["tops"]
    return {
        "metric": METRIC,
        "value": pairs / (ms_per_step * 1e-3),
        "unit": "query-key pairs/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i32 (int8 query x int4 K)",
        "data": "synthetic (seeded N(0,1) q/K, 4 outlier channels x8)",
        "config": {
            "workload": f"cfg5: {cfg.name}", "batch": cfg.batch, "q_heads": cfg.q_heads,
            "kv_heads": cfg.kv_heads, "head_dim": cfg.head_dim, "queries": cfg.queries, "context": cfg.tokens,
            "q_pos0": cfg.q_pos0, "block": cfg.block, "topk_blocks": cfg.topk, "layer_buffers": layers,
            "graph": not args.eager,
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "prefill_scores_kernel (v_mfma_i32_16x16x64_i8, causal block-64 max)",
            "achieved": achieved,
            "peak": INT8_PEAK_TOPS,
            "unit": "TOP/s (int8)",
            "frac": achieved / INT8_PEAK_TOPS,
            "traffic": read_traffic("cfg5", "prefill_scores_kernel"),
            "ops_per_launch": ops,
        },
        "kernels": kernels,
        "cpu_baseline": cpu,
    }


# The candidate-reuse workload: Qwen3-8B heads, one sequence, 32768 history
# tokens, the reference's most-run reuse mode with its default final
# fraction and the sink/recent protection of its timed runs.
REUSE = {"name": "qwen3-8b-reuse-b1-h32768", "batch": 1, "q_heads": 32, "kv_heads": 8, "head_dim": 128,
         "history": 32768, "mode": "qabs8cand5reuse", "top_fraction": 0.02, "sink": 10, "recent": 10}


def cpu_baseline_reuse(budget_s: float, steps: int = 3) -> dict:
    """The reference's reuse op sequence (oracle/ref_semantics.py
    qabs_reuse_step_cpu) for consecutive decode steps of one layer on CPU
    tensors, about ``budget_s`` seconds."""
    import torch

    from oracle import ref_semantics as R
    from kv_cache_amd.reuse import parse_reuse_mode

    c = REUSE
    torch.set_num_threads(host_threads())
    g = torch.Generator().manual_seed(0)
    t = c["history"] + steps + 1
    k = torch.randn((1, c["kv_heads"], t, c["head_dim"]), generator=g).to(torch.bfloat16)
    v = torch.randn((1, c["kv_heads"], t, c["head_dim"]), generator=g).to(torch.bfloat16)
    dims, cand, _, _, _ = parse_reuse_mode(c["mode"])
    pc = pf = None
    times = []
    t_end = time.perf_counter() + budget_s
    for s in range(steps):
        n = c["history"] + s + 1
        q = torch.randn((1, c["q_heads"], 1, c["head_dim"]), generator=g).to(torch.bfloat16)
        fit = (lambda m: None if m is None else torch.cat([m, torch.zeros_like(m[..., :1])], dim=-1))
        t0 = time.perf_counter()
        _, pc, pf = R.qabs_reuse_step_cpu(q, k[:, :, :n], v[:, :, :n], dims, cand, c["top_fraction"],
                                          c["head_dim"] ** -0.5, c["sink"], c["recent"], True, fit(pc), fit(pf))
        times.append(time.perf_counter() - t0)
        if time.perf_counter() > t_end:
            break
    med = statistics.median(times[1:] if len(times) > 1 else times)
    keys = c["kv_heads"] * c["history"]
    return {
        "value": keys / med,
        "unit": "keys/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{len(times)} consecutive decode steps of one layer ({c['mode']}, {c['q_heads']}/{c['kv_heads']} "
                   f"heads, history {c['history']}): the reference's reuse op sequence on CPU tensors; "
                   f"median of the steps after the first = {med * 1e3:.1f} ms per layer-step"),
    }


def run_reuse(args) -> dict:
    """Decode steps of the candidate-reuse path (kv_cache_amd.reuse).  A step
    is one decode token through every layer; each layer keeps its own K/V,
    dim-major K copy and masks, and the history grows by one token per step.
    Timed eagerly (the step sizes change every token; host launch time
    included), then one step at a fixed history is captured in a HIP graph
    (GPU time), and each piece alone (per-kernel time)."""
    import torch

    from kv_cache_amd import reuse as RU

    c = dict(REUSE, mode=args.reuse_mode or REUSE["mode"])
    selection = args.candidate_selection
    layers = args.layers or 8
    b, hq, hkv, d, t0 = c["batch"], c["q_heads"], c["kv_heads"], c["head_dim"], c["history"]
    cap = -(-(t0 + args.warmup + args.steps + 2) // 64) * 64
    scaling = d ** -0.5
    log(f"[bench] setup {c['name']}: {layers} layers, {c['mode']}, top {c['top_fraction']}, sink/recent "
        f"{c['sink']}/{c['recent']}, capacity {cap}")
    # the lagged modes (lagtop2 / lagrefresh{N} / qdrift* / pconf{T}) run their own step
    lagged = RU.is_lagged_mode(c["mode"])
    step_cls = RU.LaggedReuseDecodeStep if lagged else RU.ReuseDecodeStep
    g = torch.Generator(device="cuda").manual_seed(0)
    ks, vs, qs, steps = [], [], [], []
    for layer in range(layers):
        k = torch.randn((b, hkv, cap, d), generator=g, device="cuda").to(torch.bfloat16)
        v = torch.randn((b, hkv, cap, d), generator=g, device="cuda").to(torch.bfloat16)
        q = torch.randn((b, hq, d), generator=g, device="cuda").to(torch.bfloat16)
        st = step_cls(c["mode"], b, hq, hkv, d, cap, top_fraction=c["top_fraction"],
                      protect_sink=c["sink"], protect_recent=c["recent"], candidate_selection=selection)
        st.prefill(k[:, :, :t0])
        ks.append(k)
        vs.append(v)
        qs.append(q)
        steps.append(st)
    torch.cuda.synchronize()
    log(f"[bench] resident: {torch.cuda.memory_allocated() / 2**30:.1f} GiB")

    hist = t0

    def decode_step():
        nonlocal hist
        for layer in range(layers):
            steps[layer](qs[layer], ks[layer][:, :, : hist + 1], vs[layer][:, :, : hist + 1], scaling)
        hist += 1

    for _ in range(args.warmup):
        decode_step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    h0 = hist
    e0.record()
    for _ in range(args.steps):
        decode_step()
    e1.record()
    torch.cuda.synchronize()
    ms_per_step = e0.elapsed_time(e1) / args.steps
    log(f"[bench] eager step: {ms_per_step:.3f} ms ({ms_per_step * 1e3 / layers:.1f} us/layer), "
        f"history {h0}..{hist - 1}")

    # Union size and final list of the last step (layer 0), for the byte counts.
    st0 = steps[0]
    hist_fixed = hist - 1
    cur, prev, fin = st0.cand[1 - st0.flip], st0.cand[st0.flip], st0.fin
    if lagged:   # the union the lagged step reranked (previous final | candidates | protected ranges)
        union = int((RU.expand_bits(st0.union, hist_fixed) if st0.bits else st0.union[:, :hist_fixed]).count_nonzero())
    elif st0.bits:
        union = int(RU.expand_bits((cur | prev) | fin, hist_fixed).count_nonzero())
    else:
        union = int(((cur[:, :hist_fixed] | prev[:, :hist_fixed]) | fin[:, :hist_fixed]).count_nonzero())
    n_out = st0.n_out
    rows = b * hq

    # One step at a fixed history with steady-state masks, as a graph.
    def fixed(layer):
        st = steps[layer]
        kk, vv = ks[layer][:, :, : hist_fixed + 1], vs[layer][:, :, : hist_fixed + 1]
        return st, kk, vv

    def run_fixed():
        for layer in range(layers):
            st, kk, vv = fixed(layer)
            st.launch(qs[layer], kk, vv, scaling, st.cand[0], st.cand[1], st.fin,
                      previous_thresholds=selection == "previous_threshold")

    reps = max(1, -(-16 // layers))

    def repeated(fn):
        def run():
            for _ in range(reps):
                fn()
        return run

    gr = graph_of(repeated(run_fixed))
    ms_graph = time_replays(gr.replay, args.kernel_reps) / reps
    del gr
    log(f"[bench] graph step (history {hist_fixed}): {ms_graph * 1e3 / layers:.1f} us/layer")

    mask_ws = [steps[l].mask_ws for l in range(layers)]
    if lagged:
        _, _, s_dims, cand_frac = RU.parse_lagged_mode(c["mode"])
        block = None
    else:
        s_dims, cand_frac, _, _, block = RU.parse_reuse_mode(c["mode"])
    requested = RU.budget_count(hist_fixed, cand_frac)

    def run_partial():
        for layer in range(layers):
            RU.reuse_partial_scores(qs[layer], steps[layer].kdm, hist_fixed, s_dims, out=steps[layer].partial)

    n_s = steps[0].columns.count(hist_fixed) if selection == "sample_quantile" else 0
    mask_name, mask_bytes = "threshold_mask", rows * hist_fixed * (4 + 1)

    def run_mask():
        for layer in range(layers):
            RU.candidate_mask(steps[layer].partial, hist_fixed, "topk", requested, steps[layer].cand[0], None,
                              mask_ws[layer])

    if selection == "topk" and not lagged and st0.bits:
        # the step's candidates call: the partial scores with their first-digit
        # counts, then the selection across several workgroups per row
        mask_name = "reuse_candidates"
        mask_bytes = rows * hist_fixed * (s_dims * 2 + 4) + rows * hist_fixed * 4 + rows * hist_fixed // 8

        def run_mask():
            for layer in range(layers):
                st = steps[layer]
                RU._lib.check(lib.qkv_reuse_candidates(
                    qs[layer].data_ptr(), st.kdm.data_ptr(), RU._lib.strides(*st.kdm.stride()), 0, b, hq, hkv,
                    hist_fixed, d, s_dims, requested, st.partial.data_ptr(), st.partial.stride(0), None, 0,
                    st.cand[0].data_ptr(), st.cand[0].stride(0), None, st.cand_ws.data_ptr(), st.cand_ws.numel() * 4,
                    RU._lib.stream_of(qs[layer])))
    elif n_s:   # the sampled columns gathered (index and score), then the mask pass
        mask_name, mask_bytes = "sample_quantile_mask", n_s * 4 + rows * n_s * 8 + rows * hist_fixed * (4 + 1)

        def run_mask():
            k_s = RU.budget_count(n_s, cand_frac)
            for layer in range(layers):
                st = steps[layer]
                RU.candidate_mask(st.partial, hist_fixed, "sample_quantile", k_s, st.cand[0], st.thresholds,
                                  mask_ws[layer], st.columns.row(hist_fixed), n_s)
    elif selection == "previous_threshold":   # the row's threshold, then the mask pass
        mask_name, mask_bytes = "previous_threshold_mask", rows * 4 + rows * hist_fixed * (4 + 1)

        def run_mask():
            for layer in range(layers):
                st = steps[layer]
                RU.candidate_mask(st.partial, hist_fixed, "previous_threshold", requested, st.cand[0], st.thresholds,
                                  mask_ws[layer])

    lib = RU._lib.load()
    n_sel = int(lib.qkv_reuse_final_count(hist_fixed, c["sink"], c["recent"], c["top_fraction"], 1))

    # the selection writes its final mask elsewhere, so that every timed launch
    # reads the previous final (block-expanded in the blk modes) the step reads
    fin_out = [torch.empty_like(steps[l].fin) for l in range(layers)]

    fused_expand = block is not None and st0.bits   # the block expansion inside the selection's launch

    def run_select():
        for layer in range(layers):
            st, kk, _ = fixed(layer)
            if fused_expand:
                RU._lib.check(lib.qkv_reuse_select_bits_blocks(
                    qs[layer].data_ptr(), kk.data_ptr(), RU._lib.strides(*kk.stride()), 0, b, hq, hkv,
                    hist_fixed + 1, d, st.cand[0].data_ptr(), st.cand[1].data_ptr(), st.fin.data_ptr(),
                    st.fin.stride(0), c["sink"], c["recent"], c["top_fraction"], 1, scaling, block,
                    st.select_ws.data_ptr(), st.select_ws.numel() * 4, st.final_idx.data_ptr(),
                    st.final_valid.data_ptr(), st.attn_ids.data_ptr(), n_out, fin_out[layer].data_ptr(),
                    fin_out[layer].stride(0), RU._lib.stream_of(qs[layer])))
                continue
            select = lib.qkv_reuse_select_bits if st.bits else lib.qkv_reuse_select
            extra = (None, None, None) if st.bits else ()   # the selection alone (no fused attention)
            RU._lib.check(select(
                qs[layer].data_ptr(), kk.data_ptr(), RU._lib.strides(*kk.stride()), 0, b, hq, hkv, hist_fixed + 1, d,
                st.cand[0].data_ptr(), st.cand[1].data_ptr(), st.fin.data_ptr(), st.fin.stride(0), c["sink"],
                c["recent"], c["top_fraction"], 1, scaling, st.select_ws.data_ptr(), st.select_ws.numel() * 4,
                st.final_idx.data_ptr(), st.final_valid.data_ptr(), st.attn_ids.data_ptr(), n_sel,
                fin_out[layer].data_ptr(), fin_out[layer].stride(0), *extra, RU._lib.stream_of(qs[layer])))

    def run_expand():
        for layer in range(layers):
            st = steps[layer]
            RU._lib.check(lib.qkv_reuse_expand_blocks(
                st.fin.data_ptr(), cap, rows, hist_fixed + 1, block, c["sink"], c["recent"], c["top_fraction"], 1,
                st.final_idx.data_ptr(), st.final_valid.data_ptr(), st.attn_ids.data_ptr(), n_out,
                RU._lib.stream_of(qs[layer])))

    def run_attn():
        for layer in range(layers):
            st, kk, vv = fixed(layer)
            RU.token_attention(qs[layer], kk, vv, st.attn_ids[: rows * n_out].view(rows, n_out), scaling,
                               workspace=st.attn_ws, out=st.out)

    plan = [
        ("reuse_partial_scores", run_partial, rows * hist_fixed * (s_dims * 2 + 4)),
        (mask_name, run_mask, mask_bytes),
        # three mask bytes, the f32 score and the final mask byte per token, plus
        # the K row of every union token
        ("reuse_select", run_select, rows * hist_fixed * (3 + 4 + 1) + union * d * 2),
        ("token_attention", run_attn, rows * n_out * d * 2 * 2),
    ]
    if st0.bits:   # mask bits in words (and, with blocks, the expansion in the same launch)
        plan[2] = ("reuse_select_expand" if fused_expand else "reuse_select", run_select,
                   rows * hist_fixed * 4 + rows * hist_fixed // 2 + union * d * 2)
    elif block is not None:   # one byte read and one written per history position
        plan.insert(3, ("reuse_expand_blocks", run_expand, rows * hist_fixed * 2))
    if lagged:
        test = RU.LAGGED_KINDS[st0.kind][0]
        refresh = st0.refresh_of(hist_fixed, True)
        share = st0.kind == "qdriftshare"

        def run_flags():
            for layer in range(layers):
                st, kk, _ = fixed(layer)
                RU.lag_flags(qs[layer], hkv, test, s_dims, st.qdims[st.flip], st.qvals[st.flip], st.flags,
                             previous_dims=st.qdims[1 - st.flip], previous_values=st.qvals[1 - st.flip], key=kk,
                             history=hist_fixed, previous_final=st.fin, scaling=scaling,
                             ess_threshold=float(st.param) if st.kind == "pconf" else 0.0,
                             workspace=st.ess_ws if test == "ess" else None)

        def run_union():
            for layer in range(layers):
                st = steps[layer]
                RU.lag_union(st.cand[0], st.fin, st.flags, b, hq, hist_fixed, refresh, share, c["sink"], c["recent"],
                             st.union)

        # candidates and previous final read, union written per position (bits or bytes)
        plan.insert(2, ("lag_union", run_union, rows * hist_fixed * 3 // (8 if st0.bits else 1)))
        if test is not None:   # ess: the mask row, then the K row of every previous final token
            fin_tokens = int((RU.expand_bits(st0.fin, hist_fixed) if st0.bits else st0.fin[:, :hist_fixed])
                             .count_nonzero())
            plan.insert(0, ("lag_flags", run_flags,
                            rows * hist_fixed // (8 if st0.bits else 1) + fin_tokens * d * 2 if test == "ess"
                            else rows * (d * 2 + s_dims * 16)))
        # partial scores and candidate mask of the rows that refresh only
        flagged = int(st0.flags.count_nonzero())
        n_fresh = {"none": 0, "all": rows, "per_row": flagged, "any": rows if flagged else 0,
                   "majority": rows if 2 * flagged > rows else 0}[refresh]

        def run_cands():
            for layer in range(layers):
                st = steps[layer]
                RU.lag_candidates(qs[layer], st.kdm, hist_fixed, s_dims, requested, st.flags, refresh, st.partial,
                                  st.cand[0], st.cand_ws if st.bits else mask_ws[layer])

        plan = [p for p in plan if p[0] not in ("reuse_partial_scores", mask_name)]
        if refresh != "none":
            plan.insert(1 if test is not None else 0,
                        ("lag_candidates", run_cands, n_fresh * hist_fixed * (s_dims * 2 + 4 + 4) +
                         n_fresh * hist_fixed // (8 if st0.bits else 1)))
    kernels = {}
    for name, fn, nbytes in plan:
        gk = graph_of(repeated(fn))
        ms = time_replays(gk.replay, args.kernel_reps) / (layers * reps)
        kernels[name] = {"us_per_launch": ms * 1e3, "bytes_per_launch": nbytes, "gbs": nbytes / (ms * 1e-3) / 1e9,
                         "frac_hbm_peak": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
        log(f"[bench] {name}: {ms * 1e3:.2f} us/launch, {kernels[name]['gbs']:.0f} GB/s")
        del gk
    for _ in range(args.profile_steps):
        run_fixed()
    torch.cuda.synchronize()

    cpu = None
    if lagged:   # the CPU leg restates the default reuse mode's op sequence only
        log("[bench] cpu baseline: not measured for the lagged modes")
    elif not args.no_cpu_baseline:
        log("[bench] cpu baseline ...")
        cpu = cpu_baseline_reuse(args.cpu_seconds)
        log(f"[bench] cpu baseline: {cpu['value']:.3e} keys/s on {cpu['cores']} cores")
    dom = max(kernels, key=lambda n: kernels[n]["us_per_launch"])
    keys_per_layer = b * hkv * hist_fixed
    return {
        "metric": "reuse decode: keys/s (history tokens x KV heads) through the qabs reuse step; us/layer",
        "value": layers * keys_per_layer / (ms_per_step * 1e-3),
        "unit": "keys/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 -> f32 scores and attention",
        "data": "synthetic (seeded N(0,1) K/V/q)",
        "config": {"workload": f"reuse: {c['name']}", "batch": b, "q_heads": hq, "kv_heads": hkv, "head_dim": d,
                   "history": t0, "layers": layers, "mode": c["mode"], "candidate_selection": selection,
                   "top_fraction": c["top_fraction"], "sink": c["sink"], "recent": c["recent"], "graph": False,
                   **({"refresh": st0.refresh_of(hist_fixed, True),
                       "flagged_rows": int(st0.flags.count_nonzero())} if lagged else {})},
        "us_per_layer": ms_per_step * 1e3 / layers,
        "graph_us_per_layer": None if ms_graph is None else ms_graph * 1e3 / layers,
        "union_tokens_per_row": union / rows,
        "final_entries_per_row": n_out,
        "roofline": {
            "bound": "hbm", "kernel": dom, "achieved": kernels[dom]["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": kernels[dom]["gbs"] / HBM_PEAK_GBS, "traffic": read_traffic("reuse", dom),
        },
        "kernels": kernels,
        "cpu_baseline": cpu,
    }


def cpu_baseline_qabs_attn(mode: str, budget_s: float) -> dict:
    """The reference's qabs{S}cand{pct}attn op sequence (oracle/ref_semantics.py
    qabs_candidate_attention_cpu, pinned to the reference's vectors) for one
    layer of the REUSE shape, repeated for about ``budget_s`` seconds."""
    import torch

    from kv_cache_amd.reuse import parse_qabs_attn_mode
    from oracle import ref_semantics as R

    c = REUSE
    dims, frac, _, _ = parse_qabs_attn_mode(mode)
    torch.set_num_threads(host_threads())
    g = torch.Generator().manual_seed(0)
    t = c["history"] + 1
    k = torch.randn((1, c["kv_heads"], t, c["head_dim"]), generator=g).to(torch.bfloat16)
    v = torch.randn((1, c["kv_heads"], t, c["head_dim"]), generator=g).to(torch.bfloat16)
    q = torch.randn((1, c["q_heads"], 1, c["head_dim"]), generator=g).to(torch.bfloat16)
    run = lambda: R.qabs_candidate_attention_cpu(q, k, v, dims, frac, c["head_dim"] ** -0.5,  # noqa: E731
                                                 c["sink"], c["recent"], True)
    run()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 100):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    keys = c["kv_heads"] * c["history"]
    return {
        "value": keys / med,
        "unit": "keys/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"one layer ({mode}, {c['q_heads']}/{c['kv_heads']} heads, history {c['history']}): the "
                   f"reference's candidate-attention op sequence on CPU tensors; median of {len(times)} calls = "
                   f"{med * 1e3:.1f} ms; {host_note(torch.get_num_threads())}"),
    }


def time_dropin_calls(args, step, q, k, v, hist: int, dims: int, n_out: int, scaling: float, reps: int) -> dict:
    """The two reference-signature calls the reference's timed qabs{S}cand{pct}attn
    mode makes (qabs_cuda_kernels.partial_scores_dim_major, QK:659-665, and
    final_attention, QK:694-705) on one layer of the same workload, with their
    inputs as the reference builds them: K/V and the dim-major copy expanded to
    the query heads (EV:6248-6251), int64 top-|q| dims and the step's final
    index list."""
    import torch

    from kv_cache_amd import qabs_cuda_kernels as Q

    b, hq, d = q.shape
    g = hq // k.size(1)
    kdm = step.kdm[..., :hist].repeat_interleave(g, dim=1).contiguous()        # [B, Hq, D, hist]
    kx = k[:, :, : hist + 1].repeat_interleave(g, dim=1).contiguous()          # [B, Hq, T, D]
    vx = v[:, :, : hist + 1].repeat_interleave(g, dim=1).contiguous()
    dim_idx = torch.topk(q.float().abs(), k=dims, dim=-1).indices                # int64 [B, Hq, S]
    rows = b * hq
    idx = step.final_idx[: rows * n_out].view(b, hq, n_out)
    valid = step.final_valid[: rows * n_out].view(b, hq, n_out)
    out = {}
    plan = [("dropin_partial_scores_dim_major", lambda: Q.partial_scores_dim_major(q, kdm, dim_idx),
             rows * hist * (dims * 2 + 4)),
            ("dropin_final_attention", lambda: Q.final_attention(q, kx, vx, idx, valid, scaling),
             rows * n_out * (d * 2 * 2 + 9))]
    for name, fn, nbytes in plan:
        def run():
            for _ in range(reps):
                fn()
        gk = graph_of(run)
        ms = time_replays(gk.replay, args.kernel_reps) / reps
        out[name] = {"us_per_launch": ms * 1e3, "bytes_per_launch": nbytes, "gbs": nbytes / (ms * 1e-3) / 1e9,
                     "frac_hbm_peak": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
        log(f"[bench] {name}: {ms * 1e3:.2f} us/launch, {out[name]['gbs']:.0f} GB/s")
        del gk
    del kdm, kx, vx
    return out


def run_qabs_attn(args) -> dict:
    """Decode steps of the exact qabs{S}cand{pct}[append]attn mode
    (kv_cache_amd.reuse.QabsCandidateAttentionStep) on the REUSE shape: eager
    steps with a growing history, one fixed-history step as a HIP graph, and
    each kernel alone."""
    import torch

    from kv_cache_amd import reuse as RU

    c = REUSE
    mode = args.qabs_mode
    dims, frac, append, interval = RU.parse_qabs_attn_mode(mode)
    layers = args.layers or 8
    b, hq, hkv, d, t0 = c["batch"], c["q_heads"], c["kv_heads"], c["head_dim"], c["history"]
    cap = -(-(t0 + args.warmup + args.steps + 2) // 64) * 64
    scaling = d ** -0.5
    log(f"[bench] setup qabsattn {mode}: {layers} layers, {hq}/{hkv} heads, history {t0}, sink/recent "
        f"{c['sink']}/{c['recent']}, capacity {cap}")
    g = torch.Generator(device="cuda").manual_seed(0)
    ks, vs, qs, steps = [], [], [], []
    for _ in range(layers):
        k = torch.randn((b, hkv, cap, d), generator=g, device="cuda").to(torch.bfloat16)
        v = torch.randn((b, hkv, cap, d), generator=g, device="cuda").to(torch.bfloat16)
        q = torch.randn((b, hq, d), generator=g, device="cuda").to(torch.bfloat16)
        st = RU.QabsCandidateAttentionStep(mode, b, hq, hkv, d, cap, protect_sink=c["sink"],
                                           protect_recent=c["recent"])
        st.prefill(k[:, :, :t0])
        ks.append(k)
        vs.append(v)
        qs.append(q)
        steps.append(st)
    torch.cuda.synchronize()
    hist = t0

    def decode_step():
        nonlocal hist
        for layer in range(layers):
            steps[layer](qs[layer], ks[layer][:, :, : hist + 1], vs[layer][:, :, : hist + 1], scaling)
        hist += 1

    for _ in range(args.warmup):
        decode_step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    h0 = hist
    e0.record()
    for _ in range(args.steps):
        decode_step()
    e1.record()
    torch.cuda.synchronize()
    ms_per_step = e0.elapsed_time(e1) / args.steps
    log(f"[bench] eager step: {ms_per_step:.3f} ms ({ms_per_step * 1e3 / layers:.1f} us/layer), "
        f"history {h0}..{hist - 1}")
    hf = hist - 1
    rows = b * hq
    for layer in range(layers):   # (r{N}attn steps between refreshes leave the copy behind)
        st = steps[layer]
        if st.kdm_len < hf:
            RU.dim_major_append(ks[layer][:, :, : hf + 1], st.kdm, st.kdm_len, hf)
            st.kdm_len = hf
    lib = RU._lib.load()
    n_out = int(lib.qkv_reuse_final_count(hf, c["sink"], c["recent"], frac, 1))
    reps = max(1, -(-16 // layers))

    def repeated(fn):
        def run():
            for _ in range(reps):
                fn()
        return run

    def run_fixed():
        for layer in range(layers):
            steps[layer].launch(qs[layer], ks[layer][:, :, : hf + 1], vs[layer][:, :, : hf + 1], scaling)

    gr = graph_of(repeated(run_fixed))
    ms_graph = time_replays(gr.replay, args.kernel_reps) / reps
    del gr
    log(f"[bench] graph step (history {hf}): {ms_graph * 1e3 / layers:.1f} us/layer")
    ms_graph_reuse = None
    if interval is not None:   # r{N}attn: a step between refreshes rebuilds the list from the kept selection
        def run_fixed_reuse():
            for layer in range(layers):
                steps[layer].launch(qs[layer], ks[layer][:, :, : hf + 1], vs[layer][:, :, : hf + 1], scaling,
                                    reuse_selection=True)

        gr = graph_of(repeated(run_fixed_reuse))
        ms_graph_reuse = time_replays(gr.replay, args.kernel_reps) / reps
        del gr
        log(f"[bench] graph step between refreshes: {ms_graph_reuse * 1e3 / layers:.1f} us/layer")

    def run_partial():
        for layer in range(layers):
            RU.reuse_partial_scores(qs[layer], steps[layer].kdm, hf, dims, out=steps[layer].partial)

    lib = RU._lib.load()
    need = int(lib.qkv_qabs_candidate_select_workspace_bytes(rows, hf, frac))
    select_ws = torch.empty(max(1, (need + 3) // 4), device="cuda") if need > 0 else None

    def run_select():
        for layer in range(layers):
            st = steps[layer]
            out = (st.final_idx[: rows * n_out].view(rows, n_out), st.final_valid[: rows * n_out].view(rows, n_out),
                   st.attn_ids[: rows * n_out].view(rows, n_out), st.hf)
            RU.qabs_candidate_select(st.partial, hf + 1, frac, c["sink"], c["recent"], True, append,
                                     workspace=select_ws, out=out)

    def run_candidates():   # the step's own call: partial scores and the selection across workgroups
        for layer in range(layers):
            st = steps[layer]
            q = qs[layer]
            RU._lib.check(lib.qkv_qabs_candidates(
                q.data_ptr(), st.kdm.data_ptr(), RU._lib.strides(*st.kdm.stride()), 0, b, hq, hkv, hf + 1, d, dims,
                frac, c["sink"], c["recent"], 1, int(append), st.partial.data_ptr(), st.partial.stride(0),
                st.sel_ws.data_ptr(), st.sel_ws.numel() * 4, st.final_idx.data_ptr(), st.final_valid.data_ptr(),
                st.attn_ids.data_ptr(), n_out, st.hf.data_ptr(), st.hf.stride(0), RU._lib.stream_of(q)))

    def run_attn():
        for layer in range(layers):
            st = steps[layer]
            RU.token_attention(qs[layer], ks[layer][:, :, : hf + 1], vs[layer][:, :, : hf + 1],
                               st.attn_ids[: rows * n_out].view(rows, n_out), scaling, workspace=st.attn_ws,
                               out=st.out)

    plan = [
        ("reuse_partial_scores", run_partial, rows * hf * (dims * 2 + 4)),
        # the scores read, the history mask and the index lists written
        ("qabs_candidate_select", run_select, rows * hf * (4 + 1) + rows * n_out * (8 + 1 + 4)),
        # the partial scores' bytes, the scores read back, the mask and lists written
        ("qabs_candidates", run_candidates,
         rows * hf * (dims * 2 + 4) + rows * hf * (4 + 1) + rows * n_out * (8 + 1 + 4)),
        ("token_attention", run_attn, rows * n_out * d * 2 * 2),
    ]
    kernels = {}
    for name, fn, nbytes in plan:
        gk = graph_of(repeated(fn))
        ms = time_replays(gk.replay, args.kernel_reps) / (layers * reps)
        kernels[name] = {"us_per_launch": ms * 1e3, "bytes_per_launch": nbytes, "gbs": nbytes / (ms * 1e-3) / 1e9,
                         "frac_hbm_peak": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
        log(f"[bench] {name}: {ms * 1e3:.2f} us/launch, {kernels[name]['gbs']:.0f} GB/s")
        del gk
    kernels.update(time_dropin_calls(args, steps[0], qs[0], ks[0], vs[0], hf, dims, n_out, scaling, reps))
    for _ in range(args.profile_steps):
        run_fixed()
    torch.cuda.synchronize()
    cpu = None
    if interval is not None or append:   # the CPU leg restates the plain attn op sequence only
        log("[bench] cpu baseline: not measured for the r{N}attn / appendattn variants")
    elif not args.no_cpu_baseline:
        log("[bench] cpu baseline ...")
        cpu = cpu_baseline_qabs_attn(mode, args.cpu_seconds)
        log(f"[bench] cpu baseline: {cpu['value']:.3e} keys/s on {cpu['cores']} cores")
    dom = max((n for n in kernels if not n.startswith("dropin_")), key=lambda n: kernels[n]["us_per_launch"])
    keys_per_layer = b * hkv * hf
    return {
        "metric": "candidate attention decode: keys/s (history tokens x KV heads) through the exact "
                  "qabs{S}cand{pct}attn step; us/layer",
        "value": layers * keys_per_layer / (ms_per_step * 1e-3),
        "unit": "keys/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 -> f32 scores and attention",
        "data": "synthetic (seeded N(0,1) K/V/q)",
        "config": {"workload": f"qabsattn: {c['name']}", "batch": b, "q_heads": hq, "kv_heads": hkv, "head_dim": d,
                   "history": t0, "layers": layers, "mode": mode, "sink": c["sink"], "recent": c["recent"],
                   "graph": False},
        "us_per_layer": ms_per_step * 1e3 / layers,
        "graph_us_per_layer": ms_graph * 1e3 / layers,
        **({"graph_us_per_layer_between_refreshes": ms_graph_reuse * 1e3 / layers} if interval else {}),
        "final_entries_per_row": n_out,
        "roofline": {
            "bound": "hbm", "kernel": dom, "achieved": kernels[dom]["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": kernels[dom]["gbs"] / HBM_PEAK_GBS, "traffic": read_traffic("qabsattn", dom),
        },
        "kernels": kernels,
        "cpu_baseline": cpu,
    }


# Block-metadata selector workloads (Qwen3-8B heads, one sequence, 32768
# history tokens): the reference's own qbb mode string, and brep at the same
# block size, scan and candidate fractions.
BLOCKSEL = {"qbb": "qbb64q8s3cand3", "brep": "brep64r4q8s3cand3"}


def cpu_baseline_blocksel(mode: str, budget_s: float, steps: int = 3) -> dict:
    """The reference's qbb / brep op sequence (oracle/ref_semantics.py
    block_select_step_cpu) for consecutive decode steps of one layer."""
    import torch

    from kv_cache_amd.blocksel import BREP, parse_block_mode
    from oracle import ref_semantics as R

    c = REUSE
    kind, block, reps, dims, scan, cand = parse_block_mode(mode)
    torch.set_num_threads(host_threads())
    g = torch.Generator().manual_seed(0)
    t = c["history"] + steps + 1
    k = torch.randn((1, c["kv_heads"], t, c["head_dim"]), generator=g).to(torch.bfloat16)
    v = torch.randn((1, c["kv_heads"], t, c["head_dim"]), generator=g).to(torch.bfloat16)
    times = []
    t_end = time.perf_counter() + budget_s
    for s in range(steps):
        n = c["history"] + s + 1
        q = torch.randn((1, c["q_heads"], 1, c["head_dim"]), generator=g).to(torch.bfloat16)
        t0 = time.perf_counter()
        R.block_select_step_cpu(q, k[:, :, :n], v[:, :, :n], "brep" if kind == BREP else "qbb", block, dims, scan,
                                cand, c["top_fraction"], c["head_dim"] ** -0.5, c["sink"], c["recent"], True, reps)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() > t_end:
            break
    med = statistics.median(times[1:] if len(times) > 1 else times)
    keys = c["kv_heads"] * c["history"]
    return {
        "value": keys / med,
        "unit": "keys/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{len(times)} decode steps of one layer ({mode}, {c['q_heads']}/{c['kv_heads']} heads, history "
                   f"{c['history']}): the reference's op sequence on CPU tensors; median of the steps after the "
                   f"first = {med * 1e3:.1f} ms per layer-step"),
    }


def run_blocksel(args) -> dict:
    """Decode steps of a block-metadata selector (kv_cache_amd.blocksel) over
    8 layers with their own K/V, metadata and dim-major copy; the history
    grows one token per step.  Timed eagerly, as a graph of one
    fixed-history step, and per kernel."""
    import torch

    from kv_cache_amd import _lib
    from kv_cache_amd import blocksel as BS
    from kv_cache_amd.int4 import block_topk
    from kv_cache_amd.reuse import token_attention

    c = REUSE
    mode = BLOCKSEL[args.config]
    layers = args.layers or 8
    b, hq, hkv, d, t0 = c["batch"], c["q_heads"], c["kv_heads"], c["head_dim"], c["history"]
    cap = -(-(t0 + args.warmup + args.steps + 2) // 64) * 64
    scaling = d ** -0.5
    log(f"[bench] setup {mode}: {layers} layers, Qwen3-8B heads, history {t0}, top {c['top_fraction']}, "
        f"sink/recent {c['sink']}/{c['recent']}")
    g = torch.Generator(device="cuda").manual_seed(0)
    ks, vs, qs, steps = [], [], [], []
    for _ in range(layers):
        k = torch.randn((b, hkv, cap, d), generator=g, device="cuda").to(torch.bfloat16)
        v = torch.randn((b, hkv, cap, d), generator=g, device="cuda").to(torch.bfloat16)
        st = BS.BlockSelectDecodeStep(mode, b, hq, hkv, d, cap, top_fraction=c["top_fraction"],
                                      protect_sink=c["sink"], protect_recent=c["recent"])
        st.prefill(k[:, :, :t0])
        ks.append(k)
        vs.append(v)
        qs.append(torch.randn((b, hq, d), generator=g, device="cuda").to(torch.bfloat16))
        steps.append(st)
    torch.cuda.synchronize()
    hist = t0

    def decode_step():
        nonlocal hist
        for layer in range(layers):
            steps[layer](qs[layer], ks[layer][:, :, : hist + 1], vs[layer][:, :, : hist + 1], scaling)
        hist += 1

    for _ in range(args.warmup):
        decode_step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        decode_step()
    e1.record()
    torch.cuda.synchronize()
    ms_per_step = e0.elapsed_time(e1) / args.steps
    log(f"[bench] eager step: {ms_per_step:.3f} ms ({ms_per_step * 1e3 / layers:.1f} us/layer)")

    hf = hist - 1
    kc = hf + 1
    nb, n_scan, n_cand, n_keep = BS.step_counts(hf, steps[0].block, steps[0].scan, steps[0].cand, c["top_fraction"],
                                                steps[0].unscanned)
    lib = _lib.load()
    reps = max(1, -(-16 // layers))

    def repeated(fn):
        def run():
            for _ in range(reps):
                fn()
        return run

    def run_fixed():
        for layer in range(layers):
            steps[layer].launch(qs[layer], ks[layer][:, :, :kc], vs[layer][:, :, :kc], scaling)

    gr = graph_of(repeated(run_fixed))
    ms_graph = time_replays(gr.replay, args.kernel_reps) / reps
    del gr
    log(f"[bench] graph step (history {hf}): {ms_graph * 1e3 / layers:.1f} us/layer")
    rows = b * hq
    n_tok = n_scan * steps[0].block
    n_out = steps[0].n_out

    def run_scores():
        for layer in range(layers):
            st, k = steps[layer], ks[layer][:, :, :kc]
            _lib.check(lib.qkv_block_scores(st.kind, qs[layer].data_ptr(), k.data_ptr(), _lib.strides(*k.stride()),
                                            st.meta.data_ptr(), st.meta_blocks, b, hq, hkv, hf, d, st.block,
                                            st.reps, st.dims, st.bscore.data_ptr(), st.meta_blocks,
                                            st.dtype_code, _lib.stream_of(k)))

    def run_topk():
        for layer in range(layers):
            st = steps[layer]
            block_topk(st.bscore[:, :nb], n_scan, out=st.blocks[: rows * n_scan].view(rows, n_scan),
                       workspace=st.topk_ws)

    def run_scan():
        for layer in range(layers):
            st = steps[layer]
            k = ks[layer][:, :, :kc]
            _lib.check(lib.qkv_block_scan_scores(qs[layer].data_ptr(), st.kdm.data_ptr(),
                                                 _lib.strides(*st.kdm.stride()), k.data_ptr(),
                                                 _lib.strides(*k.stride()), b, hq, hkv, hf, d,
                                                 st.blocks.data_ptr(), n_scan, st.block, st.dims, scaling,
                                                 st.partial.data_ptr(), st.full.data_ptr(), n_tok,
                                                 st.dtype_code, _lib.stream_of(qs[layer])))

    def run_rerank():
        for layer in range(layers):
            st, k = steps[layer], ks[layer][:, :, :kc]
            _lib.check(lib.qkv_block_rerank(qs[layer].data_ptr(), k.data_ptr(), _lib.strides(*k.stride()), b, hq, hkv,
                                            kc, d, st.partial.data_ptr(), st.full.data_ptr(), n_tok,
                                            st.blocks.data_ptr(), n_scan,
                                            st.block, n_cand, n_keep, c["sink"], c["recent"], 1, scaling,
                                            st.keep.data_ptr(), st.capacity, st.attn_ids.data_ptr(), n_out,
                                            int(st.unscanned), st.rerank_ws.data_ptr(), st.rerank_ws.numel() * 4,
                                            st.dtype_code, _lib.stream_of(k)))

    def run_attn():
        for layer in range(layers):
            st = steps[layer]
            token_attention(qs[layer], ks[layer][:, :, :kc], vs[layer][:, :, :kc],
                            st.attn_ids[: rows * n_out].view(rows, n_out), scaling, workspace=st.attn_ws, out=st.out)

    meta_bytes = {BS.QBB: 2 * 2 * d, BS.BREP: 4 * steps[0].reps}[steps[0].kind]   # per block, per KV head
    plan = [
        # a block's metadata record per query head, plus the f32 score written
        ("block_scores", run_scores, rows * nb * (meta_bytes + 4)),
        ("block_topk", run_topk, rows * nb * 4),
        # every scanned token's S dims (dim-major) and bf16 K row, its f32 partial and full scores
        ("scan_partial", run_scan, rows * n_tok * (steps[0].dims * 2 + d * 2 + 8)),
        # partial scores read once, the candidates' full scores, the final mask bytes
        ("rerank", run_rerank, rows * (n_tok * 4 + n_cand * 4 + kc)),
        ("token_attention", run_attn, rows * n_out * d * 2 * 2),
    ]
    kernels = {}
    for name, fn, nbytes in plan:
        gk = graph_of(repeated(fn))
        ms = time_replays(gk.replay, args.kernel_reps) / (layers * reps)
        kernels[name] = {"us_per_launch": ms * 1e3, "bytes_per_launch": nbytes, "gbs": nbytes / (ms * 1e-3) / 1e9,
                         "frac_hbm_peak": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
        log(f"[bench] {name}: {ms * 1e3:.2f} us/launch, {kernels[name]['gbs']:.0f} GB/s")
        del gk
    for _ in range(args.profile_steps):
        run_fixed()
    torch.cuda.synchronize()
    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline ...")
        cpu = cpu_baseline_blocksel(mode, args.cpu_seconds)
        log(f"[bench] cpu baseline: {cpu['value']:.3e} keys/s on {cpu['cores']} cores")
    dom = max(kernels, key=lambda n: kernels[n]["us_per_launch"])
    return {
        "metric": f"{mode} decode: keys/s (history tokens x KV heads) through the block selector step; us/layer",
        "value": layers * b * hkv * hf / (ms_per_step * 1e-3),
        "unit": "keys/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 -> f32 scores and attention",
        "data": "synthetic (seeded N(0,1) K/V/q)",
        "config": {"workload": f"{args.config}: {mode}, Qwen3-8B heads, history {t0}", "batch": b, "q_heads": hq,
                   "kv_heads": hkv, "head_dim": d, "history": t0, "layers": layers, "mode": mode,
                   "top_fraction": c["top_fraction"], "sink": c["sink"], "recent": c["recent"], "graph": False,
                   "scanned_tokens": n_tok, "candidates": n_cand, "kept": n_keep},
        "us_per_layer": ms_per_step * 1e3 / layers,
        "graph_us_per_layer": ms_graph * 1e3 / layers,
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": kernels[dom]["gbs"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": kernels[dom]["gbs"] / HBM_PEAK_GBS,
                     "traffic": read_traffic(args.config, dom)},
        "kernels": kernels,
        "cpu_baseline": cpu,
    }


if __name__ == "__main__":
    sys.exit(main())
