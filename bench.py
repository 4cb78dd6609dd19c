#!/usr/bin/env python3
"""bench.py — one MI355X, the TurboCAG KV-compression hot path.

A step is one decode-time pass over a 36-layer Qwen2.5-3B-shaped compressed
KV cache at 32K context (BASELINE configs 3 and 4): for every layer, dequant
of its turbo_prod page pool to fp16 K/V [32768, 2, 128] (config 3's work,
inputs resident in HBM) and fused GQA 16/2 decode attention over the same
pool (config 4).  The 36 distinct pools (316 MB) and fp16 outputs (2.4 GB)
rotate through more than the 256 MB Infinity Cache.

value = algorithmic bytes of the step / step time (GB/s).  roofline is the
dominant kernel (dequant): its algorithmic bytes per launch over its average
launch duration, from per-launch HIP events on the launch stream.
cpu_baseline times the CPU oracle (a port of the reference's algorithm) on a
bounded sample of the same work on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "dequant+attn GB/s & %HBM peak; decode-attn µs/layer @32K ctx, 1 MI355X"
HBM_PEAK_GBPS = 8000.0


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def gpu_kv(N, H, D, seed, dev):
    """Seeded N(0,1) K/V with the synthetic outlier channels, made on the GPU."""
    import torch
    from turborag_amd.synthetic import OUTLIER_SCALE, outlier_channels
    g = torch.Generator(device=dev).manual_seed(seed)
    k = torch.randn(N, H, D, generator=g, device=dev)
    v = torch.randn(N, H, D, generator=g, device=dev)
    for h, ch in enumerate(outlier_channels(H, D)):
        k[:, h, ch] *= OUTLIER_SCALE
        v[:, h, ch] *= OUTLIER_SCALE
    return k.half(), v.half()


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--tokens", type=int, default=32768)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the path has no cross-GPU "
              "exchange; see DESIGN.md on sharding) — run with --gpus 1", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from turborag_amd.synthetic import gqa_rows, permuted_slots, query
    from turborag_amd.turboquant_wrapper import TurboQuantWrapper

    dev = torch.device("cuda", 0)
    tq = TurboQuantWrapper()
    H, D, B, N, NL = 2, 128, 16, args.tokens, args.layers
    Q_HEADS = 16
    rows = Q_HEADS // H
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim, cfg.block_size = H, D, B
    lp = tq.make_layout_for(cfg)
    pages = (N + B - 1) // B

    log(f"[bench] setup: {NL} layers x {N} tokens, packing on the GPU")
    slots = permuted_slots(N, B, seed=401).to(dev)
    pools = []
    for layer in range(NL):
        k, v = gpu_kv(N, H, D, 300 + layer, dev)
        pool = torch.zeros(pages * lp.page_size_bytes, dtype=torch.uint8, device=dev)
        tq.pack(k, v, slots, pool, lp, cfg)
        pools.append(pool)
    del k, v
    out_k = [torch.empty(N, H, D, dtype=torch.float16, device=dev) for _ in range(NL)]
    out_v = [torch.empty(N, H, D, dtype=torch.float16, device=dev) for _ in range(NL)]
    qa = gqa_rows(query(Q_HEADS, D, seed=400), H).to(dev)
    att = [torch.empty(rows, H, D, dtype=torch.float16, device=dev) for _ in range(NL)]
    torch.cuda.synchronize()

    def dequant(layer):
        tq.dequant(pools[layer], slots, out_k[layer], out_v[layer], lp, cfg,
                   stream=torch.cuda.current_stream().cuda_stream)

    def attention(layer):
        tq.fused_attn_output(qa, pools[layer], slots, att[layer], lp, cfg, rows, N,
                             stream=torch.cuda.current_stream().cuda_stream)

    def step():
        for layer in range(NL):
            dequant(layer)
        for layer in range(NL):
            attention(layer)

    # Algorithmic bytes: pages read + fp16 written + slot map.
    pool_bytes = pages * lp.page_size_bytes
    slot_bytes = N * 4
    deq_bytes = pool_bytes + 2 * N * H * D * 2 + slot_bytes
    att_bytes = pool_bytes + slot_bytes + 2 * rows * H * D * 2
    step_bytes = NL * (deq_bytes + att_bytes)

    # Whole step, replayed from a HIP graph so host launch cost is not timed.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()  # sizes this stream's split-K workspace before capture
    torch.cuda.synchronize()
    use_graph = not args.no_graph
    graph = None
    if use_graph:
        try:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=side):
                step()
            torch.cuda.synchronize()
        except Exception as e:  # fall back to eager launches
            log(f"[bench] graph capture failed ({e}); timing eager launches")
            graph, use_graph = None, False

    run = graph.replay if graph is not None else step
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps
    log(f"[bench] step {ms_per_step:.3f} ms ({'graph' if use_graph else 'eager'})")

    # Per-launch durations from HIP events bracketing each launch on its stream.
    def per_launch_us(fn, reps=3):
        evs = []
        for _ in range(reps):
            for layer in range(NL):
                a = torch.cuda.Event(enable_timing=True)
                b = torch.cuda.Event(enable_timing=True)
                a.record()
                fn(layer)
                b.record()
                evs.append((a, b))
        torch.cuda.synchronize()
        return statistics.mean(a.elapsed_time(b) * 1e3 for a, b in evs)

    deq_us = per_launch_us(dequant)
    att_us = per_launch_us(attention)
    deq_gbps = deq_bytes / (deq_us * 1e-6) / 1e9
    att_gbps = att_bytes / (att_us * 1e-6) / 1e9
    log(f"[bench] dequant {deq_us:.2f} us/layer {deq_gbps:.0f} GB/s; "
        f"attention {att_us:.2f} us/layer {att_gbps:.0f} GB/s")

    traffic = None
    tf = ROOT / "profiles" / "traffic.json"
    if tf.exists():
        try:
            traffic = json.loads(tf.read_text()).get("dequant_turbo_prod_32k", {}).get("bytes")
        except Exception:
            traffic = None

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(tq, pools[0], slots, qa, N, H, D, B, deq_bytes, att_bytes, rows)

    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {
            "workload": "C3+C4: per layer, turbo_prod dequant [32768,2,128] + GQA 16/2 decode "
                        "attention @32K, 36 layers, shuffled 16-token pages",
            "layers": NL, "tokens": N, "kv_heads": H, "q_heads": Q_HEADS, "head_dim": D,
            "page_tokens": B, "scheme": "turbo_prod", "graph_replay": use_graph,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "turbo_prod dequant (one layer)",
            "achieved": round(deq_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(deq_gbps / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "algorithmic_bytes": deq_bytes,
            "avg_launch_us": round(deq_us, 3),
        },
        "decode_attn": {
            "us_per_layer": round(att_us, 3),
            "achieved_GBps": round(att_gbps, 1),
            "frac_hbm": round(att_gbps / HBM_PEAK_GBPS, 4),
            "algorithmic_bytes": att_bytes,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def cpu_baseline(tq, pool, slots, qa, N, H, D, B, deq_bytes, att_bytes, rows):
    """The oracle (a C port of the reference's dequant and of its attention
    kernel's fp32 algorithm) on this host's cores, one layer of each."""
    import numpy as np

    from oracle.oracle import load
    from turborag_amd.synthetic import as_u16
    orc = load()
    cores = max(1, min(16, os.cpu_count() or 1))
    orc.nthreads = cores
    pool_np = pool.cpu().numpy()
    slots_np = slots.cpu().numpy()
    q_np = as_u16(qa)
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 and (time.perf_counter() - t_start) < 20:
        t0 = time.perf_counter()
        orc.prod_dequant(pool_np, slots_np, H, D, B)
        t1 = time.perf_counter()
        orc.prod_attention_f32(q_np, pool_np, slots_np, B)
        t2 = time.perf_counter()
        times.append((t1 - t0, t2 - t1))
    td = statistics.median(t[0] for t in times)
    ta = statistics.median(t[1] for t in times)
    log(f"[bench] cpu oracle ({cores} threads): dequant {td*1e3:.1f} ms, attention {ta*1e3:.1f} ms")
    return {
        "value": round((deq_bytes + att_bytes) / (td + ta) / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"one layer: turbo_prod dequant of {N} tokens x {H} heads + the reference "
                  f"kernel's fp32 attention algorithm for {rows} GQA rows x {H} heads over "
                  f"{N} tokens; median of {len(times)} runs",
        "dequant_ms": round(td * 1e3, 2),
        "attention_ms": round(ta * 1e3, 2),
    }


if __name__ == "__main__":
    sys.exit(main())
