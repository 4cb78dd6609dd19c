#!/usr/bin/env python3
"""bench.py — one MI355X, the TurboCAG KV-compression hot path.

A step is one decode-time pass over a 36-layer Qwen2.5-3B-shaped compressed
KV cache at 32K context: for every layer, dequant of its turbo_prod page pool
to fp16 K/V [32768, 2, 128] (the layer load that feeds the model's KV cache,
inputs resident in HBM) and fused GQA 16/2 decode attention over the same
pool.  The step runs on one stream: the one-launch dequant of the 36 layers
(tq_launch_turbo_prod_dequant_kv_layers), then the 36 attention launches.
The 36 distinct pools (316 MB) and fp16 outputs (2.4 GB) rotate through more
than the 256 MB Infinity Cache.  Launches are replayed from HIP graphs, so
host launch cost is not timed.

value = algorithmic bytes of the step / step time (GB/s).  roofline is the
step's dominant kernel, that one-launch dequant: its algorithmic bytes per
launch over its average launch duration, measured with HIP events around
replays of a graph of four such launches, on the stream the graph runs on.
The per-layer dequant launches (the reference's form), and the step with
those beside the attention chain on a second stream, are second figures.
cpu_baseline times the CPU oracle (a C port of the reference's algorithm) on
a bounded sample of the same work on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
       python bench.py --launch-pass   (eager launches only, for rocprofv3)
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


# The dominant kernel (the roofline's) and the decode-attention kernels, as
# rocprofv3 names them (template argument 1 = turbo_prod).
DEQUANT_KERNEL = "tq::dequant_rows_kernel<1, 64, 128>"       # the 36-layer launch
DEQUANT_KERNEL_1 = "tq::dequant_rows_kernel<1, 1, 64>"     # one layer per launch
ATTN_KERNELS = ("tq::dec::attn_decode_split_kernel<1>", "tq::dec::attn_decode_combine_kernel")


def kernel_traffic(name: str):
    """HBM bytes per dispatch of `name` from profiles/traffic.json (calibrated
    FETCH_SIZE + WRITE_SIZE), or None when the summary does not hold it."""
    tf = ROOT / "profiles" / "traffic.json"
    try:
        k = json.loads(tf.read_text())["kernels"][name]
        return {"bytes": int(k["bytes"]), "fetch_B": int(k["fetch_B"]),
                "write_B": int(k["write_B"]), "source": "profiles/traffic.json"}
    except (OSError, ValueError, KeyError, TypeError):
        return None


def gpu_kv(N, H, D, seed, dev):
    """Seeded K/V of the synthetic spec (splitmix64, Box-Muller, outlier
    channels; turborag_amd/synthetic.py), drawn on the host, on the GPU."""
    from turborag_amd.synthetic import kv_tokens_major
    k, v = kv_tokens_major(N, H, D, seed=seed)
    return k.to(dev), v.to(dev)


class Workload:
    """The 36-layer pools, outputs and per-layer launches of one step."""

    def __init__(self, layers: int, tokens: int):
        import torch

        from turborag_amd.synthetic import gqa_rows, permuted_slots, query
        from turborag_amd.turboquant_wrapper import TurboQuantWrapper

        self.dev = dev = torch.device("cuda", 0)
        self.tq = tq = TurboQuantWrapper()
        self.H, self.D, self.B, self.N, self.NL = 2, 128, 16, tokens, layers
        self.q_heads = 16
        self.rows = self.q_heads // self.H
        H, D, B, N, NL = self.H, self.D, self.B, self.N, self.NL
        cfg = tq.default_config()
        cfg.num_kv_heads, cfg.head_dim, cfg.block_size = H, D, B
        self.cfg = cfg
        self.lp = lp = tq.make_layout_for(cfg)
        self.lm = lm = tq.make_mse_layout_for(cfg)
        pages = (N + B - 1) // B

        log(f"[bench] setup: {NL} layers x {N} tokens, packing on the GPU")
        self.slots = permuted_slots(N, B, seed=401).to(dev)
        self.pools = []
        self.mse_pools = []  # the same K/V in turbo_mse pages (config 3's second scheme)
        for layer in range(NL):
            k, v = gpu_kv(N, H, D, 300 + layer, dev)
            pool = torch.zeros(pages * lp.page_size_bytes, dtype=torch.uint8, device=dev)
            tq.pack(k, v, self.slots, pool, lp, cfg)
            self.pools.append(pool)
            pool = torch.zeros(pages * lm.page_size_bytes, dtype=torch.uint8, device=dev)
            tq.mse_pack(k, v, self.slots, pool, lm, cfg)
            self.mse_pools.append(pool)
        del k, v
        self.out_k = [torch.empty(N, H, D, dtype=torch.float16, device=dev) for _ in range(NL)]
        self.out_v = [torch.empty(N, H, D, dtype=torch.float16, device=dev) for _ in range(NL)]
        self.qa = gqa_rows(query(self.q_heads, D, seed=400), H).to(dev)
        self.att = [torch.empty(self.rows, H, D, dtype=torch.float16, device=dev)
                    for _ in range(NL)]
        torch.cuda.synchronize()

        # Algorithmic bytes per layer: pages read + fp16 written + slot map
        # read (dequant); pages + slot map read + query read + output written
        # (attention).
        self.pool_bytes = pages * lp.page_size_bytes
        slot_bytes = N * 4
        self.deq_bytes = self.pool_bytes + 2 * N * H * D * 2 + slot_bytes
        self.att_bytes = self.pool_bytes + slot_bytes + 2 * self.rows * H * D * 2
        self.step_bytes = NL * (self.deq_bytes + self.att_bytes)
        self.side2 = None  # second stream of the step (set by main)

    def _stream(self):
        import torch
        return torch.cuda.current_stream().cuda_stream

    def dequant(self, layer):
        self.tq.dequant(self.pools[layer], self.slots, self.out_k[layer], self.out_v[layer],
                        self.lp, self.cfg, stream=self._stream())

    def attention(self, layer):
        self.tq.fused_attn_output(self.qa, self.pools[layer], self.slots, self.att[layer],
                                  self.lp, self.cfg, self.rows, self.N, stream=self._stream())

    def all_dequant(self):
        """Every layer's dequant in one call (tq_launch_turbo_prod_dequant_kv_layers):
        the document's 36 layers load as one launch."""
        self.tq.dequant_layers("turbo_prod", self.pools, self.slots, self.out_k, self.out_v,
                               self.lp, self.cfg, self.N, stream=self._stream())

    def all_dequant_mse(self):
        """Config 3's turbo_mse pools, every layer in one call."""
        self.tq.dequant_layers("turbo_mse", self.mse_pools, self.slots, self.out_k, self.out_v,
                               self.lm, self.cfg, self.N, stream=self._stream())

    def all_dequant_mse_per_layer(self):
        for layer in range(self.NL):
            self.tq.mse_dequant(self.mse_pools[layer], self.slots, self.out_k[layer],
                                self.out_v[layer], self.lm, self.cfg, stream=self._stream())

    def all_dequant_per_layer(self):
        """The reference's form: one tq_launch_turbo_prod_dequant_kv per layer."""
        for layer in range(self.NL):
            self.dequant(layer)

    def all_attention(self, start: int = 0):
        """Every layer's attention, layers start, start + 1, ... (mod NL)."""
        for k in range(self.NL):
            self.attention((start + k) % self.NL)

    def step(self):
        """One step, on one stream: the one-launch dequant of the 36 layers
        (the roofline kernel), then every layer's attention.  The roofline
        and the step thus time the same dequant launch."""
        self.all_dequant()
        self.all_attention()

    def step_two_streams(self):
        """The step's other form: the 36 per-layer dequant launches on one
        stream and the attention chain on a second stream of the same graph
        (the two share no data; both only read the pools).  Attention
        workgroups fit in between the per-layer dequant grids; beside the
        one-launch dequant they cannot (its queued grid keeps them out), so
        that pairing is slower than running the two one after the other.
        The attention chain starts half the layers away from the dequant
        chain, so the two never read one layer's pages at the same time."""
        import torch
        if self.side2 is None:
            self.step()
            return
        cur = torch.cuda.current_stream()
        self.side2.wait_stream(cur)
        with torch.cuda.stream(self.side2):
            self.all_attention(start=self.NL // 2)
        self.all_dequant_per_layer()
        cur.wait_stream(self.side2)


def capture(fn, side):
    """fn's launches as a HIP graph (captured on the side stream), or None."""
    import torch
    try:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            fn()
        torch.cuda.synchronize()
        return g
    except Exception as e:  # noqa: BLE001 — fall back to eager launches
        log(f"[bench] graph capture failed ({e}); timing eager launches")
        return None


SETTLE_MS = 100.0


def settle(run, ms: float | None = None) -> None:
    """Untimed calls of run() for `ms` of wall time, 16 queued per
    synchronisation.  After the host-side set-up of a figure the GPU has
    idled, and its clocks come back over its first ~30-40 ms of work: per
    replay of the batched step's graph (10 launches) 1,290-1,400 µs at first,
    1,105 µs from the 30th on; the 36-layer attention graph 390, then 350,
    then 337 µs from the 40th on."""
    import torch
    ms = SETTLE_MS if ms is None else ms
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(16):
            run()
        torch.cuda.synchronize()


def event_time_us(run, reps, warm: int = 1, settle_ms: float | None = None):
    """Mean duration of run() in µs from HIP events on the current stream,
    after `settle_ms` of untimed calls (the clocks' return from idle) and
    `warm` more."""
    import torch
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    settle(run, settle_ms)
    for _ in range(warm):
        run()
    a.record()
    for _ in range(reps):
        run()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / reps


def launch_pass(w: Workload, reps: int) -> None:
    """Eager launches only: the 36-layer dequant (one launch and per-layer
    launches) and attention of every layer, the turbo_mse 36-layer dequant,
    the one-launch pack of the 36
    layers, the logits entry, one step of the batched paged decode (append +
    attention), then a plain device copy of the dequant's byte count (the
    calibration kernel for the FETCH_SIZE / WRITE_SIZE counters)."""
    import torch
    half = w.deq_bytes // 4  # fp16 elements copied: deq_bytes / 2 read, / 2 written
    src = torch.empty(half, dtype=torch.float16, device=w.dev).fill_(1.0)
    dst = torch.empty_like(src)
    bt = batched_setup(w)
    repacked = [torch.zeros_like(p) for p in w.pools]
    lg = torch.empty(w.rows * w.H * w.N, dtype=torch.float32, device=w.dev)
    for _ in range(reps):
        w.all_dequant()
        w.all_dequant_per_layer()
        w.all_attention()
        w.all_dequant_mse()
        # the one-launch pack of the 36 dequantized layers into other pools,
        # and the logits entry on one layer
        w.tq.pack_layers("turbo_prod", w.out_k, w.out_v, w.slots, repacked, w.lp, w.cfg,
                         stream=w._stream())
        w.tq.fused_attn_logits(w.qa, w.pools[0], w.slots, lg, w.lp, w.cfg, w.rows, w.N,
                               stream=w._stream())
        bt["batch"].repack()
        bt["batch"].attention(bt["query"], bt["row_seq"], bt["row_len"], bt["tables"], bt["out"])
        for _ in range(4):
            dst.copy_(src)
    torch.cuda.synchronize()
    bt["batch"].close()
    log(f"[bench] launch pass: {reps} x {w.NL} layers; copy calibration kernel moves "
        f"{half * 2} B read + {half * 2} B written")


def main() -> int:
    global SETTLE_MS
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--settle-ms", type=float, default=SETTLE_MS,
                    help="untimed replays, in ms of wall time, before each figure's timed ones "
                         "(for the step: before its warmup steps); the GPU's clocks return from "
                         "idle over its first ~30-40 ms of work")
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--tokens", type=int, default=32768)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--launch-pass", action="store_true",
                    help="eager launches only (for rocprofv3 counter runs); no JSON line")
    args = ap.parse_args()
    SETTLE_MS = args.settle_ms
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the path has no cross-GPU "
              "exchange; each GPU would serve its own layers' pools) — run with --gpus 1",
              file=sys.stderr)
        return 2

    # The CPU baseline's build, compiled on this host before anything touches
    # the GPU (a child process, started while this process has no GPU state).
    native = None if args.no_cpu_baseline or args.launch_pass else build_native_oracle()

    import torch

    w = Workload(args.layers, args.tokens)
    if args.launch_pass:
        launch_pass(w, max(1, args.steps))
        return 0

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    w.side2 = torch.cuda.Stream()
    w.side2.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        w.step()  # sizes each stream's split-K workspace before capture
    with torch.cuda.stream(w.side2):
        w.all_attention()
    torch.cuda.synchronize()
    use_graph = not args.no_graph
    g_step = g_two = g_att = g_deq1 = None
    if use_graph:
        g_step = capture(w.step, side)
        g_two = capture(w.step_two_streams, side)
        g_att = capture(w.all_attention, side)
        g_deq1 = capture(w.all_dequant_per_layer, side)
        use_graph = None not in (g_step, g_two, g_att, g_deq1)
    run_step = g_step.replay if use_graph else w.step
    run_two = g_two.replay if use_graph else w.step_two_streams
    run_att = g_att.replay if use_graph else w.all_attention
    run_deq1 = g_deq1.replay if use_graph else w.all_dequant_per_layer

    # The timed region: K whole steps.
    settle(run_step, args.settle_ms)
    for _ in range(args.warmup):
        run_step()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        run_step()
    ev1.record()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps
    ev_ms_per_step = ev0.elapsed_time(ev1) / args.steps
    two_ms = event_time_us(run_two, args.steps) / 1e3
    log(f"[bench] step {ms_per_step:.3f} ms wall, {ev_ms_per_step:.3f} ms events "
        f"({'graph' if use_graph else 'eager'}; one-launch dequant, then attention, one stream); "
        f"per-layer dequant beside attention on two streams: {two_ms:.3f} ms")

    # Per-kernel averages, replayed from graphs and timed with events: the
    # one-launch dequant of the 36 layers (the roofline kernel), the 36
    # per-layer dequant launches, and the 36 attention launches (split +
    # combine).
    reps = max(3, args.steps)
    # The one-launch dequant: four launches replayed from one graph, so the
    # host's per-call work (36 layers' pointer checks) stays out of the
    # window and the average is the kernel's own duration plus a graph
    # node's gap, as the kernel trace records it.
    def four_dequants():
        for _ in range(4):
            w.all_dequant()
    g4 = capture(four_dequants, side) if use_graph else None
    # (at least 100 timed launches after 12 untimed ones)
    launch_us = event_time_us(g4.replay if g4 is not None else four_dequants, max(25, reps),
                              warm=3) / 4
    deq_us = launch_us / w.NL
    deq1_us = event_time_us(run_deq1, reps) / w.NL
    att_us = event_time_us(run_att, reps) / w.NL
    deq_gbps = w.deq_bytes / (deq_us * 1e-6) / 1e9
    deq1_gbps = w.deq_bytes / (deq1_us * 1e-6) / 1e9
    att_gbps = w.att_bytes / (att_us * 1e-6) / 1e9
    log(f"[bench] dequant {deq_us:.2f} us/layer {deq_gbps:.0f} GB/s (one launch for {w.NL} "
        f"layers; {deq1_us:.2f} us/layer {deq1_gbps:.0f} GB/s as per-layer launches); "
        f"attention {att_us:.2f} us/layer {att_gbps:.0f} GB/s")

    # A plain device copy of the dequant's byte count, MALL-cold (36 buffers).
    half = w.deq_bytes // 4
    srcs = [torch.ones(half, dtype=torch.float16, device=w.dev) for _ in range(8)]
    dsts = [torch.empty_like(s) for s in srcs]

    def copies():
        for s, d in zip(srcs, dsts):
            d.copy_(s)
    copy_us = event_time_us(copies, reps) / len(srcs)

    # Config 3's turbo_mse form: the same 36 layers in turbo_mse pages.
    def four_mse():
        for _ in range(4):
            w.all_dequant_mse()
    with torch.cuda.stream(side):
        w.all_dequant_mse()
        w.all_dequant_mse_per_layer()
    torch.cuda.synchronize()
    g_m4 = capture(four_mse, side) if use_graph else None
    g_m1 = capture(w.all_dequant_mse_per_layer, side) if use_graph else None
    mse_us = event_time_us(g_m4.replay if g_m4 is not None else four_mse, reps) / 4 / w.NL
    mse1_us = event_time_us(g_m1.replay if g_m1 is not None else w.all_dequant_mse_per_layer,
                            reps) / w.NL
    # turbo_mse pages read (the used bytes: codes and the two norms) + fp16 written + slots
    mse_bytes = w.N * w.H * (w.D + 4) + 2 * w.N * w.H * w.D * 2 + w.N * 4
    dequant_mse = {"us_per_layer": round(mse_us, 3),
                   "GBps": round(mse_bytes / mse_us / 1e3, 1),
                   "frac_hbm": round(mse_bytes / mse_us / 1e3 / HBM_PEAK_GBPS, 4),
                   "per_layer_launches_us_per_layer": round(mse1_us, 3),
                   "algorithmic_bytes_per_layer": mse_bytes,
                   "kernel": "tq::dequant_rows_kernel<0, 64, 128>: 36 layers, one launch"}
    log(f"[bench] turbo_mse dequant {mse_us:.2f} us/layer one launch, {mse1_us:.2f} per-layer")
    del srcs, dsts

    # HBM bytes per dispatch of the roofline kernel on this workload, from the
    # two calibrated counter runs (FETCH_SIZE, WRITE_SIZE) summarised in
    # profiles/traffic.json.
    traffic = kernel_traffic(DEQUANT_KERNEL)
    # The attention layer's HBM bytes (split + combine) from the same summary.
    att_parts = [kernel_traffic(k) for k in ATTN_KERNELS]
    att_traffic = ({"bytes": sum(t["bytes"] for t in att_parts),
                    "ratio_to_algorithmic": round(sum(t["bytes"] for t in att_parts) / w.att_bytes, 3),
                    "source": "profiles/traffic.json"}
                   if all(att_parts) else None)

    loader = measure_loader(w)
    log(f"[bench] loader: {w.NL} layers host->device + dequant to [1,H,N,D] in "
        f"{loader['ms']:.2f} ms ({loader['host_GBps']:.1f} GB/s of pages); copies alone "
        f"{loader['h2d_only_ms']:.2f} ms")

    store = measure_store(w)
    log(f"[bench] store: {w.NL} layers .bin/.meta -> [1,H,N,D] in {store['ms']:.2f} ms; "
        f"the reference's per-layer load path {store['reference_path_ms']:.2f} ms "
        f"(outputs identical: {store['identical']})")

    pack = measure_pack(w)
    log(f"[bench] pack (36 layers x 8192 tokens): turbo_prod {pack['turbo_prod_us_per_layer']:.1f} "
        f"us/layer ({pack['turbo_prod_one_launch_us_per_layer']:.1f} as one launch), turbo_mse "
        f"{pack['turbo_mse_us_per_layer']:.1f} us/layer "
        f"({pack['turbo_mse_one_launch_us_per_layer']:.1f}); mismatched bytes "
        f"vs oracle {pack['parity']['mismatched_page_bytes']}, boundary counts "
        f"{pack['parity']['turbo_prod_boundary']}")

    logits = measure_logits(w)
    log(f"[bench] turbo_prod logits @32K: {logits['us']:.1f} us ({logits['GBps']:.0f} GB/s)")

    legacy = measure_legacy(w)
    log(f"[bench] unexported kernels @32K: qjl dequant {legacy['qjl_dequant_us']:.1f} us, "
        f"qjl attention {legacy['qjl_attention_us']:.1f} us, int4 dequant "
        f"{legacy['int4_dequant_us']:.1f} us")

    batched = measure_batched(w)
    for sch in ("turbo_prod", "turbo_mse"):
        b_ = batched[sch]
        log(f"[bench] batched decode {sch}: {b_['sequences']} sequences, {b_['rows']} rows: "
            f"append {b_['append_us']:.1f} us + attention {b_['attention_us']:.1f} us")

    floor = measure_graph_floor(w)
    log(f"[bench] graph floor: {floor['one_kernel_us']:.2f} us per small kernel, "
        f"{floor['two_dependent_kernels_us']:.2f} us per dependent pair")

    single = measure_single_query(w)
    log(f"[bench] single-query decode @32K: {single['us_per_layer']:.2f} us/layer")

    config1 = measure_config1(w)
    log(f"[bench] config 1 (turbo_mse [2,1143,128], CPU oracle): rel MSE K "
        f"{config1['rel_mse_k']}, V {config1['rel_mse_v']}; GPU identical: "
        f"{config1['gpu_pool_identical'] and config1['gpu_dequant_identical']}")

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(w, native)

    value = w.step_bytes / (ms_per_step * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms": args.settle_ms,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8 codes -> fp32 math -> fp16 (dequant); attention: fp16 MFMA on hi/lo-split "
                 "fp16 operands (~22-bit query and P), fp32 accumulate and softmax",
        "data": "synthetic",
        "config": {
            "workload": "per layer: turbo_prod dequant [32768,2,128] + GQA 16/2 decode "
                        "attention @32K, 36 layers (Qwen2.5-3B shape), shuffled 16-token pages",
            "layers": w.NL, "tokens": w.N, "kv_heads": w.H, "q_heads": w.q_heads,
            "head_dim": w.D, "page_tokens": w.B, "scheme": "turbo_prod",
            "graph_replay": bool(use_graph),
            "streams": "one stream: the one-launch 36-layer dequant (the roofline kernel), "
                       "then the 36 attention launches (step_ms_two_streams: per-layer dequant "
                       "launches beside the attention chain on a second stream)",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": f"{DEQUANT_KERNEL}: turbo_prod dequant of the {w.NL} layers, one launch",
            "achieved": round(deq_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(deq_gbps / HBM_PEAK_GBPS, 4),
            "traffic": traffic["bytes"] if traffic else None,
            "traffic_detail": traffic,
            "algorithmic_bytes": w.NL * w.deq_bytes,
            "algorithmic_bytes_per_layer": w.deq_bytes,
            "avg_launch_us": round(launch_us, 3),
            "us_per_layer": round(deq_us, 3),
            "per_layer_launches": {"us_per_layer": round(deq1_us, 3),
                                   "GBps": round(deq1_gbps, 1),
                                   "frac": round(deq1_gbps / HBM_PEAK_GBPS, 4),
                                   "kernel": DEQUANT_KERNEL_1},
            "copy_same_bytes_us": round(copy_us, 3),
        },
        "dequant_turbo_mse": dequant_mse,
        "decode_attn": {
            "us_per_layer": round(att_us, 3),
            "achieved_GBps": round(att_gbps, 1),
            "frac_hbm": round(att_gbps / HBM_PEAK_GBPS, 4),
            "algorithmic_bytes": w.att_bytes,
            "kernels_per_layer": 2,
            "kernels": list(ATTN_KERNELS),
            "traffic": att_traffic,
            "graph_floor": floor,
        },
        "loader": loader,
        "store": store,
        "pack": pack,
        "logits": logits,
        "unexported_kernels": legacy,
        "batched_decode": batched,
        "single_query_decode": single,
        "config1": config1,
        "step_ms_events": round(ev_ms_per_step, 4),
        "step_ms_two_streams": round(two_ms, 4),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def measure_loader(w: Workload, reps: int = 3) -> dict:
    """The layer-pipelined loader (tq_load_*_layers), config 3 for both
    schemes: every layer's pages from pinned host memory to the GPU on a copy
    stream, each layer dequantized into [1, H, N, D] on the compute stream as
    its copy lands.  PCIe-inclusive, so reported beside the HBM-resident
    figures, not as them.  The turbo_prod figures are also at the top level."""
    import torch
    copy = torch.cuda.Stream()
    compute = torch.cuda.current_stream()
    out = {}
    for scheme, pools, lay in (("turbo_prod", w.pools, w.lp), ("turbo_mse", w.mse_pools, w.lm)):
        host = [p.cpu().pin_memory() for p in pools]
        dev = [torch.empty_like(p) for p in pools]

        def load():
            w.tq.load_layers(scheme, host, dev, w.slots, w.out_k, w.out_v, lay, w.cfg, w.N,
                             copy_stream=copy.cuda_stream, compute_stream=compute.cuda_stream)

        def copies_only():
            with torch.cuda.stream(copy):
                for h, d in zip(host, dev):
                    d.copy_(h, non_blocking=True)
            compute.wait_stream(copy)

        load()
        torch.cuda.synchronize()
        ms = event_time_us(load, reps) / 1e3
        h2d = event_time_us(copies_only, reps) / 1e3
        page_bytes = sum(p.numel() for p in pools)
        out[scheme] = {"layers": w.NL, "ms": round(ms, 3),
                       "host_GBps": round(page_bytes / ms / 1e6, 2), "h2d_only_ms": round(h2d, 3),
                       "h2d_GBps": round(page_bytes / h2d / 1e6, 2),
                       "output": "[1, H, N, D] fp16 per layer", "host_memory": "pinned"}
        del host, dev
    out.update(out["turbo_prod"])
    return out


def measure_store(w: Workload, reps: int = 3) -> dict:
    """The on-disk store: the step's 36 layers written as .bin/.meta files
    (CAGStore format) to a temporary directory, then loaded into [1, H, N, D]
    by CAGStore.load_layers_hnd (parallel file reads into pinned staging, a
    group of layers at a time, overlapped with the copies and dequant).
    Beside it, the reference's per-layer path (cag_store.py:161-254: manifest
    check, read_bytes -> bytearray -> frombuffer -> clone -> pageable copy,
    meta load, dequant to [N, H, D], permute copy), with this library's
    dequant.  Host wall clock, page cache warm; both outputs compared."""
    import hashlib
    import shutil
    import tempfile

    import torch

    from turborag_amd.cag_store import CAGStore
    d = tempfile.mkdtemp(prefix="tqstore_", dir=os.environ.get("TMPDIR", "/tmp"))
    try:
        st = CAGStore(d, tq=w.tq)
        fmt = st._format("turbo_prod", w.cfg, w.lp, w.N)
        slots_cpu = w.slots.cpu()
        layers = list(range(w.NL))
        for l in layers:
            st.io.write_pool(st._pool_path("doc", l, "turbo_prod"), w.pools[l], fmt)
            st.io.write_meta(st._meta_path("doc", l, "turbo_prod"), w.N, slots_cpu, fmt)
            st._update_manifest("doc", l, "turbo_prod", w.N)
        manifest = os.path.join(d, "manifest.json")

        def ours():
            ks, vs, _ = st.load_layers_hnd("doc", layers, "turbo_prod", (w.H, w.D))
            torch.cuda.synchronize()
            return ks, vs

        def reference_path():
            ks, vs = [], []
            for l in layers:
                m = json.loads(open(manifest).read())
                assert m["entries"]["doc"]["sha256"] == hashlib.sha256(b"doc").hexdigest()
                meta = torch.load(st._meta_path("doc", l, "turbo_prod"), weights_only=True)
                raw = st._pool_path("doc", l, "turbo_prod").read_bytes()
                pool = torch.frombuffer(bytearray(raw[:w.pool_bytes]), dtype=torch.uint8).clone()
                pool = pool.to("cuda", non_blocking=True)
                slots = meta["slots"].to("cuda")
                ok = torch.zeros(w.N, w.H, w.D, dtype=torch.float16, device="cuda")
                ov = torch.zeros_like(ok)
                w.tq.dequant(pool, slots, ok, ov, w.lp, w.cfg)
                ks.append(ok.permute(1, 0, 2).unsqueeze(0).contiguous())
                vs.append(ov.permute(1, 0, 2).unsqueeze(0).contiguous())
            torch.cuda.synchronize()
            return ks, vs

        def best(fn):
            fn()
            ts = []
            for _ in range(reps):
                t0 = time.perf_counter()
                out = fn()
                ts.append((time.perf_counter() - t0) * 1e3)
                del out
            return min(ts)

        a, b = ours(), reference_path()
        same = all(torch.equal(x, y) for x, y in zip(a[0] + a[1], b[0] + b[1]))
        del a, b
        ms, ref_ms = best(ours), best(reference_path)
    finally:
        shutil.rmtree(d, ignore_errors=True)
    page_bytes = w.NL * w.pool_bytes
    return {"layers": w.NL, "ms": round(ms, 2), "reference_path_ms": round(ref_ms, 2),
            "speedup": round(ref_ms / ms, 2), "pages_GBps": round(page_bytes / ms / 1e6, 2),
            "identical": bool(same), "files": "page cache (written just before)",
            "output": "[1, H, N, D] fp16 per layer"}


def measure_pack(w: Workload, reps: int = 5) -> dict:
    """Config 2, quantize on append: 36 layers x 8192 tokens of K/V (H = 2,
    D = 128, seeds 200 + layer) packed into turbo_prod and turbo_mse pools,
    as 36 per-layer launches (the reference's form) and as one launch for the
    36 layers (tq_launch_*_pack_kv_layers), with slots = arange (as the
    reference's store packs a document, cag_store.py:129) and with shuffled
    16-token pages.  Graph replays, HIP events.  Algorithmic bytes per layer:
    fp16 K/V and slots read, pages written.  The pools of the last (one-launch,
    shuffled) fill are checked against the oracle."""
    import torch

    from turborag_amd.synthetic import permuted_slots
    tq, N, NL = w.tq, 8192, w.NL
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim, cfg.block_size = w.H, w.D, w.B
    lp, lm = tq.make_layout_for(cfg), tq.make_mse_layout_for(cfg)
    slot_sets = {"arange": torch.arange(N, dtype=torch.int32, device=w.dev),
                 "shuffled": permuted_slots(N, w.B, seed=402).to(w.dev)}
    kv = [gpu_kv(N, w.H, w.D, 200 + l, w.dev) for l in range(NL)]
    keys, values = [k for k, _ in kv], [v for _, v in kv]
    pages = (N + w.B - 1) // w.B
    pools = {"turbo_prod": [torch.zeros(pages * lp.page_size_bytes, dtype=torch.uint8,
                                        device=w.dev) for _ in range(NL)],
             "turbo_mse": [torch.zeros(pages * lm.page_size_bytes, dtype=torch.uint8,
                                       device=w.dev) for _ in range(NL)]}
    lays = {"turbo_prod": lp, "turbo_mse": lm}
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())

    def per_layer(scheme, slots):
        fn = tq.pack if scheme == "turbo_prod" else tq.mse_pack

        def run():
            st = torch.cuda.current_stream().cuda_stream
            for (k, v), p in zip(kv, pools[scheme]):
                fn(k, v, slots, p, lays[scheme], cfg, stream=st)
        return run

    def one_launch(scheme, slots):
        def run():
            tq.pack_layers(scheme, keys, values, slots, pools[scheme], lays[scheme], cfg,
                           stream=torch.cuda.current_stream().cuda_stream)
        return run

    def timed(fn):
        with torch.cuda.stream(side):
            fn()
        torch.cuda.synchronize()
        g = capture(fn, side)
        return event_time_us(g.replay if g is not None else fn, reps) / NL

    out = {"layers": NL, "tokens": N}
    fp16 = 2 * N * w.H * w.D * 2
    for scheme in ("turbo_prod", "turbo_mse"):
        alg = fp16 + N * 4 + pages * lays[scheme].page_size_bytes
        for form, make in (("", per_layer), ("one_launch_", one_launch)):
            for sk, slots in slot_sets.items():
                us = timed(make(scheme, slots))
                key = f"{scheme}_{form}{'' if sk == 'arange' else 'shuffled_'}us_per_layer"
                out[key] = round(us, 2)
                if sk == "arange":
                    out[f"{scheme}_{form}GBps"] = round(alg / us / 1e3, 1)
                    out[f"{scheme}_{form}frac_hbm"] = round(alg / us / 1e3 / HBM_PEAK_GBPS, 4)
    out["algorithmic_bytes_per_layer_turbo_prod"] = fp16 + N * 4 + pages * lp.page_size_bytes
    out["slots"] = "arange (the store's form); *_shuffled_*: a permutation of 16-token pages"
    torch.cuda.synchronize()
    out["parity"] = pack_parity(w, kv, slot_sets["shuffled"], pools["turbo_prod"],
                                pools["turbo_mse"], pages)
    del kv, keys, values, pools
    return out


def pack_parity(w: Workload, kv, slots, pp, pm, pages) -> dict:
    """Config 2's parity report: every layer's GPU-packed pages against the
    oracle's pack of the same K/V (mismatching bytes, expected 0), and the
    decision-boundary counts the north star asks to report: rotated values
    within one float ulp of a codebook decision boundary, where the exact
    bits of the reference build's rsqrtf(128) (tq_turbo_prod_kernels.cu:188)
    or its FMA contraction of the pair sum (tq_turbo_mse_kernels.cu:108)
    could flip a code.  Both schemes, all layers, the oracle on this host."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np

    from oracle.oracle import load
    from turborag_amd.synthetic import as_u16
    orc = load()
    orc.nthreads = host_cpu()["usable"]
    slots_np = slots.cpu().numpy()
    host = [(as_u16(k), as_u16(v)) for k, v in kv]
    mism = {"turbo_prod": 0, "turbo_mse": 0}
    for (k, v), p, q in zip(host, pp, pm):
        mism["turbo_prod"] += int(np.count_nonzero(
            p.cpu().numpy() != orc.prod_pack(k, v, slots_np, pages, w.B)))
        mism["turbo_mse"] += int(np.count_nonzero(
            q.cpu().numpy() != orc.mse_pack(k, v, slots_np, pages, w.B)))
    with ThreadPoolExecutor(orc.nthreads) as ex:
        pl = list(ex.map(lambda kv_: orc.prod_boundary_list(*kv_), host))
        mc = list(ex.map(lambda kv_: orc.boundary_counts("turbo_mse", *kv_), host))
    # Each flagged turbo_prod value beside the GPU's own normalised value: the
    # debug pack (tq_launch_turbo_prod_pack_kv_debug) of the same layer.
    import torch
    cfg = w.tq.default_config()
    cfg.num_kv_heads, cfg.head_dim, cfg.block_size = w.H, w.D, w.B
    lp = w.tq.make_layout_for(cfg)
    scratch = torch.zeros(pages * lp.page_size_bytes, dtype=torch.uint8, device=w.dev)
    kinds = ("k_code", "k_residual_sign", "v_code")
    flagged = []
    for layer, ((k, v), (elem, kind, val)) in enumerate(zip(kv, pl)):
        if len(elem) == 0:
            continue
        dbg = w.tq.pack_debug(k, v, slots, scratch, lp, cfg)
        idx = torch.from_numpy(elem).to(w.dev)
        gkn = dbg["kn"].reshape(-1)[idx].cpu().numpy()
        gvn = dbg["vn"].reshape(-1)[idx].cpu().numpy()
        for e, kd, x, a, b in zip(elem, kind, val, gkn, gvn):
            t, rest = divmod(int(e), w.H * w.D)
            g_ = float(b if kd == 2 else a)
            flagged.append({"layer": layer, "token": t, "head": rest // w.D, "d": rest % w.D,
                            "kind": kinds[int(kd)], "oracle": float(x), "gpu": g_})
        del dbg
    values = len(host) * host[0][0].size
    return {
        "layers_checked": len(host),
        "mismatched_page_bytes": mism,
        "values_per_tensor": values,
        "turbo_prod_boundary": {kinds[c]: int(sum(int((kd == c).sum()) for _, kd, _ in pl))
                                for c in range(3)},
        "turbo_prod_boundary_values": flagged,
        "turbo_prod_boundary_gpu_equals_oracle": all(f["gpu"] == f["oracle"] for f in flagged),
        "turbo_mse_boundary": {"rows_norm_differs_unfused_pairsum": sum(c[0] for c in mc),
                               "code_bytes_differ_unfused_pairsum": sum(c[1] for c in mc),
                               "codes_within_1ulp": sum(c[2] for c in mc)},
    }


def measure_logits(w: Workload, reps: int = 10) -> dict:
    """The turbo_prod logits entry on every layer of the step (GQA 16/2 rows,
    32K tokens): fp32 logits [8, 2, 32768] written per layer, 36 calls
    replayed from a graph.  Algorithmic bytes: pool + slots + query read,
    logits written."""
    import torch
    lg = [torch.empty(w.rows * w.H * w.N, dtype=torch.float32, device=w.dev) for _ in range(w.NL)]

    def run():
        for layer in range(w.NL):
            w.tq.fused_attn_logits(w.qa, w.pools[layer], w.slots, lg[layer], w.lp, w.cfg, w.rows,
                                   w.N, stream=w._stream())
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.synchronize()
    g = capture(run, side)
    us = event_time_us(g.replay if g is not None else run, reps) / w.NL
    # read: each (token, head)'s K codes (D/2 bytes) and its K and residual
    # scales (the V half of the page is not read), the slots and the query
    alg = w.N * w.H * (w.D // 2 + 4) + w.N * 4 + w.qa.numel() * 2 + lg[0].numel() * 4
    del lg
    return {"us": round(us, 2), "algorithmic_bytes": alg, "GBps": round(alg / us / 1e3, 1),
            "shape": "8 GQA rows x 2 kv heads x 32768 tokens, fp32; 36 layers from a graph"}


def measure_legacy(w: Workload, reps: int = 10) -> dict:
    """The kernels the reference compiles but does not export, on one layer
    of the step's shape (32K tokens, H = 2, D = 128, the step's shuffled
    slots): QJL-1b pack / dequant / GQA 16/2 attention and legacy INT4 pack /
    dequant.  Each timed as a graph of 10 launches (HIP events), per launch."""
    import torch
    tq = w.tq
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim, cfg.block_size, cfg.group_size = w.H, w.D, w.B, w.D
    k, v = gpu_kv(w.N, w.H, w.D, 999, w.dev)
    pages = (w.N + w.B - 1) // w.B
    lq, li = tq.make_qjl_layout_for(cfg), tq.make_int4_layout_for(cfg)
    pq = torch.zeros(pages * lq.page_size_bytes, dtype=torch.uint8, device=w.dev)
    pi = torch.zeros(pages * li.page_size_bytes, dtype=torch.uint8, device=w.dev)
    ok = torch.empty(w.N, w.H, w.D, dtype=torch.float16, device=w.dev)
    ov = torch.empty_like(ok)
    out = torch.empty_like(w.att[0])
    st = w._stream
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())

    def graph_us(call, n=10):
        def run():
            for _ in range(n):
                call()
        with torch.cuda.stream(side):
            run()
        torch.cuda.synchronize()
        g = capture(run, side)
        return event_time_us(g.replay if g is not None else run, reps) / n

    # (pack first: the dequant and attention read its pages)
    t = {
        "qjl_pack_us": graph_us(lambda: tq.qjl_pack(k, v, w.slots, pq, lq, cfg, st())),
        "qjl_dequant_us": graph_us(lambda: tq.qjl_dequant(pq, w.slots, ok, ov, lq, cfg, st())),
        "qjl_attention_us": graph_us(
            lambda: tq.qjl_fused_attn_output(w.qa, pq, w.slots, out, lq, cfg, w.rows, w.N, st())),
        "int4_pack_us": graph_us(lambda: tq.int4_pack(k, v, w.slots, pi, li, cfg, st())),
        "int4_dequant_us": graph_us(lambda: tq.int4_dequant(pi, w.slots, ok, ov, li, cfg, st())),
    }
    fp16 = 2 * w.N * w.H * w.D * 2
    t = {k_: round(v_, 2) for k_, v_ in t.items()}
    t["qjl_dequant_GBps"] = round((pages * lq.page_size_bytes + fp16 + w.N * 4)
                                  / t["qjl_dequant_us"] / 1e3, 1)
    t["int4_dequant_GBps"] = round((pages * li.page_size_bytes + fp16 + w.N * 4)
                                   / t["int4_dequant_us"] / 1e3, 1)
    t["shape"] = "32768 tokens x 2 kv heads x 128, 8 GQA rows per kv head for attention"
    del k, v, pq, pi, ok, ov
    return t


def measure_config1(w: Workload) -> dict:
    """Config 1: K, V [2 kv heads, 1143 tokens, 128] (seed 101, HF [H, S, D]
    permuted to the ABI's [S, H, D]), turbo_mse pack then dequant on the CPU
    reference path (the oracle), the same on the GPU for parity.  Reported as
    the config asks: packed bytes, per-(token, head) fp16 scales and the
    reconstruction MSE (relative to the input variance, as the reference's
    tests/test_cag.py:240-247 measures it; its bound is 0.25)."""
    import hashlib

    import numpy as np
    import torch

    from oracle.oracle import load
    from turborag_amd.synthetic import as_u16, kv_tokens_major
    orc = load()
    N, H, D, B = 1143, 2, 128, 16
    k, v = kv_tokens_major(N, H, D, seed=101)
    slots = np.arange(N, dtype=np.int32)
    pages = (N + B - 1) // B
    t0 = time.perf_counter()
    pool = orc.mse_pack(as_u16(k), as_u16(v), slots, pages, B)
    ok, ov = orc.mse_dequant(pool, slots, H, D, B)
    cpu_ms = (time.perf_counter() - t0) * 1e3
    tq, cfg = w.tq, w.tq.default_config()
    cfg.num_kv_heads, cfg.head_dim, cfg.block_size = H, D, B
    lm = tq.make_mse_layout_for(cfg)
    gpool = torch.zeros(pages * lm.page_size_bytes, dtype=torch.uint8, device=w.dev)
    gs = torch.from_numpy(slots).to(w.dev)
    tq.mse_pack(k.to(w.dev), v.to(w.dev), gs, gpool, lm, cfg)
    gk = torch.empty(N, H, D, dtype=torch.float16, device=w.dev)
    gv = torch.empty_like(gk)
    tq.mse_dequant(gpool, gs, gk, gv, lm, cfg)
    torch.cuda.synchronize()
    same_pool = bool(np.array_equal(gpool.cpu().numpy(), pool))
    same_kv = bool(np.array_equal(as_u16(gk), ok) and np.array_equal(as_u16(gv), ov))

    def rel_mse(x, y_u16):
        y = torch.from_numpy(y_u16.view(np.float16)).float()
        return float(torch.mean((x.float() - y) ** 2) / torch.var(x.float()))

    codes = 2 * N * H * (D // 2)
    scales = 2 * N * H
    kn = pool.reshape(pages, -1)[:, lm.k_norms_offset:lm.k_norms_offset + B * H * 2]
    return {
        "shape": "K, V [2, 1143, 128] fp16, seed 101; turbo_mse, 16-token pages",
        "pool_bytes": int(pool.size), "code_bytes": codes, "scale_count": scales,
        "scale_bytes": 2 * scales,
        "pool_sha256": hashlib.sha256(pool.tobytes()).hexdigest(),
        "k_scales_first": [int(x) for x in kn[0].view(np.uint16)[:4]],
        "rel_mse_k": round(rel_mse(k, ok), 5), "rel_mse_v": round(rel_mse(v, ov), 5),
        "rel_mse_bound": 0.25,
        "cpu_ms": round(cpu_ms, 2),
        "gpu_pool_identical": same_pool, "gpu_dequant_identical": same_kv,
    }


def measure_single_query(w: Workload, reps: int = 5) -> dict:
    """Decode attention with one query row per kv head (num_queries = 1, the
    call the reference's store makes: cag_store.py:284-287) over every layer
    of the step at 32K, replayed from a graph, beside the GQA 16/2 figure."""
    import torch
    qa1 = w.qa[:1].contiguous()
    outs = [torch.empty(1, w.H, w.D, dtype=torch.float16, device=w.dev) for _ in range(w.NL)]
    st = w._stream

    def run():
        for layer in range(w.NL):
            w.tq.fused_attn_output(qa1, w.pools[layer], w.slots, outs[layer], w.lp, w.cfg, 1,
                                   w.N, stream=st())
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.synchronize()
    g = capture(run, side)
    us = event_time_us(g.replay if g is not None else run, reps) / w.NL
    alg = w.pool_bytes + w.N * 4 + 2 * w.H * w.D * 2
    return {"us_per_layer": round(us, 3), "algorithmic_bytes": alg,
            "GBps": round(alg / us / 1e3, 1), "frac_hbm": round(alg / us / 1e3 / HBM_PEAK_GBPS, 4),
            "path": "matrix-core split kernel (one row per kv head in an 8-row group)"}


def measure_graph_floor(w: Workload, reps: int = 10) -> dict:
    """What a graph-replayed layer costs before any attention work: 36 nodes
    of one small kernel (a 1 MB fill, the size of the split-K partials), and
    36 pairs of dependent small kernels (the fill, then a 16 KB read of what
    it wrote: the split/combine pair with trivial bodies), in µs per node and
    per pair."""
    import torch
    buf = torch.empty(1 << 18, dtype=torch.float32, device=w.dev)
    out = torch.empty(1 << 12, dtype=torch.float32, device=w.dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())

    def one():
        for _ in range(w.NL):
            buf.fill_(1.0)

    def pair():
        for _ in range(w.NL):
            buf.fill_(1.0)
            out.copy_(buf[: out.numel()])
    res = {}
    for name, fn in (("one_kernel_us", one), ("two_dependent_kernels_us", pair)):
        with torch.cuda.stream(side):
            fn()
        torch.cuda.synchronize()
        g = capture(fn, side)
        res[name] = round(event_time_us(g.replay if g is not None else fn, reps) / w.NL, 3)
    return res


def batched_setup(w: Workload, scheme: str = "turbo_prod") -> dict:
    """The batch of the batched-decode step: 32 sequences, lengths
    U[1024, 32768] (seed 500), 1-8 new tokens each (seed 501), appended."""
    import numpy as np
    import torch

    from turborag_amd.batched import PagedBatch
    from turborag_amd.synthetic import uniform_ints
    lens = uniform_ints(500, 32, 1024, 32768)
    widths = uniform_ints(501, 32, 1, 8)
    b = PagedBatch(w.tq, scheme, lens, widths, seed=500, device=w.dev)
    b.append_new_tokens(seed=503)
    query, row_seq, row_len = b.decode_rows(seed=504)
    return {"batch": b, "query": query, "row_seq": row_seq, "row_len": row_len,
            "tables": b.block_tables(), "out": torch.empty_like(query), "lens": lens,
            "widths": widths}


def measure_batched(w: Workload, reps: int = 10) -> dict:
    """Config 5 for both schemes: see measure_batched_scheme."""
    out = {s: measure_batched_scheme(w, s, reps) for s in ("turbo_prod", "turbo_mse")}
    out.update(out["turbo_prod"])  # the turbo_prod figures also at the top level
    return out


def measure_batched_scheme(w: Workload, scheme: str, reps: int = 10) -> dict:
    """One serving step of a batch of paged sequences (32 sequences, lengths
    U[1024, 32768], 1-8 new tokens each, pages scattered by the allocator):
    one pack launch appending every new token, then one paged-attention
    launch for 8 GQA rows per new token (causal over the new tokens)."""
    import torch

    st = batched_setup(w, scheme)
    b, query, row_seq, row_len = st["batch"], st["query"], st["row_seq"], st["row_len"]
    bt, out, lens, widths = st["tables"], st["out"], st["lens"], st["widths"]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())

    def graph_us(call, n=10):  # n launches replayed from a graph, per launch
        def run():
            for _ in range(n):
                call(torch.cuda.current_stream().cuda_stream)
        with torch.cuda.stream(side):
            run()
        torch.cuda.synchronize()
        g = capture(run, side)
        return event_time_us(g.replay if g is not None else run, reps) / n
    att_us = graph_us(lambda st: b.attention(query, row_seq, row_len, bt, out, stream=st))
    app_us = graph_us(lambda st: b.repack(stream=st))
    rows = int(query.shape[0])
    # Algorithmic bytes: each sequence's cells once per kv head (+4 B slot
    # per token), the new tokens' fp16 K/V in and cells out, query and output.
    # turbo_prod: 64 + 64 + 3 * 2 bytes per (token, head); turbo_mse: 64 + 64 + 2 * 2.
    cell = (134 if scheme == "turbo_prod" else 132) * w.H
    kv_tokens = int((lens + widths).sum())
    alg = kv_tokens * (cell + 4) + int(widths.sum()) * (2 * w.H * 128 * 2 + cell) + 2 * rows * w.H * 256
    # What this kernel reads: every new-token row group reads its own range.
    read = int(sum(sum(L + j + 1 for j in range(wd)) for L, wd in zip(lens, widths))) * cell
    b.close()
    return {"scheme": scheme, "sequences": 32, "rows": rows, "kv_tokens": kv_tokens,
            "new_tokens": int(widths.sum()), "append_us": round(app_us, 2),
            "attention_us": round(att_us, 2), "step_us": round(app_us + att_us, 2),
            "algorithmic_bytes": alg, "GBps_algorithmic": round(alg / (app_us + att_us) / 1e3, 1),
            "cells_read_bytes": read}


def host_cpu() -> dict:
    """This host's CPU: logical CPUs (nproc), the ones this process may use,
    and the model name (lscpu's "Model name", from /proc/cpuinfo)."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return {"nproc": os.cpu_count(), "usable": usable, "model": model}


NATIVE_FLAGS = ["-O2", "-march=native", "-ffp-contract=off"]


def build_native_oracle():
    """The oracle's C restatement compiled on this host with the CPU
    baseline's flags (-O2 -march=native -ffp-contract=off, no fast-math;
    -march=native is this host's CPU, so it is built here, into a temporary
    directory, not shipped).  Returns (path, command), or (None, reason)
    when gcc is missing or fails; the prebuilt oracle
    (oracle/build_oracle.sh: -O3 -march=x86-64-v3) is timed instead then."""
    import shutil
    import subprocess
    import tempfile
    gcc = shutil.which("gcc")
    if gcc is None:
        return None, "gcc not found"
    src = os.path.join(os.path.dirname(os.path.abspath(__file__)), "oracle", "tq_oracle.c")
    out = os.path.join(tempfile.mkdtemp(prefix="tq_cpu_baseline_"), "libtq_oracle_native.so")
    cmd = [gcc, *NATIVE_FLAGS, "-std=gnu99", "-fPIC", "-shared", "-o", out, src, "-lm",
           "-lpthread"]
    try:
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    except (OSError, subprocess.TimeoutExpired) as e:
        return None, f"gcc failed: {e}"
    if r.returncode != 0:
        return None, f"gcc failed: {r.stderr.strip()[-300:]}"
    return out, "gcc " + " ".join(NATIVE_FLAGS) + " -std=gnu99 -fPIC -shared oracle/tq_oracle.c"


def cpu_baseline(w: Workload, native=None, runs: int = 5, layers_per_run: int = 3):
    """The reference's CPU path for one decode step of this workload, on this
    host: per layer, the dequant (the oracle's C
    restatement of the reference kernel's operation order) to [N, H, D] fp16,
    the permute to [H, N, D] the reference's store does, and
    attention_ref_single_head (src/tq_attention_ref.cpp:10-56 semantics) for
    each of the 16 query heads over its kv head's dequantized K/V.  Timed on
    1 thread and on every usable core (the dequant's token rows and the
    query heads split over threads), each as the median of `runs` runs of
    `layers_per_run` layers after one warm-up run.  `native` is
    build_native_oracle()'s result: that build is timed when there is one
    (its dequant checked bit-identical to the prebuilt oracle's first)."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np

    from oracle.oracle import Oracle, load
    from turborag_amd.synthetic import as_u16
    orc = load()
    build = "gcc -O3 -march=x86-64-v3 -ffp-contract=off (oracle/build_oracle.sh)"
    same = None
    if native is not None and native[0] is not None:
        nat = Oracle(native[0])
        p0 = w.pools[0].cpu().numpy()
        s0 = w.slots.cpu().numpy()
        a = orc.prod_dequant(p0, s0, w.H, w.D, w.B)
        b = nat.prod_dequant(p0, s0, w.H, w.D, w.B)
        same = all(np.array_equal(x.view(np.uint16), y.view(np.uint16)) for x, y in zip(a, b))
        if same:
            orc, build = nat, native[1] + " (built on this host)"
        else:
            build += "; the -march=native build's dequant differed: not used"
    elif native is not None:
        build += f"; the -march=native build: {native[1]}"
    info = host_cpu()
    slots_np = w.slots.cpu().numpy()
    q_heads = as_u16(w.qa).transpose(1, 0, 2).reshape(w.q_heads, w.D)  # [h * rows + g]
    pools = [w.pools[l].cpu().numpy() for l in range(layers_per_run)]
    group = w.q_heads // w.H

    def layer(pool_np, threads, ex):
        orc.nthreads = threads
        t0 = time.perf_counter()
        ok, ov = orc.prod_dequant(pool_np, slots_np, w.H, w.D, w.B)
        kh = np.ascontiguousarray(ok.transpose(1, 0, 2))  # [H, N, D]
        vh = np.ascontiguousarray(ov.transpose(1, 0, 2))
        t1 = time.perf_counter()
        heads = range(w.q_heads)
        fn = lambda j: orc.sdpa_single_head(q_heads[j], kh[j // group], vh[j // group])
        outs = list(ex.map(fn, heads)) if ex is not None else [fn(j) for j in heads]
        t2 = time.perf_counter()
        assert len(outs) == w.q_heads
        return t1 - t0, t2 - t1

    def timed(threads):
        ex = ThreadPoolExecutor(threads) if threads > 1 else None
        try:
            for p in pools:  # warm-up run
                layer(p, threads, ex)
            samples = []
            for _ in range(runs):
                d = a = 0.0
                for p in pools:
                    dd, aa = layer(p, threads, ex)
                    d += dd
                    a += aa
                samples.append((d + a, d, a))
        finally:
            if ex is not None:
                ex.shutdown()
        samples.sort()
        tot, d, a = samples[len(samples) // 2]
        n = len(pools)
        return {"threads": threads,
                "value": round(n * (w.deq_bytes + w.att_bytes) / tot / 1e9, 3),
                "ms_per_layer": round(tot / n * 1e3, 2),
                "dequant_ms_per_layer": round(d / n * 1e3, 2),
                "attention_ms_per_layer": round(a / n * 1e3, 2)}

    one = timed(1)
    allc = timed(max(1, info["usable"]))
    log(f"[bench] cpu reference path ({info['model']}, nproc {info['nproc']}): "
        f"1 thread {one['ms_per_layer']:.1f} ms/layer, {allc['threads']} threads "
        f"{allc['ms_per_layer']:.1f} ms/layer")
    return {
        "value": allc["value"],
        "unit": "GB/s",
        "cores": allc["threads"],
        "kind": "port",
        "sample": f"{len(pools)} layers per run, median of {runs} runs after one warm-up: "
                  f"turbo_prod dequant of {w.N} tokens x {w.H} heads to fp16, permute to "
                  f"[H, N, D], then attention_ref_single_head for {w.q_heads} query heads "
                  f"over {w.N} tokens (GQA {w.q_heads}/{w.H}); same algorithmic bytes as "
                  f"the GPU step",
        "single_thread": one,
        "all_cores": allc,
        "host": info,
        "build": build,
        "native_build_matches_prebuilt": same,
    }


if __name__ == "__main__":
    sys.exit(main())
