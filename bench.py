#!/usr/bin/env python3
"""Benchmark of the batched multi-LoRA INT4 linear on one MI355X: tokens/s of a whole pass and the roofline fraction
of its dominant kernel, with the CPU restatement of the reference's torch layer timed beside it.

A step is one pass over one batch: route the request rows by adapter, then every fused group of every layer
(int4_product: LoRA first factor, then the INT4 base product with the second factor fused) and, where the workload
gathers each request's last-token output (prefill-skewed-28l), the decision head on it. The step is recorded once
as a HIP graph and replayed. Inputs (weights, adapter pool, activations) are resident in HBM before timing.

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--no-cpu]

Workloads (jeff_amd.workloads): prefill-1layer (default: one 1024 -> 3072 INT4 g128 layer, 16 adapters r16, 64
requests of 16..256 tokens), decode-28l, prefill-skewed-28l, decode-pool-28l. One JSON line is printed."""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

METRIC = "tokens/s for batched multi-LoRA int4 linear; % of HBM/MFMA roofline"
PEAK_HBM = 8.0e12      # bytes/s, MI355X HBM3E
PEAK_BF16 = 2.5e15     # flop/s, MI355X dense bf16 MFMA
DOMINANT = {"prefill-1layer": "gate_up", "decode-28l": "gate_up", "prefill-skewed-28l": "gate_up",
            "decode-pool-28l": "gate_up"}


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="prefill-1layer")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=20.0, help="bound on the CPU baseline's timed work")
    ap.add_argument("--kernel-reps", type=int, default=0, help="launches of the dominant kernel timed (0: auto)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain device copy of COPY_BYTES five times (the scale of the HBM byte counters)")
    return ap.parse_args()


COPY_BYTES = 1 << 30
TRAFFIC_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")


def copy_calibration() -> int:
    """Five copies of COPY_BYTES between two device buffers (torch's copy kernel): a profile of this run reads
    FETCH_SIZE and WRITE_SIZE for a known number of bytes moved, the factor that turns those counters into bytes."""
    import torch
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "copies": 5}))
    return 0


def measured_traffic(workload: str) -> float | None:
    """HBM bytes per launch of the dominant kernel from the committed counter profile of this workload
    (profiles/traffic_<workload>.txt, a line `bytes_per_launch=<N>`), or None when there is none."""
    path = os.path.join(TRAFFIC_DIR, f"traffic_{workload}.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("bytes_per_launch="):
                return float(line.split("=", 1)[1])
    return None


def main() -> int:
    args = parse()
    if args.copy_calibration:
        return copy_calibration()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE {world}). Run it with --gpus 1.", file=sys.stderr)
        return 2
    import torch

    from jeff_amd import workloads
    from jeff_amd.fast_path import DT, Workspace
    from jeff_amd.int4_kernels import base_expand, int4_product, shrink
    from jeff_amd.int4_tiles import int4_tiles
    from jeff_amd.epilogues import add_rms, silu_mul
    from jeff_amd.readout import readout_rows

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    w = workloads.make(args.workload, device="cuda")
    pool_rows = w.pool.lora_pool.shape[0]
    per_layer_acts = args.workload.startswith("decode")
    gen = torch.Generator(device="cuda").manual_seed(1234)
    xs = {}
    for li, layer in enumerate(w.layers):
        for label in layer:
            if per_layer_acts or li == 0:
                xs[(li, label)] = workloads.inputs(w, label, gen)
    max_rank = max(lin.rank for layer in w.layers for lin in layer.values())
    ws = Workspace(w.tokens, 1, max_rank=max_rank, max_requests=w.requests)
    last = torch.empty(w.requests, w.layers[-1]["down"].out, dtype=DT, device=dev) if w.gather_last else None
    keep: list[torch.Tensor] = []

    def step() -> None:
        ws._routed = None
        ws.route(w.adp, pool_rows, tokens=w.tokens, cu_seqlens=w.cu_seqlens)
        keep.clear()
        for li, layer in enumerate(w.layers):
            for label, lin in layer.items():
                x = xs[(li if per_layer_acts else 0, label)]
                gather = last if (last is not None and li == len(w.layers) - 1 and label == "down") else None
                keep.append(int4_product(lin, x, ws, w.adp, last_out=gather))
        if w.readout is not None:  # the decision head on each request's last-token output
            keep.append(readout_rows(last, w.readout["readout_pool"], w.readout["temp_pool"], w.adp,
                                     w.readout["counts"]))
        if len(keep) > 8:
            del keep[:-8]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    ws.check()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    tokens_per_s = w.tokens / (ms_per_step / 1e3)

    # the dominant kernel alone: the base product and the LoRA second factor of the largest group of layer 0 (one
    # launch of the fused 256-tile kernel for prefill; for decode the narrow or split product's launches), timed with
    # HIP events on the stream it runs on (the first factors it reads are computed once beforehand)
    label = DOMINANT[args.workload]
    lin = w.layers[0][label]
    x = xs[(0, label)]
    y = torch.empty(w.tokens, lin.out, dtype=DT, device=dev)
    ws._routed = None
    ws.route(w.adp, pool_rows, tokens=w.tokens, cu_seqlens=w.cu_seqlens)
    shrink(lin, x, ws, w.adp)
    base_expand(lin, x, ws, w.adp, y)
    torch.cuda.synchronize()
    kflops = 2.0 * w.tokens * lin.k * lin.out
    tok = workloads.token_ids(w)
    mean_rank = float(sum(w.adapter_ranks.get(int(a), 0) for a in tok)) / max(len(tok), 1)
    kflops += 2.0 * w.tokens * mean_rank * lin.out
    present = sorted({int(a) for a in tok} - {0})
    kbytes = float(lin.int4.nbytes()) + 2.0 * w.tokens * (lin.k + lin.out)
    kbytes += sum(2.0 * min(w.adapter_ranks[a], c) * n for a in present for n, c in zip(lin.sizes, lin.caps))
    reps = args.kernel_reps or max(5, min(200, int(2e12 / max(kflops, 1.0))))
    kgraph = torch.cuda.CUDAGraph()
    stream = torch.cuda.current_stream()
    with torch.cuda.graph(kgraph):
        for _ in range(reps):
            base_expand(lin, x, ws, w.adp, y)
    kgraph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    launch_ms = []
    for _ in range(3):
        e0.record(stream)
        kgraph.replay()
        e1.record(stream)
        e1.synchronize()
        launch_ms.append(e0.elapsed_time(e1) / reps)
    kms = statistics.median(launch_ms)
    mfma_bound = args.workload.startswith("prefill")
    traffic = measured_traffic(args.workload)
    if mfma_bound:
        achieved = kflops / (kms / 1e3)
        roof = {"bound": "mfma", "achieved": achieved / 1e12, "peak": PEAK_BF16 / 1e12, "unit": "TFLOP/s",
                "frac": achieved / PEAK_BF16, "traffic": traffic}
    else:
        achieved = kbytes / (kms / 1e3)
        roof = {"bound": "hbm", "achieved": achieved / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                "frac": achieved / PEAK_HBM, "traffic": traffic}
    tiles = int4_tiles(lin.int4.columns, lin.k, w.tokens, w.requests, pool_rows)
    kernel = {"mfma": "base_mfma256_kernel (INT4 base + fused LoRA expand)" if w.tokens >= 1024 else
              "base_mfma_kernel<true> (INT4 base + fused LoRA expand)",
              "split": "base_mfma256_kernel, split mode + finish_kernel (INT4 base + LoRA expand, 2 launches)",
              "narrow": "dec_kernel (INT4 base + fused LoRA expand; dec_reduce_kernel adds split input ranges)",
              "gemv": "base_gemv_kernel<true> (INT4 base + fused LoRA expand)"}[tiles.base]
    roof.update({"kernel": kernel, "group": f"layer0.{label}", "launch_ms": kms, "flops_per_launch": kflops,
                 "bytes_per_launch": kbytes})
    step_flops = workloads.flops_per_token(w) * w.tokens
    step_bytes = workloads.hbm_bytes(w)
    step_roof = {"mfma_frac": step_flops / (ms_per_step / 1e3) / PEAK_BF16,
                 "hbm_frac": step_bytes / (ms_per_step / 1e3) / PEAK_HBM,
                 "flops": step_flops, "bytes": step_bytes}

    head = None
    if w.readout is not None:  # the decision head alone: its two launches, timed as the dominant kernel is
        r = w.readout
        hreps = 50
        hgraph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(hgraph):
            for _ in range(hreps):
                readout_rows(last, r["readout_pool"], r["temp_pool"], w.adp, r["counts"])
        hgraph.replay()
        torch.cuda.synchronize()
        head_ms = []
        for _ in range(3):
            e0.record(stream)
            hgraph.replay()
            e1.record(stream)
            e1.synchronize()
            head_ms.append(e0.elapsed_time(e1) / hreps)
        hms = statistics.median(head_ms)
        hbytes = workloads.readout_bytes(w)
        head = {"kernels": "readout_logits_kernel + option_softmax_kernel", "ms": hms, "bytes": hbytes,
                "hbm_frac": hbytes / (hms / 1e3) / PEAK_HBM, "rows": w.requests,
                "options": int(r["readout_pool"].shape[1]), "dim": int(r["readout_pool"].shape[2])}
        del hgraph

    # the element-wise steps around the linear at this pass's shapes: residual add + RMSNorm of the hidden rows before
    # the gate_up product, SiLU(gate) * up after it; each timed alone as above
    gl = w.layers[0]["gate_up"]
    hid, inter = gl.k, gl.out // 2
    eg = torch.Generator(device="cuda").manual_seed(77)
    ex = torch.randn(w.tokens, hid, device=dev, generator=eg).to(DT)
    ed = torch.randn(w.tokens, hid, device=dev, generator=eg).to(DT)
    ew = (1 + 0.1 * torch.randn(hid, device=dev, generator=eg)).float()
    egu = torch.randn(w.tokens, 2 * inter, device=dev, generator=eg).to(DT)

    def timed(fn, nbytes: float) -> dict:
        reps = 20
        g = torch.cuda.CUDAGraph()
        fn()
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            for _ in range(reps):
                fn()
        g.replay()
        torch.cuda.synchronize()
        ts = []
        for _ in range(3):
            e0.record(stream)
            g.replay()
            e1.record(stream)
            e1.synchronize()
            ts.append(e0.elapsed_time(e1) / reps)
        ms = statistics.median(ts)
        return {"ms": ms, "bytes": nbytes, "hbm_frac": nbytes / (ms / 1e3) / PEAK_HBM}

    epilogues = {"rows": w.tokens, "hidden": hid, "inter": inter,
                 "add_rms": timed(lambda: add_rms(ex, ed, ew), 2.0 * w.tokens * hid * 4 + 4.0 * hid),
                 "silu_mul": timed(lambda: silu_mul(egu), 2.0 * w.tokens * inter * 3)}
    del ex, ed, egu

    cpu = None if args.no_cpu else cpu_baseline(w, xs, per_layer_acts, args.cpu_seconds)
    del graph, kgraph
    config = {"workload": args.workload, "tokens": w.tokens, "requests": w.requests, "layers": len(w.layers),
              "groups": {k: [v.k, v.out] for k, v in w.layers[0].items()},
              "adapters": len(w.adapter_ranks), "ranks": sorted(set(w.adapter_ranks.values())),
              "group_size": 128, "zero_points": True, "step_roofline": step_roof}
    if head is not None:
        config["decision_head"] = head
    config["epilogues"] = epilogues
    print(json.dumps({"metric": METRIC, "value": tokens_per_s, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
                      "warmup": args.warmup, "ms_per_step": ms_per_step, "higher_is_better": True, "scaling": "weak",
                      "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded; random INT4 weights and "
                      "adapters at the configuration's shapes)", "config": config, "roofline": roof,
                      "cpu_baseline": cpu}))
    return 0


def cpu_baseline(w, xs, per_layer_acts: bool, budget_s: float) -> dict:
    """The oracle's restatement of the reference's torch layer (LoraLinear.forward per adapter segment, bf16 "model"
    precision) on the host cores, over one layer's groups and all tokens (3 warm-up runs, then the median of up to
    10 runs within the budget), scaled to the whole pass."""
    import numpy as np
    import torch

    from jeff_amd import workloads
    from oracle.layer import layer_model
    from oracle.pool_view import adapters_of, weights_of

    threads = min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    tok = workloads.token_ids(w)
    present = np.unique(tok)
    layer = w.layers[0]
    data = []
    for label, lin in layer.items():
        data.append((xs[(0, label)].cpu(), weights_of(lin.int4), adapters_of(lin, present), lin.sizes))

    def run() -> None:
        for x, wt, adapters, sizes in data:
            layer_model(x, wt, tok, adapters, sizes)

    times = []
    start = time.perf_counter()
    for i in range(13):
        t0 = time.perf_counter()
        run()
        dt = time.perf_counter() - t0
        if i >= 3:
            times.append(dt)
        if time.perf_counter() - start > budget_s and len(times) >= 1:
            break
    per_layer = statistics.median(times)
    scale = len(w.layers)
    value = w.tokens / (per_layer * scale)
    return {"value": value, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"one layer of {scale} ({', '.join(layer)}), all {w.tokens} tokens, bf16 torch on the CPU, "
                      f"median of {len(times)} runs after 3 warm-ups" + (f", scaled by {scale}" if scale > 1 else ""),
            "per_layer_s": per_layer}


if __name__ == "__main__":
    sys.exit(main())
