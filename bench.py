#!/usr/bin/env python3
"""Benchmark of the batched multi-LoRA INT4 linear on one MI355X: tokens/s of a whole pass and the roofline fraction
of its dominant kernel, with the CPU restatement of the reference's torch layer timed beside it on every workload,
and the reference's other product ("cublas": torch's GEMM on the dequantised bf16 weights, then lora_add) timed
against the INT4 product by the reference's own choice rule.

A step is one pass over one batch: route the request rows by adapter, then every fused group of every layer
(int4_product: LoRA first factor, then the INT4 base product with the second factor fused; the decoder's gate_up
group writes SiLU(gate) * up from its output tile, the activation the down product reads) and, where the workload
gathers each request's last-token output (prefill-skewed-28l), the decision head on it. The step is recorded once
as a HIP graph and replayed. Inputs (weights, adapter pool, activations) are resident in HBM before timing.

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--also NAMES|none] [--no-cpu]

The printed line's workload is prefill-skewed-28l (default): 28 layers of hidden 2048 / intermediate 6144, 512
requests of LogNormal(ln 200, 1) lengths clipped to 16..2048, 128 adapters of rank 32 with Zipf(1.1) popularity, the
largest single-GPU workload by work. The same run measures decode-28l (256 one-token rows, 64 adapters of ranks
8..64), decode-pool-28l (4096 one-token rows, 1024 adapters of rank 64, a 142.8 GB pool), prefill-1layer (one
1024 -> 3072 layer, 64 requests of 16..256 tokens) and cpu-1024 (the CPU reference configuration: one bf16 1024 ->
1024 layer, 256 tokens in 8 requests of 32, 4 adapters of rank 16), each with its own roofline block and CPU
baseline, under config.workloads.
Progress goes to stderr; stdout holds the one JSON line."""

from __future__ import annotations

import argparse
import gc
import json
import os
import statistics
import sys
import time

METRIC = "tokens/s for batched multi-LoRA int4 linear; % of HBM/MFMA roofline"
PEAK_HBM = 8.0e12      # bytes/s, MI355X HBM3E
PEAK_BF16 = 2.5e15     # flop/s, MI355X dense bf16 MFMA
HEADLINE = "prefill-skewed-28l"
ALSO = ("decode-28l", "decode-pool-28l", "prefill-1layer", "cpu-1024")
DOMINANT = "gate_up"   # the largest group of every workload: its layer-0 product is the dominant kernel
EPILOGUE = {"gate_up": "silu_mul"}  # SiLU(gate) * up in the gate_up product's output tile (decoder workloads)
BOX_THREADS = 16       # the host threads one GPU's share of the machine offers
REFERENCE_THREADS = 8  # the reference's default torch thread count (engine/model.py:166-170)
CPU_SAMPLE_TOKENS = 16384  # tokens of the CPU baseline's sample (the pass's first requests up to at least this)


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default=HEADLINE)
    ap.add_argument("--also", default=",".join(ALSO), help="other workloads measured in the same run, or 'none'")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--no-choice", action="store_true",
                    help="skip timing the library GEMM product (\"cublas\") beside the INT4 product")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="bound on each CPU thread count's timed work")
    ap.add_argument("--kernel-reps", type=int, default=0, help="launches of the dominant kernel timed (0: auto)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain device copy of COPY_BYTES five times (the scale of the HBM byte counters)")
    return ap.parse_args()


COPY_BYTES = 1 << 30
TRAFFIC_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")


def note(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


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


def replay_ms(graph, stream, reps: int, rounds: int = 3) -> float:
    """Median over `rounds` of one replay of `graph` (holding `reps` repetitions of some work), per repetition, timed
    with HIP events on `stream` (the stream the graph is launched on)."""
    import torch
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    graph.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(rounds):
        e0.record(stream)
        graph.replay()
        e1.record(stream)
        e1.synchronize()
        ts.append(e0.elapsed_time(e1) / reps)
    return statistics.median(ts)


def capture(fn, reps: int):
    import torch
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    return g


def cpu_sample(w, xs: dict) -> dict:
    """What the CPU baseline of a workload needs, on the host: one layer's groups (the oracle's dequantised weights,
    or the bf16 W of a bf16 base; the adapters the sample's tokens read) over the pass's first requests up to
    CPU_SAMPLE_TOKENS tokens (the whole pass when it is smaller)."""
    import numpy as np

    from jeff_amd import workloads
    from oracle.pool_view import adapters_of, weights_of

    tok = workloads.token_ids(w)
    cu = np.concatenate([[0], np.cumsum(w.lengths)])
    m = int(np.searchsorted(cu, min(CPU_SAMPLE_TOKENS, w.tokens)))
    t_s = int(cu[m])
    tok_s = tok[:t_s]
    pres = sorted({int(a) for a in tok_s})
    groups = []
    for label, lin in w.layers[0].items():
        wt = lin.W.cpu() if lin.int4 is None else weights_of(lin.int4)
        groups.append((label, xs[(0, label)][:t_s].cpu(), wt, adapters_of(lin, pres), lin.sizes))
    return {"tok": tok_s, "layers": len(w.layers), "tokens": t_s, "requests": m, "all_tokens": w.tokens,
            "groups": groups}


def product_choice(w, xs: dict, ws, per_layer_acts: bool) -> dict:
    """The reference's choice between its product kernels for this pass (engine/batched_path.py:492-524 with
    product_choice.choose_product): every fused group of every layer once, in layer order, plain products (no
    epilogue), recorded as one graph per candidate and timed in alternating rounds, the median of each kept. "cublas"
    is Lin.__call__ (torch's GEMM on the dequantised bf16 W, then the HIP lora_add); "int4" is int4_product."""
    import torch

    from jeff_amd.int4 import dequantize_kernel
    from jeff_amd.product_choice import choose_product, product

    lins = [(li, label, lin) for li, layer in enumerate(w.layers) for label, lin in layer.items()]
    for _, _, lin in lins:
        lin.W = dequantize_kernel(lin.int4)
    stream = torch.cuda.current_stream()
    graphs = {}

    def time_ms(kernel: str) -> float:
        if kernel not in graphs:
            prod = product(kernel)

            def products() -> None:
                for li, label, lin in lins:
                    prod(lin, xs[(li if per_layer_acts else 0, label)], ws, w.adp)

            graphs[kernel] = capture(products, 1)
        return replay_ms(graphs[kernel], stream, 1, rounds=1)

    pick = choose_product(("cublas", "int4"), time_ms)
    graphs.clear()
    for _, _, lin in lins:
        lin.W = None
    torch.cuda.empty_cache()
    note(f"{w.name}: product choice {pick.kernel} {pick.ms}")
    return {"kernel": pick.kernel, "ms_per_pass": pick.ms,
            "note": "the reference's rule: every group of every layer once per candidate, medians of 3 alternating "
                    "rounds, the faster recorded (cublas: torch GEMM on the dequantised bf16 W + HIP lora_add)"}


def measure(name: str, steps: int, warmup: int, kernel_reps: int, headline: bool, want_cpu: bool = True,
            compare_products: bool = True) -> tuple[dict, dict]:
    """One workload: (its measurements, the objects its CPU baseline needs)."""
    import torch

    from jeff_amd import workloads
    from jeff_amd.epilogues import add_rms, rms, silu_mul
    from jeff_amd.fast_path import DT, Workspace
    from jeff_amd.int4_kernels import base_expand, int4_product, shrink
    from jeff_amd import _lib
    from jeff_amd.int4_tiles import int4_plan
    from jeff_amd.readout import readout_rows

    dev = torch.device("cuda:0")
    t_build = time.perf_counter()
    w = workloads.make(name, device="cuda")
    pool_rows = w.pool.lora_pool.shape[0]
    per_layer_acts = name.startswith("decode")
    gen = torch.Generator(device="cuda").manual_seed(1234)
    xs = {}
    for li, layer in enumerate(w.layers):
        for label in layer:
            if per_layer_acts or li == 0:
                xs[(li, label)] = workloads.inputs(w, label, gen)
    max_rank = max(lin.rank for layer in w.layers for lin in layer.values())
    shapes = {(lin.k, lin.out) for layer in w.layers for lin in layer.values()}
    ws = Workspace(w.tokens, 1, shapes, max_rank=max_rank, max_requests=w.requests)
    last = torch.empty(w.requests, w.layers[-1]["down"].out, dtype=DT, device=dev) if w.gather_last else None
    keep: list[torch.Tensor] = []
    torch.cuda.synchronize()
    note(f"{name}: built in {time.perf_counter() - t_build:.1f} s ({w.tokens} tokens, {len(w.layers)} layers)")

    bf16_base = all(lin.int4 is None for layer in w.layers for lin in layer.values())

    def step() -> None:
        ws.route(w.adp, pool_rows, tokens=w.tokens, cu_seqlens=w.cu_seqlens)
        keep.clear()
        for li, layer in enumerate(w.layers):
            for label, lin in layer.items():
                x = xs[(li if per_layer_acts else 0, label)]
                if bf16_base:  # the reference's "cublas" product: torch's GEMM on W, then lora_add
                    keep.append(lin(x, ws, w.adp))
                    continue
                gather = last if (last is not None and li == len(w.layers) - 1 and label == "down") else None
                epi = EPILOGUE.get(label) if w.gated else None
                keep.append(int4_product(lin, x, ws, w.adp, last_out=gather, epilogue=epi))
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
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        graph.replay()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / steps
    tokens_per_s = w.tokens / (ms_per_step / 1e3)
    note(f"{name}: {steps} steps of {ms_per_step:.3f} ms")
    del graph
    cpu_inputs = cpu_sample(w, xs) if want_cpu else {}
    step_flops = workloads.flops_per_token(w) * w.tokens
    step_bytes = workloads.hbm_bytes(w, gated=tuple(EPILOGUE) if w.gated else ())
    step_roof = {"mfma_frac": step_flops / (ms_per_step / 1e3) / PEAK_BF16,
                 "hbm_frac": step_bytes / (ms_per_step / 1e3) / PEAK_HBM,
                 "flops": step_flops, "bytes": step_bytes}
    if bf16_base:
        # one bf16 layer: the step is the whole product (x W^T on torch's GEMM, then the HIP lora_add), so the step's
        # time is the product's; launch-bound at this size
        result = {"workload": name, "value": tokens_per_s, "unit": "tokens/s", "ms_per_step": ms_per_step,
                  "steps": steps, "warmup": warmup, "tokens": w.tokens, "requests": w.requests,
                  "layers": len(w.layers), "groups": {k: [v.k, v.out] for k, v in w.layers[0].items()},
                  "adapters": len(w.adapter_ranks), "ranks": sorted(set(w.adapter_ranks.values())),
                  "base": "bf16 (torch GEMM on W, then mlora_lora_add: the reference's Lin.__call__)",
                  "roofline": {"bound": "mfma", "achieved": step_flops / (ms_per_step / 1e3) / 1e12,
                               "peak": PEAK_BF16 / 1e12, "unit": "TFLOP/s",
                               "frac": step_flops / (ms_per_step / 1e3) / PEAK_BF16, "traffic": None,
                               "kernel": "torch GEMM + lora_add (shrink_seg_kernel, base_mfma_kernel<false>)",
                               "note": "launch-bound: 0.55 GFLOP per step"},
                  "step_roofline": step_roof}
        del w, xs, keep, ws, last
        gc.collect()
        torch.cuda.empty_cache()
        return result, cpu_inputs
    choice = product_choice(w, xs, ws, per_layer_acts) if compare_products else None

    # the dominant kernel alone: the base product and the LoRA second factor of layer 0's gate_up (one launch of the
    # fused 256-tile kernel for prefill; for decode the narrow or split product's launches), timed with HIP events on
    # the stream it runs on, the first factors it reads computed once beforehand. Its timing graph starts with the
    # pass's routing launch (the products of a recorded pass share it), so a graph of that launch alone is timed too
    # and subtracted.
    lin = w.layers[0][DOMINANT]
    x = xs[(0, DOMINANT)]
    gated = w.gated and DOMINANT in EPILOGUE
    epi = EPILOGUE.get(DOMINANT) if gated else None
    out_cols = lin.out // 2 if gated else lin.out
    y = torch.empty(w.tokens, out_cols, dtype=DT, device=dev)
    ws.route(w.adp, pool_rows, tokens=w.tokens, cu_seqlens=w.cu_seqlens)
    shrink(lin, x, ws, w.adp)
    base_expand(lin, x, ws, w.adp, y, epilogue=epi)
    torch.cuda.synchronize()
    kflops = 2.0 * w.tokens * lin.k * lin.out
    tok = workloads.token_ids(w)
    mean_rank = float(sum(w.adapter_ranks.get(int(a), 0) for a in tok)) / max(len(tok), 1)
    kflops += 2.0 * w.tokens * mean_rank * lin.out
    present = sorted({int(a) for a in tok} - {0})
    kbytes = float(lin.int4.nbytes()) + 2.0 * w.tokens * (lin.k + out_cols)
    kbytes += sum(2.0 * min(w.adapter_ranks[a], c) * n for a in present for n, c in zip(lin.sizes, lin.caps))
    reps = kernel_reps or max(5, min(200, int(2e12 / max(kflops, 1.0))))
    stream = torch.cuda.current_stream()

    def route_then(k: int):
        def fn() -> None:
            ws.route(w.adp, pool_rows, tokens=w.tokens, cu_seqlens=w.cu_seqlens)
            for _ in range(k):
                base_expand(lin, x, ws, w.adp, y, epilogue=epi)
        return fn

    kgraph = capture(route_then(reps), 1)
    rgraph = capture(route_then(0), 1)
    full_ms, route_ms = replay_ms(kgraph, stream, 1), replay_ms(rgraph, stream, 1)
    kms = (full_ms - route_ms) / reps
    del kgraph, rgraph
    if name.startswith("prefill"):
        achieved = kflops / (kms / 1e3)
        roof = {"bound": "mfma", "achieved": achieved / 1e12, "peak": PEAK_BF16 / 1e12, "unit": "TFLOP/s",
                "frac": achieved / PEAK_BF16, "traffic": measured_traffic(name)}
    else:
        achieved = kbytes / (kms / 1e3)
        roof = {"bound": "hbm", "achieved": achieved / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                "frac": achieved / PEAK_HBM, "traffic": measured_traffic(name)}
    base, _, ranges = int4_plan(lin.int4.columns, lin.k, w.tokens, w.requests, pool_rows, lin.rank, lin.out,
                                _lib.EPILOGUE_SILU_MUL if gated else 0)
    fin = " + silu(gate) * up" if gated else ""
    kernel = {"mfma": f"base_mfma256_kernel (INT4 base + fused LoRA expand{fin})" if w.tokens >= 1024 or gated else
              "base_mfma_kernel<true> (INT4 base + fused LoRA expand)",
              "split": f"base_mfma256_kernel, split mode ({ranges} input ranges) + "
                       f"{'finish_gated_kernel' if gated else 'finish_kernel'} (INT4 base + LoRA expand{fin})",
              "narrow": (f"dec_kernel (INT4 base, {ranges} input ranges) + dec_expand_kernel (the ranges' sum + "
                         f"LoRA expand{fin})" if ranges > 1 else f"dec_kernel (INT4 base + fused LoRA expand{fin}; "
                                                                 f"1 input range)"),
              "gemv": "base_gemv_kernel<true> (INT4 base + fused LoRA expand)"}[base]
    roof.update({"kernel": kernel, "group": f"layer0.{DOMINANT}", "launch_ms": kms, "reps": reps,
                 "route_ms_subtracted": route_ms, "flops_per_launch": kflops, "bytes_per_launch": kbytes})
    result = {"workload": name, "value": tokens_per_s, "unit": "tokens/s", "ms_per_step": ms_per_step,
              "steps": steps, "warmup": warmup, "tokens": w.tokens, "requests": w.requests, "layers": len(w.layers),
              "groups": {k: [v.k, v.out] for k, v in w.layers[0].items()},
              "adapters": len(w.adapter_ranks), "ranks": sorted(set(w.adapter_ranks.values())),
              "group_size": 128, "zero_points": True, "roofline": roof, "step_roofline": step_roof}
    if choice is not None:
        result["product_choice"] = choice
    note(f"{name}: dominant kernel {kms:.4f} ms, {roof['frac']:.3f} of the {roof['bound']} roofline")

    if gated:
        # SiLU(gate) * up in the product's output tile against the plain product followed by the separate silu_mul
        # launch: the whole gate_up product (first factor included) each way, timed alone as above
        g_reps = max(3, min(100, reps))
        plain = capture(lambda: silu_mul(int4_product(lin, x, ws, w.adp)), g_reps)
        fused = capture(lambda: int4_product(lin, x, ws, w.adp, epilogue="silu_mul"), g_reps)
        plain_ms, fused_ms = replay_ms(plain, stream, g_reps), replay_ms(fused, stream, g_reps)
        del plain, fused
        inter = lin.out // 2
        result["fused_silu_mul"] = {"group": f"layer0.{DOMINANT}", "plain_product_and_silu_mul_ms": plain_ms,
                                    "fused_product_ms": fused_ms,
                                    "hbm_bytes_saved": 2.0 * w.tokens * inter * 4,
                                    "note": "the plain product writes 2 inter columns, silu_mul reads them and writes "
                                            "inter; the fused product writes inter columns once"}

    if w.gated:
        # the residual add in the down product's output tile, then the RMSNorm of the sums, against the plain product
        # followed by add_rms (which adds and normalises): the whole down product each way (first factor included)
        dl = w.layers[0]["down"]
        dx = xs[(0, "down")]
        rg = torch.Generator(device="cuda").manual_seed(78)
        resid0 = torch.randn(w.tokens, dl.out, device=dev, generator=rg).to(DT)
        resid = resid0.clone()
        nw = (1 + 0.1 * torch.randn(dl.out, device=dev, generator=rg)).float()
        d_reps = max(3, min(100, int(reps * lin.out * lin.k / (dl.out * dl.k))))

        def fused_down() -> None:  # (the residual grows by the product each repetition: timing only)
            int4_product(dl, dx, ws, w.adp, epilogue="residual", residual=resid)
            rms(resid, nw)

        plain = capture(lambda: add_rms(resid0, int4_product(dl, dx, ws, w.adp), nw), d_reps)
        fused = capture(fused_down, d_reps)
        plain_ms, fused_ms = replay_ms(plain, stream, d_reps), replay_ms(fused, stream, d_reps)
        del plain, fused, resid, resid0
        result["fused_residual_add"] = {"group": "layer0.down", "plain_product_and_add_rms_ms": plain_ms,
                                        "fused_product_and_rms_ms": fused_ms,
                                        "hbm_bytes_saved": 2.0 * w.tokens * dl.out * 2,
                                        "note": "the plain product writes d, add_rms reads x and d and writes x + d "
                                                "and the norm; the fused product reads x and writes x + d in its "
                                                "output tile, rms reads x + d and writes the norm"}

    if name == "decode-28l":
        # the few-token GEMV (at most 8 tokens: base_gemv_kernel) at this workload's gate_up shape: its first 8
        # requests (one token each) and their adapters, the plain product, timed as the dominant kernel is; HBM-bound
        # on the weights
        gl = w.layers[0]["gate_up"]
        t8 = 8
        x8 = xs[(0, "gate_up")][:t8]
        adp8 = w.adp[:t8].contiguous()
        cu8 = torch.arange(t8 + 1, dtype=torch.int32, device=dev)
        ws8 = Workspace(t8, 1, max_rank=gl.rank, max_requests=t8)
        y8 = torch.empty(t8, gl.out, dtype=DT, device=dev)
        base8 = int4_plan(gl.int4.columns, gl.k, t8, t8, pool_rows, gl.rank, gl.out)[0]
        ws8.route(adp8, pool_rows, tokens=t8, cu_seqlens=cu8)
        shrink(gl, x8, ws8, adp8)

        def gemv_then(k: int):
            def fn() -> None:
                ws8.route(adp8, pool_rows, tokens=t8, cu_seqlens=cu8)
                for _ in range(k):
                    base_expand(gl, x8, ws8, adp8, y8)
            return fn

        g_reps = 100
        ggraph, grgraph = capture(gemv_then(g_reps), 1), capture(gemv_then(0), 1)
        gms = (replay_ms(ggraph, stream, 1) - replay_ms(grgraph, stream, 1)) / g_reps
        del ggraph, grgraph
        ids8 = sorted({int(a) for a in adp8.cpu().tolist()} - {0})
        gbytes = float(gl.int4.nbytes()) + 2.0 * t8 * (gl.k + gl.out)
        gbytes += sum(2.0 * min(w.adapter_ranks[a], c) * n for a in ids8 for n, c in zip(gl.sizes, gl.caps))
        result["gemv"] = {"kernel": f"{base8} (base_gemv_kernel<true>: INT4 base + fused LoRA expand)",
                          "group": "layer0.gate_up", "tokens": t8, "adapters": len(ids8), "ms": gms,
                          "bytes": gbytes, "achieved_gb_s": gbytes / (gms / 1e3) / 1e9,
                          "hbm_frac": gbytes / (gms / 1e3) / PEAK_HBM}
        del x8, ws8, y8

    if w.readout is not None:  # the decision head alone: its two launches, timed as the dominant kernel is
        r = w.readout
        hreps = 50
        hgraph = capture(lambda: readout_rows(last, r["readout_pool"], r["temp_pool"], w.adp, r["counts"]), hreps)
        hms = replay_ms(hgraph, stream, hreps)
        del hgraph
        hbytes = workloads.readout_bytes(w)
        result["decision_head"] = {"kernels": "readout_logits_kernel + option_softmax_kernel", "ms": hms,
                                   "bytes": hbytes, "hbm_frac": hbytes / (hms / 1e3) / PEAK_HBM, "rows": w.requests,
                                   "options": int(r["readout_pool"].shape[1]), "dim": int(r["readout_pool"].shape[2])}

    if headline:
        # the element-wise steps around the linear at this pass's shapes: residual add + RMSNorm of the hidden rows
        # before the gate_up product, SiLU(gate) * up after it; each timed alone as above
        gl = w.layers[0]["gate_up"]
        hid, inter = gl.k, gl.out // 2
        eg = torch.Generator(device="cuda").manual_seed(77)
        ex = torch.randn(w.tokens, hid, device=dev, generator=eg).to(DT)
        ed = torch.randn(w.tokens, hid, device=dev, generator=eg).to(DT)
        ew = (1 + 0.1 * torch.randn(hid, device=dev, generator=eg)).float()
        egu = torch.randn(w.tokens, 2 * inter, device=dev, generator=eg).to(DT)

        def timed(fn, nbytes: float) -> dict:
            g = capture(fn, 20)
            ms = replay_ms(g, stream, 20)
            return {"ms": ms, "bytes": nbytes, "hbm_frac": nbytes / (ms / 1e3) / PEAK_HBM}

        result["epilogues"] = {"rows": w.tokens, "hidden": hid, "inter": inter,
                               "add_rms": timed(lambda: add_rms(ex, ed, ew), 2.0 * w.tokens * hid * 4 + 4.0 * hid),
                               "silu_mul": timed(lambda: silu_mul(egu), 2.0 * w.tokens * inter * 3)}
        del ex, ed, egu

    del w, xs, keep, ws, last, y, x, lin
    gc.collect()
    torch.cuda.empty_cache()
    return result, cpu_inputs


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def lscpu() -> dict:
    """The host's lscpu fields that say what the CPU baseline ran on (empty when lscpu is missing)."""
    import subprocess
    keep = ("Model name", "Vendor ID", "CPU(s)", "On-line CPU(s) list", "Thread(s) per core", "Core(s) per socket",
            "Socket(s)", "NUMA node(s)", "CPU max MHz", "L3 cache", "Flags")
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
    except (OSError, subprocess.SubprocessError):
        return {}
    info = {}
    for line in out.splitlines():
        key, _, val = line.partition(":")
        key = key.strip()
        if key in keep:
            val = val.strip()
            if key == "Flags":  # the vector extensions torch's CPU GEMM can use
                val = " ".join(f for f in val.split() if f.startswith(("avx512", "avx2", "amx", "fma")))
            info[key] = val
    return info


def cpu_baseline(inp: dict, budget_s: float) -> dict:
    """The oracle's restatement of the reference's torch layer (LoraLinear.forward per adapter segment, bf16 "model"
    precision) on the host, over one layer's four groups and a sample of the pass's requests (3 warm-up runs, then
    the median of up to 10 runs within the budget), scaled to the whole pass; at the box's thread share and at the
    reference's 8."""
    import torch

    from oracle.layer import layer_model

    tok = inp["tok"]

    def run() -> None:
        for _, x, wt, adapters, sizes in inp["groups"]:
            layer_model(x, wt, tok, adapters, sizes)

    def timed(threads: int) -> tuple[float, int]:
        torch.set_num_threads(threads)
        times = []
        start = time.perf_counter()
        for i in range(13):
            t0 = time.perf_counter()
            run()
            dt = time.perf_counter() - t0
            if i >= 3:
                times.append(dt)
            if time.perf_counter() - start > budget_s and times:
                break
        return statistics.median(times), len(times)

    host = os.cpu_count() or 1
    share = min(BOX_THREADS, host)
    per_layer, runs = timed(share)
    note(f"cpu baseline: {share} threads, {per_layer:.3f} s per layer")
    per_layer8, runs8 = timed(min(REFERENCE_THREADS, host))
    note(f"cpu baseline: {min(REFERENCE_THREADS, host)} threads, {per_layer8:.3f} s per layer")
    scale = inp["layers"]
    tokens = inp["tokens"]
    labels = ", ".join(g[0] for g in inp["groups"])
    whole = tokens == inp["all_tokens"]
    what = (f"the whole pass ({tokens} tokens in {inp['requests']} requests)" if whole else
            f"the pass's first {inp['requests']} requests ({tokens} of its {inp['all_tokens']} tokens)")
    if scale == 1:
        sample = f"{labels} over {what}, bf16 torch on the CPU, median of {runs} runs after 3 warm-ups"
    else:
        sample = (f"one layer of {scale} ({labels}) over {what}, bf16 torch on the CPU, median of {runs} runs after 3 "
                  f"warm-ups; tokens/s scaled by 1/{scale} for the whole pass (an extrapolation: the {scale} layers "
                  f"have the same shapes)")
    return {"value": tokens / (per_layer * scale), "unit": "tokens/s", "cores": share, "kind": "port",
            "sample": sample, "per_layer_s": per_layer,
            "threads_8": {"value": tokens / (per_layer8 * scale), "cores": min(REFERENCE_THREADS, host),
                          "per_layer_s": per_layer8, "runs": runs8},
            "host_cpus": host, "cpu_model": cpu_model(), "lscpu": lscpu()}


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
    torch.cuda.set_device(0)
    also = [] if args.also in ("", "none") else [n for n in args.also.split(",") if n != args.workload]
    want_cpu = not args.no_cpu
    head, cpu_inputs = measure(args.workload, args.steps, args.warmup, args.kernel_reps, headline=True,
                               want_cpu=want_cpu, compare_products=not args.no_choice)
    others, other_inputs = {}, {}
    for name in also:
        others[name], other_inputs[name] = measure(name, args.steps, args.warmup, args.kernel_reps, headline=False,
                                                   want_cpu=want_cpu, compare_products=not args.no_choice)
    # the CPU baselines after every GPU measurement, so host work never overlaps the GPU's timed regions
    cpu = cpu_baseline(cpu_inputs, args.cpu_seconds) if want_cpu else None
    for name, inp in other_inputs.items():
        if inp:
            others[name]["cpu_baseline"] = cpu_baseline(inp, args.cpu_seconds)
            other_inputs[name] = None
    config = {k: v for k, v in head.items() if k not in ("value", "unit", "ms_per_step", "steps", "warmup",
                                                         "roofline")}
    config["workloads"] = others
    print(json.dumps({"metric": METRIC, "value": head["value"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
                      "warmup": args.warmup, "ms_per_step": head["ms_per_step"], "higher_is_better": True,
                      "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
                      "data": "synthetic (seeded; random INT4 weights and adapters at the configuration's shapes)",
                      "config": config, "roofline": head["roofline"], "cpu_baseline": cpu}))
    return 0


if __name__ == "__main__":
    sys.exit(main())
