"""Seeded synthetic workloads at the benchmark configurations' shapes (no checkpoints are available offline).

A workload is a set of fused groups (Lin) with INT4 weights and an adapter pool, plus the requests of one pass:
- "cpu-1024": one bf16 layer 1024 -> 1024, 256 tokens in 8 requests of 32, 4 adapters of rank 16;
- "prefill-1layer": one INT4 layer 1024 -> 3072 (g128, asymmetric), 16 adapters rank 16, 64 requests of U{16..256};
- "decode-28l": 28 layers x {qkv 2048->4096, o 2048->2048, gate_up 2048->12288, down 6144->2048}, 256 one-token
  rows, 64 adapters with ranks 8/16/32/64 (16 each), adapter per row uniform;
- "prefill-skewed-28l": the same layers, 512 requests with lengths LogNormal(ln 200, 1) clipped to [16, 2048],
  128 adapters of rank 32 chosen with Zipf(1.1) popularity, each request's last-token output gathered for the
  decision head (a readout of 255 options x 2048 per adapter row, bf16 0.05 N(0, 1); temperatures U(0.5, 2); option
  counts uniform in [1, 255]);
- "decode-pool-28l": the same layers, 4096 one-token rows, 1024 adapters of rank 64 all resident, uniform ids.
Weights: codes uniform in [0, 15], zero points uniform in [0, 15], bf16 scales U(0.005, 0.02), 128 inputs per
group. LoRA: A ~ N(0, (1/32)^2), B ~ N(0, 0.02^2), scale alpha/r = 2 folded into B. x ~ N(0, 1) bf16."""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

from jeff_amd.fast_path import DT, AdapterPool, Lin
from jeff_amd.int4 import KernelInt4, pack_kernel_asym

HIDDEN, INTER, Q_OUT, KV_OUT = 2048, 6144, 16 * 128, 8 * 128
GROUPS_28L = {  # label: (matrix names, outputs, inputs)
    "qkv": (["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"], [Q_OUT, KV_OUT, KV_OUT], HIDDEN),
    "o": (["self_attn.o_proj"], [HIDDEN], Q_OUT),
    "gate_up": (["mlp.gate_proj", "mlp.up_proj"], [INTER, INTER], HIDDEN),
    "down": (["mlp.down_proj"], [HIDDEN], INTER),
}
SIGMA_A, SIGMA_B, LORA_SCALE = 1.0 / 32, 0.02, 2.0
READOUT_OPTIONS = 255  # the decision head's options (engine/batched_kernels.py READOUT_ROWS)


@dataclass
class Workload:
    name: str
    layers: list[dict[str, Lin]]
    pool: AdapterPool
    adp: torch.Tensor                     # int32 (requests,) pool rows
    cu_seqlens: torch.Tensor | None       # int32 (requests + 1,) or None for one-token rows
    tokens: int
    requests: int
    lengths: np.ndarray
    adapter_ranks: dict[int, int]         # pool row -> rank of every adapted matrix
    gather_last: bool = False
    readout: dict | None = None           # decision head: readout_pool, temp_pool, counts (gather_last workloads)
    gated: bool = False                   # gate_up is a gate and an up matrix of one width (SiLU(gate) * up applies)
    notes: dict = field(default_factory=dict)


def _int4_weights(out: int, k: int, gen: torch.Generator, device: str, group: int = 128) -> KernelInt4:
    codes = torch.randint(0, 16, (out, k), generator=gen, device=device, dtype=torch.uint8)
    zeros = torch.randint(0, 16, (out, k // group), generator=gen, device=device, dtype=torch.uint8)
    scales = (torch.rand(out, k // group, generator=gen, device=device) * 0.015 + 0.005).to(torch.bfloat16)
    return pack_kernel_asym(codes, scales, zeros, group)


def _fill_adapters(pool: AdapterPool, ranks: dict[int, int], gen: torch.Generator, device: str) -> None:
    """Fill pool rows 1..n with random adapters, a whole group's block of rows at a time: A ~ N(0, SIGMA_A),
    sB = 2 B with B ~ N(0, SIGMA_B) rounded to bf16 (doubling is exact, so this is bf16(2 B) as fold_scale gives)."""
    rows = sorted(ranks)
    assert rows == list(range(1, len(rows) + 1)), "adapters fill the rows after the base row in order"
    n = len(rows)
    for lin in pool.lins:
        block = pool.lora_pool[1:n + 1, lin.off_a:lin.off_a + lin.numel()]
        block[:, :lin.rank * lin.k].normal_(0.0, SIGMA_A, generator=gen)
        b = block[:, lin.rank * lin.k:]
        b.normal_(0.0, SIGMA_B, generator=gen)
        b.mul_(LORA_SCALE)
    r = torch.tensor([ranks[a] for a in rows], dtype=torch.int32, device=device)
    col = 0
    for lin in pool.lins:
        for cap in lin.caps:
            pool.ranks[1:n + 1, col] = torch.clamp(r, max=cap)
            col += 1
    for a in rows:
        name = f"adapter-{a}"
        pool.adapter_index[name] = a
        pool.free_rows.remove(a)


def _layers(n_layers: int, cap: int, gen: torch.Generator, device: str) -> list[dict[str, Lin]]:
    layers = []
    for i in range(n_layers):
        layer = {}
        for label, (names, sizes, k) in GROUPS_28L.items():
            lin = Lin([f"layers.{i}.{n}" for n in names], sizes=sizes, k=k, ranks=[cap] * len(names))
            lin.int4 = _int4_weights(lin.out, k, gen, device)
            layer[label] = lin
        layers.append(layer)
    return layers


def make(name: str, device: str = "cuda", seed: int = 0, n_layers: int | None = None) -> Workload:
    """Build a workload on `device`. n_layers overrides the 28 layers of the decoder workloads (tests use fewer)."""
    gen = torch.Generator(device=device).manual_seed(seed)
    rng = np.random.default_rng(seed)
    if name == "cpu-1024":
        # one bf16 layer (no INT4 weights: the reference's "cublas" product, x W^T then lora_add), W ~ N(0, 0.02)
        w16 = (0.02 * torch.randn(1024, 1024, generator=gen, device=device)).to(DT)
        lin = Lin(["layers.0.self_attn.o_proj"], [w16], ranks=[16])
        pool = AdapterPool([lin], 4, device)
        ranks = {a: 16 for a in range(1, 5)}
        _fill_adapters(pool, ranks, gen, device)
        lengths = np.full(8, 32, dtype=np.int64)
        ids = rng.integers(1, 5, 8)
        layers = [{"o": lin}]
        gather = False
    elif name == "prefill-1layer":
        lin = Lin(["layers.0.mlp.gate_proj"], sizes=[3072], k=1024, ranks=[16])
        lin.int4 = _int4_weights(3072, 1024, gen, device)
        pool = AdapterPool([lin], 16, device)
        ranks = {a: 16 for a in range(1, 17)}
        _fill_adapters(pool, ranks, gen, device)
        lengths = rng.integers(16, 257, 64)
        ids = rng.integers(1, 17, 64)
        layers = [{"gate_up": lin}]
        gather = False
    elif name in ("decode-28l", "prefill-skewed-28l", "decode-pool-28l"):
        nl = 28 if n_layers is None else n_layers
        if name == "decode-28l":
            n_adapters, cap = 64, 64
            ranks = {a: (8, 16, 32, 64)[(a - 1) // 16] for a in range(1, 65)}
            lengths = np.ones(256, dtype=np.int64)
            ids = rng.integers(1, 65, 256)
            gather = False
        elif name == "prefill-skewed-28l":
            n_adapters, cap = 128, 32
            ranks = {a: 32 for a in range(1, 129)}
            lengths = np.clip(np.rint(rng.lognormal(math.log(200.0), 1.0, 512)), 16, 2048).astype(np.int64)
            pop = np.arange(1, 129, dtype=np.float64) ** -1.1
            ids = rng.choice(128, 512, p=pop / pop.sum()) + 1
            gather = True
        else:
            n_adapters, cap = 1024, 64
            ranks = {a: 64 for a in range(1, 1025)}
            lengths = np.ones(4096, dtype=np.int64)
            ids = rng.integers(1, 1025, 4096)
            gather = False
        layers = _layers(nl, cap, gen, device)
        pool = AdapterPool([lin for layer in layers for lin in layer.values()], n_adapters, device)
        _fill_adapters(pool, ranks, gen, device)
    else:
        raise ValueError(f"unknown workload {name!r}")
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    ragged = not bool((lengths == 1).all())
    readout = None
    if gather:
        dim, rows = layers[-1]["down"].out, pool.lora_pool.shape[0]
        readout = {"readout_pool": (0.05 * torch.randn(rows, READOUT_OPTIONS, dim, generator=gen, device=device)).to(DT),
                   "temp_pool": 0.5 + 1.5 * torch.rand(rows, generator=gen, device=device),
                   "counts": torch.tensor(rng.integers(1, READOUT_OPTIONS + 1, len(lengths)).astype(np.int32),
                                          device=device)}
    return Workload(name=name, layers=layers, pool=pool,
                    adp=torch.tensor(ids.astype(np.int32), device=device),
                    cu_seqlens=torch.tensor(cu, device=device) if ragged else None,
                    tokens=int(cu[-1]), requests=len(lengths), lengths=lengths, adapter_ranks=ranks,
                    gather_last=gather, readout=readout, gated=name not in ("prefill-1layer", "cpu-1024"))


def inputs(w: Workload, label: str, gen: torch.Generator | None = None) -> torch.Tensor:
    """x ~ N(0, 1) bf16 (tokens, k) for the group `label`."""
    k = w.layers[0][label].k
    x = torch.empty(w.tokens, k, device=w.adp.device, dtype=torch.float32)
    x.normal_(generator=gen)
    return x.to(DT)


def token_ids(w: Workload) -> np.ndarray:
    """The pool row each original token reads (numpy, host)."""
    return np.repeat(w.adp.cpu().numpy(), w.lengths)


def flops_per_token(w: Workload) -> float:
    """Algorithmic FLOPs per token of one pass: base 2 k out plus LoRA 2 r (k + out_j) per adapted matrix, at the
    workload's mean live rank per token."""
    tok = token_ids(w)
    mean_rank = float(np.mean([w.adapter_ranks.get(int(a), 0) for a in tok])) if tok.size else 0.0
    total = 0.0
    for layer in w.layers:
        for lin in layer.values():
            total += 2.0 * lin.k * lin.out + sum(2.0 * mean_rank * (lin.k + n) for n in lin.sizes)
    return total


def hbm_bytes(w: Workload, gated: tuple[str, ...] = ()) -> float:
    """Algorithmic HBM bytes of one pass: INT4 codes, scales and zero points of every group once, activations in and
    out once, and the A and sB of every adapter present once (its live ranks only). Groups named in `gated` write
    silu(gate) * up, half their columns."""
    present = sorted({int(a) for a in token_ids(w)} - {0})
    total = 0.0
    for layer in w.layers:
        for label, lin in layer.items():
            total += lin.int4.nbytes() if lin.int4 is not None else 2.0 * lin.k * lin.out
            total += 2.0 * w.tokens * (lin.k + (lin.out // 2 if label in gated else lin.out))
            for a in present:
                r = w.adapter_ranks[a]
                total += sum(2.0 * min(r, c) * (lin.k + n) for n, c in zip(lin.sizes, lin.caps) if c)
    if w.gather_last:
        total += 2.0 * w.requests * w.layers[-1]["down"].out
    if w.readout is not None:
        total += readout_bytes(w)
    return total


def readout_bytes(w: Workload) -> float:
    """Algorithmic HBM bytes of the decision head: the readout of every adapter row present once, each request's
    hidden row in, its logits out and back in (float32) and its probabilities out (float32)."""
    pool = w.readout["readout_pool"]
    present = len({int(a) for a in w.adp.cpu().tolist()})
    options, dim = pool.shape[1], pool.shape[2]
    return 2.0 * present * options * dim + w.requests * (2.0 * dim + 3 * 4.0 * options)
