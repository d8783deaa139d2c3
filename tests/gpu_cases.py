"""Helpers of the GPU parity tests: random fused groups with INT4 weights and a filled adapter pool, and the oracle's
view of the same data (test infrastructure)."""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from jeff_amd.fast_path import DT, AdapterPool, Lin, fold_scale
from jeff_amd.int4 import pack_kernel, pack_kernel_asym
from oracle import codec
from oracle.layer import exact_and_bound, reference_f32, within_tolerance
from oracle.pool_view import adapters_of
from oracle.routing import token_adapters


@dataclass
class Case:
    lin: Lin
    pool: AdapterPool
    codes: torch.Tensor       # uint8 (out, k), CPU
    scales: torch.Tensor      # bf16 (out, k/group), CPU
    zeros: torch.Tensor | None
    group: int
    w: torch.Tensor           # bf16 (out, k) dequantised by the oracle, CPU


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def make_case(sizes: list[int], k: int, group: int, asym: bool, adapter_ranks: dict[int, list[int]],
              caps: list[int], seed: int, max_adapters: int | None = None) -> Case:
    """A fused group of matrices `sizes` x k with random INT4 weights, and adapters {pool row: rank per matrix}."""
    g = torch.Generator().manual_seed(seed)
    out = sum(sizes)
    codes = torch.randint(0, 16, (out, k), generator=g, dtype=torch.uint8)
    scales = (torch.rand(out, k // group, generator=g) * 0.015 + 0.005).to(torch.bfloat16)
    zeros = torch.randint(0, 16, (out, k // group), generator=g, dtype=torch.uint8) if asym else None
    names = [f"layers.0.m{j}.q_proj" for j in range(len(sizes))]
    lin = Lin(names, sizes=sizes, k=k, ranks=caps)
    rows = max(adapter_ranks) if adapter_ranks else 1
    pool = AdapterPool([lin], max_adapters or rows)
    for row in range(1, rows + 1):
        ranks = adapter_ranks.get(row)
        if ranks is None:
            pool.add_adapter(f"empty-{row}", {})
            continue
        updates = {}
        for j, (name, n, r) in enumerate(zip(names, sizes, ranks)):
            if r == 0:
                continue
            a = (torch.randn(r, k, generator=g) / 32).to(DT)
            b = torch.randn(n, r, generator=g) * 0.02
            updates[name] = (a.cuda(), fold_scale(b, 2.0).cuda())
        assert pool.add_adapter(f"a{row}", updates) == row
    if asym:
        lin.int4 = pack_kernel_asym(codes.cuda(), scales.cuda(), zeros.cuda(), group)
    else:
        lin.int4 = pack_kernel((codes.to(torch.int16) - 8).to(torch.int8).cuda(), scales.cuda(), group)
    wbits = codec.dequantize(codes.numpy(), bf16_bits(scales), None if zeros is None else zeros.numpy(), group)
    w = torch.from_numpy(wbits.view(np.int16)).view(torch.bfloat16)
    return Case(lin, pool, codes, scales, zeros, group, w)


def oracle_adapters(lin: Lin, rows) -> dict:
    """{pool row: [(A (r, k), sB (out_j, r)) or None per matrix]} read back from the device pool."""
    return adapters_of(lin, rows)


def judge(lin: Lin, w: torch.Tensor, x: torch.Tensor, tok_adp: np.ndarray, got: torch.Tensor,
          rows: np.ndarray | None = None) -> dict:
    """The HIP output `got` against the oracle on the CPU, on all tokens or on the sampled `rows` (original token
    indices): within the forward error bound of exact arithmetic everywhere, and within rtol 1e-2 / atol 2e-2 of the
    fp32 reference. Returns the numbers (the caller asserts)."""
    if rows is not None:
        x = x[torch.as_tensor(rows, device=x.device)]
        got = got[torch.as_tensor(rows, device=got.device)]
        tok_adp = tok_adp[rows]
    xc, gc = x.cpu(), got.cpu()
    adapters = oracle_adapters(lin, np.unique(tok_adp))
    exact, bound = exact_and_bound(xc, w, tok_adp, adapters, lin.sizes, lin.rank)
    err = (gc.double() - exact).abs()
    ref32 = reference_f32(xc, w, tok_adp, adapters, lin.sizes)
    tol = within_tolerance(gc, ref32)
    return {"beyond_bound": int((err > bound).sum()), "worst_over_bound": float((err / bound).max()),
            "outside_tolerance": int((~tol).sum()), "finite": bool(torch.isfinite(gc.float()).all()),
            "max_abs_err": float(err.max()), "mean_abs_err": float(err.mean())}


def mean_abs_error(lin: Lin, w: torch.Tensor, x: torch.Tensor, tok_adp: np.ndarray,
                   got: torch.Tensor) -> float:
    """Mean absolute error of `got` against the float64 exact result (the reference's accuracy measure)."""
    adapters = oracle_adapters(lin, np.unique(tok_adp))
    exact, _ = exact_and_bound(x.cpu(), w, tok_adp, adapters, lin.sizes, lin.rank)
    return float((got.cpu().double() - exact).abs().mean())


def token_ids(adp: torch.Tensor, pool_rows: int, row_len: int | None = None,
              cu: torch.Tensor | None = None) -> np.ndarray:
    return token_adapters(adp.cpu().numpy(), pool_rows, row_len=row_len,
                          cu_seqlens=None if cu is None else cu.cpu().numpy())


def reference_f32_gpu(lin: Lin, w: torch.Tensor, x: torch.Tensor, tok_adp: np.ndarray) -> torch.Tensor:
    """oracle.layer.reference_f32 evaluated on the GPU, for the rtol/atol check of every row of a pass too large for
    the CPU: x W^T + (x A^T) sB^T from the same bfloat16 values in float32 (w: the oracle's dequantised (out, k)
    weights; the adapters read back from the pool as the oracle reads them)."""
    dev = x.device
    xf = x.float()
    y = xf @ w.to(dev).float().T.contiguous()
    edges = np.concatenate([[0], np.cumsum(lin.sizes)]).astype(int)
    for a, ups in oracle_adapters(lin, np.unique(tok_adp)).items():
        idx = torch.from_numpy(np.nonzero(tok_adp == a)[0]).to(dev)
        if idx.numel() == 0:
            continue
        xs = xf.index_select(0, idx)
        for j, upd in enumerate(ups):
            if upd is None:
                continue
            a_mat, sb = (t.to(dev).float() for t in upd)
            y[idx, int(edges[j]):int(edges[j + 1])] += (xs @ a_mat.T.contiguous()) @ sb.T.contiguous()
    return y
