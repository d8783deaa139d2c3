"""The oracle's view of the device adapter pool and INT4 weights (test infrastructure; see oracle/__init__.py):
copies one fused group's adapters and weights back to the host in the form oracle.layer takes."""

from __future__ import annotations

import numpy as np
import torch

from oracle import codec


def adapters_of(lin, rows) -> dict:
    """{pool row: [(A (r, k), sB (out_j, r)) or None per matrix]} of a bound jeff_amd Lin, read from the device.
    The layout read here is the pool's: A (rank, k) at off_a with matrix j in rows rho_j.., then sB_j at off_bj[j],
    (out_j, s) with row stride s = the live rank r rounded up to a power of two, at least 8, at most cap_j; only the
    live ranks (the ranks table) are returned."""
    out = {}
    n = len(lin.names)
    for row in rows:
        row = int(row)
        if row == 0:
            continue
        ranks = lin.ranks_table[row, lin.rank_col:lin.rank_col + n].cpu().tolist()
        flat = lin.pool[row, lin.off_a:lin.off_a + lin.numel()].cpu()
        a_all = flat[:lin.rank * lin.k].view(lin.rank, lin.k)
        ups = []
        for j, (size, cap, r) in enumerate(zip(lin.sizes, lin.caps, ranks)):
            if r == 0:
                ups.append(None)
                continue
            start = lin.off_bj[j] - lin.off_a
            stride = min(max(8, 1 << (r - 1).bit_length()), cap)
            sb = flat[start:start + size * stride].view(size, stride)[:, :r].contiguous()
            ups.append((a_all[lin.rho[j]:lin.rho[j] + r].contiguous(), sb))
        out[row] = ups
    return out


def weights_of(packed) -> torch.Tensor:
    """The bf16 (out, k) weights bf16((c - z) s) of a jeff_amd KernelInt4, dequantised on the host by the oracle."""
    words = packed.words.cpu().numpy()
    scales = packed.scales.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
    zeros = None if packed.zeros is None else packed.zeros.cpu().numpy()
    bits = codec.dequantize_kernel(words, scales, zeros, packed.out, packed.group)
    return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
