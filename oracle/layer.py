"""The reference's torch layer of the multi-LoRA INT4 linear, restated on the CPU (test infrastructure; see
oracle/__init__.py), plus the float64 exact result and the forward error bounds the HIP kernels are judged by.

A fused group (`engine/fast_path.py:301-349`) stacks J matrices that read the same input x (T, K) along the output:
matrix j has N_j outputs, base weights W_j = bf16((c - z) s) and, for the adapter of each token, a LoRA update
(A_j (r, K), sB_j (N_j, r)), sB = bf16(float(B) * alpha / r) (`engine/lora.py:204-210`).

- `layer_model`: `LoraLinear.forward` in "model" precision (`engine/lora.py:218-219`), applied to each adapter's
  segment of tokens as `AdapterSet.use` does per call (`engine/lora.py:328-337`): y = base(x), then
  y[seg] = addmm(y[seg], x[seg] @ A^T, (sB)^T), all in bfloat16 on the CPU. This is also the timed CPU baseline.
- `layer_float32`: "float32" precision (`engine/lora.py:220`): y + ((x.float() @ A^T) @ sB^T).to(bf16).
- `reference_f32`: everything in float32 without intermediate rounding: the fp32 reference of the rtol/atol check.
- `exact_and_bound`: float64 exact result from the same bfloat16 values and the forward error bound of a kernel that
  accumulates the base and the LoRA first factor in float32, rounds the first factor to bfloat16 (as the reference's
  kernels do: `engine/fast_path.py:196`, `engine/int4_kernels.py:120`), and rounds the output once. The quantities
  are those of `tests/test_int4_kernels_cuda.py:114-168` (u32 = 2^-23 a whole float32 unit, n = K + rank)."""

from __future__ import annotations

from collections.abc import Mapping, Sequence

import numpy as np
import torch

Update = tuple[torch.Tensor, torch.Tensor] | None  # (A (r, K) bf16, sB (N_j, r) bf16), or no update for matrix j
Adapters = Mapping[int, Sequence[Update]]          # pool row -> one entry per matrix of the group


def _segments(token_adp: np.ndarray) -> dict[int, np.ndarray]:
    return {int(a): np.nonzero(token_adp == a)[0] for a in np.unique(token_adp)}


def _col_ranges(cols: Sequence[int]) -> list[tuple[int, int]]:
    edges = np.concatenate([[0], np.cumsum(cols)]).astype(int)
    return [(int(edges[j]), int(edges[j + 1])) for j in range(len(cols))]


def layer_model(x: torch.Tensor, w: torch.Tensor, token_adp: np.ndarray, adapters: Adapters,
                cols: Sequence[int]) -> torch.Tensor:
    """engine/lora.py:212-219 ("model" precision) per matrix and per adapter segment; bf16 in, bf16 out (CPU)."""
    y = x @ w.T  # base(x): torch.nn.Linear without bias, in the weights' dtype
    for a, rows in _segments(token_adp).items():
        updates = adapters.get(a)
        if updates is None or len(rows) == 0:
            continue
        idx = torch.from_numpy(rows)
        xs = x.index_select(0, idx)
        for (o0, o1), upd in zip(_col_ranges(cols), updates, strict=True):
            if upd is None:
                continue
            a_mat, sb = upd
            y[idx, o0:o1] = torch.addmm(y[idx, o0:o1], xs @ a_mat.t(), sb.t())
    return y


def layer_float32(x: torch.Tensor, w: torch.Tensor, token_adp: np.ndarray, adapters: Adapters,
                  cols: Sequence[int]) -> torch.Tensor:
    """engine/lora.py:220 ("float32" precision): y + ((x.float() @ A^T) @ sB^T).to(y.dtype), per segment."""
    y = x @ w.T
    for a, rows in _segments(token_adp).items():
        updates = adapters.get(a)
        if updates is None or len(rows) == 0:
            continue
        idx = torch.from_numpy(rows)
        xs = x.index_select(0, idx).float()
        for (o0, o1), upd in zip(_col_ranges(cols), updates, strict=True):
            if upd is None:
                continue
            a_mat, sb = upd
            y[idx, o0:o1] = y[idx, o0:o1] + ((xs @ a_mat.float().t()) @ sb.float().t()).to(y.dtype)
    return y


def reference_f32(x: torch.Tensor, w: torch.Tensor, token_adp: np.ndarray, adapters: Adapters,
                  cols: Sequence[int]) -> torch.Tensor:
    """The fp32 reference: x W^T + (x A^T) sB^T from the same bfloat16 values, computed in float32, never rounded to
    bfloat16."""
    xf = x.float()
    y = xf @ w.float().T
    for a, rows in _segments(token_adp).items():
        updates = adapters.get(a)
        if updates is None or len(rows) == 0:
            continue
        idx = torch.from_numpy(rows)
        xs = xf.index_select(0, idx)
        for (o0, o1), upd in zip(_col_ranges(cols), updates, strict=True):
            if upd is None:
                continue
            a_mat, sb = upd
            y[idx, o0:o1] += (xs @ a_mat.float().t()) @ sb.float().t()
    return y


def step(v: torch.Tensor) -> torch.Tensor:
    """tests/test_int4_kernels_cuda.py:108-111: the bfloat16 unit in the last place at |v| (0 at 0)."""
    _, e = torch.frexp(v.abs())
    return torch.where(v == 0, torch.zeros_like(v), torch.ldexp(torch.ones_like(v), e - 8))


def exact_and_bound(x: torch.Tensor, w: torch.Tensor, token_adp: np.ndarray, adapters: Adapters,
                    cols: Sequence[int], rank_cap: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(exact float64 result, bound) per output; the bound of a single final rounding:
        |got - exact| <= slack + lora + step(|exact| + slack + lora) / 2,
    slack = (K + rank_cap) 2^-23 (|x| |W|^T + (|x| |A|^T) |sB|^T) (tests/test_int4_kernels_cuda.py:127-130,163),
    lora  = 2^-9 (|x A^T| |sB|^T) (tests/test_int4_kernels_cuda.py:131-133,162)."""
    xd = x.double()
    wd = w.double()
    exact = xd @ wd.T
    magnitude = xd.abs() @ wd.abs().T
    lora = torch.zeros_like(exact)
    for a, rows in _segments(token_adp).items():
        updates = adapters.get(a)
        if updates is None or len(rows) == 0:
            continue
        idx = torch.from_numpy(rows)
        xs = xd.index_select(0, idx)
        for (o0, o1), upd in zip(_col_ranges(cols), updates, strict=True):
            if upd is None:
                continue
            a_mat, sb = (t.double() for t in upd)
            mid = xs @ a_mat.T
            exact[idx, o0:o1] += mid @ sb.T
            magnitude[idx, o0:o1] += (xs.abs() @ a_mat.abs().T) @ sb.abs().T
            lora[idx, o0:o1] = 2.0 ** -9 * (mid.abs() @ sb.abs().T)
    slack = (x.shape[1] + rank_cap) * 2.0 ** -23 * magnitude
    before = slack + lora
    return exact, before + step(exact.abs() + before) / 2


def uncut_bound(x: torch.Tensor, w: torch.Tensor, exact: torch.Tensor, bound: torch.Tensor) -> torch.Tensor:
    """tests/test_int4_kernels_cuda.py:135-143,164-167: the bound of a product that rounds the base to bfloat16
    before adding the LoRA update (lora_add, and "model" precision): half a step of the rounded base plus the half
    step of the final rounding taken at an upper bound of the rounded value. `exact`, `bound` from exact_and_bound."""
    rounded_base = (x.double() @ w.double().T).to(torch.bfloat16).double()
    final_half = step(exact.abs()) / 2
    before = bound - final_half + step(rounded_base) / 2          # slack + lora + step(B) / 2 (up to the final half)
    return before + step(exact.abs() + before) / 2


def within_tolerance(got: torch.Tensor, ref32: torch.Tensor, rtol: float = 1e-2, atol: float = 2e-2) -> torch.Tensor:
    """The element-wise rtol/atol check of bf16 outputs against the fp32 reference: |got - ref| <= atol + rtol |ref|."""
    return (got.float() - ref32).abs() <= atol + rtol * ref32.abs()
