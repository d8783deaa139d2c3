"""The element-wise steps around the fused linear on the HIP library: residual add + RMSNorm, and SiLU(gate) * up.

Mirrors the reference's engine/fast_path.py:80-100 (`add_rms`), 141-156 (`silu_mul`) and 295-298 (`rms`, the
standard path's RMSNorm): same arguments, results and ValueError before any launch. `add_rms(x, d, w1)` returns
(x + d rounded to bf16, RMSNorm of it times w1 rounded to bf16); with d None it returns x itself and its norm.
`silu_mul(gu)` takes the gate_up product (gate half, then up half) and returns bf16(bf16(silu(g)) * u). The row
length of add_rms is at most 8192 and a multiple of 8; the gated width a multiple of 8."""

from __future__ import annotations

import torch

from jeff_amd import _lib

EPS = 1e-6  # engine/fast_path.py:58
DT = torch.bfloat16


def _check_rows(name: str, t: torch.Tensor, shape: tuple[int, ...] | None = None) -> None:
    if t.dim() != 2 or t.dtype != DT or t.stride(1) != 1 or t.device.type != "cuda":
        raise ValueError(f"{name}: expected a bfloat16 (rows, n) tensor on the GPU with unit column stride, got "
                         f"{t.dtype} {tuple(t.shape)} strides {tuple(t.stride())} on {t.device}")
    if shape is not None and tuple(t.shape) != shape:
        raise ValueError(f"{name}: expected shape {shape}, got {tuple(t.shape)}")


def add_rms(x: torch.Tensor, d: torch.Tensor | None, w1: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """engine/fast_path.py:93-100: x (M, N) bf16; d (M, N) bf16 or None; w1 = 1 + weight (N,) float32. Returns
    (x + d, rms(x + d) * w1), both bf16 (M, N); with d None the first is x itself."""
    _check_rows("add_rms x", x)
    m, n = x.shape
    if d is not None:
        _check_rows("add_rms d", d, (m, n))
    if w1.dim() != 1 or w1.shape[0] != n or w1.dtype != torch.float32 or not w1.is_contiguous():
        raise ValueError(f"add_rms: w1 must be a contiguous float32 vector of {n} values (1 + the norm's weight), got "
                         f"{w1.dtype} {tuple(w1.shape)}")
    if n % 8 or n > _lib.EPILOGUE_MAX_N:
        raise ValueError(f"add_rms: the row length must be a multiple of 8 up to {_lib.EPILOGUE_MAX_N}, got {n}")
    h = torch.empty(m, n, device=x.device, dtype=DT)
    xo = torch.empty(m, n, device=x.device, dtype=DT) if d is not None else x
    stream = torch.cuda.current_stream(x.device).cuda_stream
    _lib.check(_lib.lib().mlora_add_rms(x.data_ptr(), x.stride(0), d.data_ptr() if d is not None else None,
                                        d.stride(0) if d is not None else 0, w1.data_ptr(),
                                        xo.data_ptr() if d is not None else None, xo.stride(0), h.data_ptr(),
                                        h.stride(0), m, n, EPS, stream), "mlora_add_rms")
    return xo, h


def rms(x: torch.Tensor, w1: torch.Tensor) -> torch.Tensor:
    """engine/fast_path.py:295-298 on the library: the RMSNorm of each row of x times w1, bf16."""
    return add_rms(x, None, w1)[1]


def silu_mul(gu: torch.Tensor) -> torch.Tensor:
    """engine/fast_path.py:151-156: gu (rows, 2 inter) bf16, the gate half then the up half of the gate_up product.
    Returns bf16 (rows, inter) = bf16(bf16(g / (1 + exp(-g))) * u)."""
    _check_rows("silu_mul gu", gu)
    rows, width = gu.shape
    if width % 16:
        raise ValueError(f"silu_mul: the gate_up width must be twice a multiple of 8, got {width}")
    inter = width // 2
    y = torch.empty(rows, inter, device=gu.device, dtype=DT)
    stream = torch.cuda.current_stream(gu.device).cuda_stream
    _lib.check(_lib.lib().mlora_silu_mul(gu.data_ptr(), gu.stride(0), y.data_ptr(), y.stride(0), rows, inter, stream),
               "mlora_silu_mul")
    return y
