"""The element-wise steps around the fused linear restated on the CPU (test infrastructure; see oracle/__init__.py).

Restates engine/fast_path.py:80-100 (`_add_rms_kernel`, `add_rms`), 141-156 (`_silu_mul_kernel`, `silu_mul`) and the
standard path's RMSNorm (fast_path.py:295-298, `rms`):
- add_rms: x' = bf16(float32(x) + float32(d)) (an IEEE float32 addition, as the kernel adds), then
  h = x' rsqrt(mean(x'^2) + eps) w1 computed exactly (float64) and rounded to bfloat16 through float32;
- silu_mul: s = bf16(g / (1 + exp(-g))) with the quotient exact (float64) and rounded through float32, then
  y = bf16(s u) (the product of two bfloat16 values is exact in float64).
The kernels compute in float32 with their own summation order and exp; their results may differ from these in the
last bfloat16 place where the exact value lies within float32 rounding of a bfloat16 rounding boundary."""

from __future__ import annotations

import numpy as np

from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

EPS = 1e-6  # engine/fast_path.py:58


def add_rms(x_bits: np.ndarray, d_bits: np.ndarray | None, w1: np.ndarray, eps: float = EPS):
    """engine/fast_path.py:80-100: (x' bits uint16, h exact float64, h bits uint16) for rows of x (uint16 bf16 bits,
    (rows, n)), d (the same or None) and w1 float32 (n)."""
    x = bf16_bits_to_f32(x_bits)
    if d_bits is not None:
        xo_bits = f32_to_bf16_bits((x + bf16_bits_to_f32(d_bits)).astype(np.float32))
    else:
        xo_bits = np.asarray(x_bits, dtype=np.uint16)
    xo = bf16_bits_to_f32(xo_bits).astype(np.float64)
    r = 1.0 / np.sqrt((xo * xo).sum(axis=1, keepdims=True) / xo.shape[1] + float(np.float32(eps)))
    h = xo * r * np.asarray(w1, dtype=np.float64)[None, :]
    return xo_bits, h, f32_to_bf16_bits(h.astype(np.float32))


def silu_mul(gu_bits: np.ndarray):
    """engine/fast_path.py:141-156: (y exact float64 from the rounded SiLU, y bits uint16, s bits uint16) for the
    gate_up rows gu (uint16 bf16 bits, (rows, 2 inter))."""
    inter = gu_bits.shape[1] // 2
    g = bf16_bits_to_f32(gu_bits[:, :inter]).astype(np.float64)
    u = bf16_bits_to_f32(gu_bits[:, inter:]).astype(np.float64)
    with np.errstate(over="ignore"):
        s_exact = g / (1.0 + np.exp(-g))
    s_bits = f32_to_bf16_bits(s_exact.astype(np.float32))
    y = bf16_bits_to_f32(s_bits).astype(np.float64) * u
    return y, f32_to_bf16_bits(y.astype(np.float32)), s_bits
