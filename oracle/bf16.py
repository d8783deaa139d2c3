"""float32 <-> bfloat16 on bit patterns, round to nearest even (test infrastructure; see oracle/__init__.py).

The reference rounds with torch's `.to(torch.bfloat16)` (`engine/int4.py:208`) and Triton's `.to(tl.bfloat16)`
(`engine/int4_kernels.py:59`); both are IEEE round-to-nearest-even. This restates that on the uint32 pattern."""

from __future__ import annotations

import numpy as np


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """uint16 bfloat16 patterns of float32 values, round to nearest even; NaN stays NaN (quiet)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    bias = ((u >> 16) & 1) + 0x7FFF
    rounded = ((u + bias) >> 16).astype(np.uint32)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    rounded = np.where(nan, ((u >> 16) | 0x40).astype(np.uint32), rounded)
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    """float32 values of uint16 bfloat16 patterns (exact)."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest bfloat16 (even on ties), as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))
