"""The decision head restated on the CPU (test infrastructure; see oracle/__init__.py).

Restates engine/batched_kernels.py:492-559 (`readout_logits`, `option_softmax`, `readout_rows`) and the softmax of
DecisionModel.forward that its tests hold the kernels to (tests/test_batched_kernels.py:399-437):
- logits[b, o] = bf16(float32(sum_d pool[adapters[b], o, d] * hidden[b, d])), the sum exact (float64: every product
  of two bfloat16 values is exact in float64 and the sums of at most 2048 of them are within float64 rounding of
  exact), rounded to float32 and then to bfloat16, as the reference's test forms its expected values
  (`bf(exact.float())`, tests/test_batched_kernels.py:430-431);
- probs[b] = softmax((o < counts[b] ? logits[b, o] : -1e9) / temp_pool[adapters[b]]) over all options, the mask and
  the division in float32 as torch does them, the softmax in float64 (tests/test_batched_kernels.py:413-416)."""

from __future__ import annotations

import numpy as np

from oracle.bf16 import bf16_bits_to_f32, round_to_bf16


def readout_exact(hidden_bits: np.ndarray, pool_bits: np.ndarray, adapters: np.ndarray) -> np.ndarray:
    """float64 (B, options): sum_d pool[adapters[b], o, d] * hidden[b, d], hidden uint16 bf16 bits (B, dim), pool
    uint16 bf16 bits (pool_rows, options, dim), adapters int (B) inside [0, pool_rows)."""
    h = bf16_bits_to_f32(hidden_bits).astype(np.float64)
    w = bf16_bits_to_f32(pool_bits).astype(np.float64)
    a = np.asarray(adapters, dtype=np.int64)
    return np.einsum("bd,bod->bo", h, w[a])


def readout_logits(hidden_bits: np.ndarray, pool_bits: np.ndarray, adapters: np.ndarray) -> np.ndarray:
    """engine/batched_kernels.py:492-504,522-536: float32 (B, options), the exact sum rounded to float32 and then to
    bfloat16 (tests/test_batched_kernels.py:430-431)."""
    return round_to_bf16(readout_exact(hidden_bits, pool_bits, adapters).astype(np.float32))


def option_softmax(logits: np.ndarray, adapters: np.ndarray, counts: np.ndarray, temp_pool: np.ndarray) -> np.ndarray:
    """engine/batched_kernels.py:507-519,539-553: float64 (B, options) probabilities; options from counts[b] on get
    the logit -1e9, then division by temp_pool[adapters[b]] (float32) and the softmax over all options."""
    logits = np.asarray(logits, dtype=np.float32)
    options = logits.shape[1]
    keep = np.arange(options)[None, :] < np.asarray(counts, dtype=np.int64)[:, None]
    masked = np.where(keep, logits, np.float32(-1e9)).astype(np.float32)
    t = np.asarray(temp_pool, dtype=np.float32)[np.asarray(adapters, dtype=np.int64)][:, None]
    x = (masked / t).astype(np.float64)
    e = np.exp(x - x.max(axis=1, keepdims=True))
    return e / e.sum(axis=1, keepdims=True)


def readout_rows(hidden_bits, pool_bits, temp_pool, adapters, counts) -> np.ndarray:
    """engine/batched_kernels.py:556-559: option_softmax of readout_logits."""
    return option_softmax(readout_logits(hidden_bits, pool_bits, adapters), adapters, counts, temp_pool)
