"""Which HIP kernels run an INT4 product of a given shape (kept apart from the library so the rule can be checked
without a GPU). The reference chooses Triton tiles here (engine/int4_tiles.py:57-71); the MI355X kernels pick a
kernel family instead, and the tiles inside each family are fixed for gfx950.

- base: "gemv" (at most GEMV_MAX_TOKENS tokens: one pass over the weights, every token dotted with each dequantised
  word), "mfma" (32x32x16 bf16 MFMA tiles, the LoRA second factor fused into the epilogue), "narrow" (few tokens per
  adapter segment and at most NARROW_MAX_TOKENS tokens: one row tile of every token by 64 columns, the second factor
  fused, the input dimension split into float32 ranges only when the columns are too few for the CUs) or "split"
  (few tokens per segment, more tokens: MFMA tiles over ranges of the input dimension into float32 partials, then
  one epilogue workgroup per adapter segment and 256 columns).
- shrink (the LoRA first factor): "segment" when segments are short on average (decode: one workgroup per segment
  and 32 ranks of its adapter's A, the segment's rows as the second MFMA operand) or "mfma" when they are long
  (prefill: 32 sorted rows per workgroup on MFMA).
The library makes the same choice itself when no flag forces one (api.hip, shrink_on_mfma)."""

from __future__ import annotations

from dataclasses import dataclass

from jeff_amd import _lib

GEMV_MAX_TOKENS = 8
NARROW_MAX_TOKENS = 256
SHRINK_MFMA_MIN_TOKENS_PER_SEGMENT = 16
BASES = ("gemv", "mfma", "narrow", "split")
SHRINKS = ("segment", "mfma")


@dataclass(frozen=True)
class Int4Tiles:
    base: str
    shrink: str
    ranges: int | None = None  # a narrow product's input ranges (1, 2, 4 or 8); None: the library's choice

    def flags(self) -> int:
        f = {"gemv": _lib.FORCE_BASE_GEMV, "mfma": _lib.FORCE_BASE_MFMA, "narrow": _lib.FORCE_BASE_NARROW,
             "split": _lib.FORCE_BASE_SPLIT}[self.base]
        f |= 0 if self.ranges is None else _lib.force_ranges(self.ranges)
        return f | (_lib.FORCE_SHRINK_SEGMENT if self.shrink == "segment" else _lib.FORCE_SHRINK_MFMA)


def int4_tiles(columns: int, inputs: int, tokens: int, requests: int | None = None,
               pool_rows: int | None = None) -> Int4Tiles:
    """The kernels for `tokens` tokens in `requests` request rows through a group of `inputs` inputs and `columns`
    kernel columns; ValueError for a shape the kernels cannot run."""
    if columns <= 0 or columns % 64 or inputs <= 0 or inputs % 64 or tokens <= 0:
        raise ValueError(f"The INT4 kernels need columns and inputs that are positive multiples of 64 and at least one "
                         f"token; got {columns} columns, {inputs} inputs, {tokens} tokens")
    requests = tokens if requests is None else requests
    segs = max(1, min(requests, pool_rows if pool_rows is not None else requests))
    long_segments = tokens >= SHRINK_MFMA_MIN_TOKENS_PER_SEGMENT * segs
    base = ("gemv" if tokens <= GEMV_MAX_TOKENS else "mfma" if long_segments
            else "narrow" if tokens <= NARROW_MAX_TOKENS else "split")
    return Int4Tiles(base, "mfma" if long_segments else "segment")
