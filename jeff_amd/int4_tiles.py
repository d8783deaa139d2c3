"""Which HIP kernels run an INT4 product of a given shape. The reference chooses Triton tiles here
(engine/int4_tiles.py:57-71); the MI355X library picks a kernel family instead, with the tiles inside each family
fixed for gfx950. The rule lives in the library alone (api.hip); int4_tiles asks it through mlora_int4_plan, a host-only
call that needs no GPU, so the kernel a benchmark names is the one the product runs.

- base: "gemv" (at most 8 tokens: one pass over the weights, every token dotted with each dequantised word), "mfma"
  (32x32x16 bf16 MFMA tiles, the LoRA second factor fused into the epilogue), "narrow" (few tokens per adapter
  segment and at most 256 tokens: one row tile of every token by 64 columns, the second factor fused, the input
  dimension split into float32 ranges only when the columns are too few for the CUs) or "split" (few tokens per
  segment, more tokens: MFMA tiles over ranges of the input dimension into float32 partials, then one epilogue
  workgroup per adapter segment and 256 columns).
- shrink (the LoRA first factor): "segment" when segments are short on average (decode: one workgroup per segment
  and 32 ranks of its adapter's A, the segment's rows as the second MFMA operand) or "mfma" when they are long
  (prefill: 32 sorted rows per workgroup on MFMA)."""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

from jeff_amd import _lib

BASES = ("gemv", "mfma", "split", "narrow")  # in the library's numbering (mlora_int4_plan *base)
SHRINKS = ("segment", "mfma")


@dataclass(frozen=True)
class Int4Tiles:
    base: str
    shrink: str
    ranges: int | None = None  # input ranges of a narrow product (1, 2, 4 or 8); None: the library's choice

    def flags(self) -> int:
        f = {"gemv": _lib.FORCE_BASE_GEMV, "mfma": _lib.FORCE_BASE_MFMA, "narrow": _lib.FORCE_BASE_NARROW,
             "split": _lib.FORCE_BASE_SPLIT}[self.base]
        f |= 0 if self.ranges is None else _lib.force_ranges(self.ranges)
        return f | (_lib.FORCE_SHRINK_SEGMENT if self.shrink == "segment" else _lib.FORCE_SHRINK_MFMA)


def int4_plan(columns: int, inputs: int, tokens: int, requests: int | None = None, pool_rows: int | None = None,
              rank_cap: int = 0, out: int | None = None, flags: int = 0) -> tuple[str, str, int]:
    """(base kernel, first-factor kernel, input ranges) the library runs for this shape; ValueError for a shape the
    kernels cannot run."""
    requests = tokens if requests is None else requests
    pool_rows = requests + 1 if pool_rows is None else pool_rows
    if columns <= 0 or columns % 64 or inputs <= 0 or inputs % 64 or tokens <= 0:
        raise ValueError(f"The INT4 kernels need columns and inputs that are positive multiples of 64 and at least one "
                         f"token; got {columns} columns, {inputs} inputs, {tokens} tokens")
    base, shrink, ranges = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    rc = _lib.lib().mlora_int4_plan(inputs, columns, columns if out is None else out, tokens, requests, pool_rows,
                                    rank_cap, flags, ctypes.byref(base), ctypes.byref(shrink), ctypes.byref(ranges))
    if rc != _lib.OK:
        raise ValueError(f"no INT4 kernel runs {tokens} tokens through {inputs} -> {columns} with flags {flags}: "
                         f"{_lib.ERRORS.get(rc, rc)}")
    return BASES[base.value], SHRINKS[shrink.value], ranges.value


def int4_tiles(columns: int, inputs: int, tokens: int, requests: int | None = None,
               pool_rows: int | None = None) -> Int4Tiles:
    """The kernels for `tokens` tokens in `requests` request rows through a group of `inputs` inputs and `columns`
    kernel columns (the library's choice); ValueError for a shape the kernels cannot run."""
    base, shrink, _ = int4_plan(columns, inputs, tokens, requests, pool_rows)
    return Int4Tiles(base, shrink)
