"""Adapter routing restated in numpy (test infrastructure; see oracle/__init__.py).

The reference routes token t to pool row adp[t // row_len] (`engine/fast_path.py:167,189`,
`engine/int4_kernels.py:72,113`): request rows of uniform length, one adapter index per row. The MI355X path sorts
the request rows by adapter index (stable), so each adapter's tokens form one contiguous segment of the sorted
order; ragged rows are given by cu_seqlens. This is the closed form the HIP routing kernel must equal bit for bit."""

from __future__ import annotations

import numpy as np

STATUS_BAD_ADAPTER = 1  # some adapter index lay outside [0, pool_rows); those rows were routed to row 0 (the base)


def route(adp: np.ndarray, pool_rows: int, row_len: int | None = None,
          cu_seqlens: np.ndarray | None = None) -> dict[str, np.ndarray | int]:
    """Stable segment sort of request rows by adapter index.

    adp int32 (B,); either row_len (every row has row_len tokens) or cu_seqlens int32 (B+1,) token offsets.
    Returns:
      req_order (B,)   request rows in sorted order (np.argsort kind="stable" of the adapter indices)
      tok_perm  (T,)   sorted token position -> original token index (each row's tokens stay in order)
      seg_start (S+1,) sorted token positions where each segment begins (and the end)
      seg_adapter (S,) the pool row of each segment, increasing; S = number of distinct adapters present
      last_of   (T,)   per sorted position: the request row whose last token sits there, else -1
      seg_of    (T,)   per sorted position: the segment it lies in
      status    int    STATUS_BAD_ADAPTER if an index was out of range (those rows use row 0)"""
    adp = np.asarray(adp, dtype=np.int64)
    b = adp.shape[0]
    if cu_seqlens is None:
        if row_len is None:
            raise ValueError("give row_len or cu_seqlens")
        cu = np.arange(b + 1, dtype=np.int64) * row_len
    else:
        cu = np.asarray(cu_seqlens, dtype=np.int64)
    bad = (adp < 0) | (adp >= pool_rows)
    status = STATUS_BAD_ADAPTER if bad.any() else 0
    ids = np.where(bad, 0, adp)
    order = np.argsort(ids, kind="stable")
    lengths = cu[1:] - cu[:-1]
    starts_sorted = np.concatenate([[0], np.cumsum(lengths[order])]).astype(np.int64)
    t = int(cu[-1]) if b else 0
    tok_perm = np.zeros(t, dtype=np.int64)
    last_of = np.full(t, -1, dtype=np.int64)
    for i, r in enumerate(order):
        n = int(lengths[r])
        tok_perm[starts_sorted[i]:starts_sorted[i] + n] = np.arange(cu[r], cu[r] + n)
        if n:
            last_of[starts_sorted[i] + n - 1] = r
    sorted_ids = ids[order]
    seg_adapter, first = np.unique(sorted_ids, return_index=True)  # ids are sorted: first index of each run
    seg_start = np.concatenate([starts_sorted[first], [t]]) if b else np.zeros(1, dtype=np.int64)
    return {"req_order": order.astype(np.int32), "tok_perm": tok_perm.astype(np.int32),
            "seg_start": seg_start.astype(np.int32), "seg_adapter": seg_adapter.astype(np.int32),
            "last_of": last_of.astype(np.int32),
            "seg_of": np.repeat(np.arange(seg_adapter.size), np.diff(seg_start)).astype(np.int32), "status": status}


def token_adapters(adp: np.ndarray, pool_rows: int, row_len: int | None = None,
                   cu_seqlens: np.ndarray | None = None) -> np.ndarray:
    """The pool row each original token reads: adp[t // row_len] (engine/fast_path.py:167) or, for ragged rows, the
    adapter of the row whose token range holds t. Out-of-range indices read row 0."""
    adp = np.asarray(adp, dtype=np.int64)
    ids = np.where((adp < 0) | (adp >= pool_rows), 0, adp)
    if cu_seqlens is None:
        return np.repeat(ids, row_len).astype(np.int32)
    lengths = np.diff(np.asarray(cu_seqlens, dtype=np.int64))
    return np.repeat(ids, lengths).astype(np.int32)
