"""The oracle's adapter routing (stable segment sort), pinned by invariants, by equality with the reference's
per-token rule adp[t // row_len] (engine/fast_path.py:167), and by brute force on tiny inputs."""

from __future__ import annotations

import itertools

import numpy as np

from oracle.routing import STATUS_BAD_ADAPTER, route, token_adapters


def check_invariants(adp, pool_rows, row_len=None, cu=None):
    r = route(adp, pool_rows, row_len=row_len, cu_seqlens=cu)
    tok_adp = token_adapters(adp, pool_rows, row_len=row_len, cu_seqlens=cu)
    t = tok_adp.size
    perm = r["tok_perm"]
    assert sorted(perm.tolist()) == list(range(t))                       # bijection
    sa, ss = r["seg_adapter"], r["seg_start"]
    assert ss[0] == 0 and ss[-1] == t and np.all(np.diff(ss) >= 0)       # coverage
    assert np.all(np.diff(sa) > 0)                                         # one segment per adapter, increasing
    for s in range(sa.size):
        assert np.all(tok_adp[perm[ss[s]:ss[s + 1]]] == sa[s])           # a segment holds one adapter's tokens
        assert np.all(np.diff(perm[ss[s]:ss[s + 1]]) > 0)                 # stable: original order kept
    assert set(sa.tolist()) >= set(tok_adp.tolist())
    so = r["seg_of"]                                                      # each position lies in its segment
    assert so.size == t and np.all(ss[so] <= np.arange(t)) and np.all(np.arange(t) < ss[so + 1])
    last = r["last_of"]
    lengths = np.diff(cu) if cu is not None else np.full(len(adp), row_len)
    ends = (np.cumsum(lengths) - 1)
    for req, n in enumerate(lengths):
        if n:
            p = int(np.nonzero(perm == ends[req])[0][0])
            assert last[p] == req
    assert (last >= 0).sum() == int((lengths > 0).sum())
    return r


def test_uniform_rows_match_the_reference_rule() -> None:
    rng = np.random.default_rng(0)
    for b, row_len, rows in [(4, 32, 5), (64, 1, 65), (256, 1, 65), (16, 8, 3), (1, 16, 2)]:
        adp = rng.integers(0, rows, b).astype(np.int32)
        r = check_invariants(adp, rows, row_len=row_len)
        ref = np.array([adp[t // row_len] for t in range(b * row_len)])
        # every sorted position reads the adapter the reference gives its original token
        seg_of = np.repeat(r["seg_adapter"], np.diff(r["seg_start"]))
        assert np.array_equal(seg_of, ref[r["tok_perm"]])


def test_ragged_zipf_and_empty_rows() -> None:
    rng = np.random.default_rng(1)
    for b in (1, 7, 512):
        lengths = rng.integers(0, 40, b)
        lengths[0] = 0
        cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
        ranks = np.arange(1, 129)
        p = ranks ** -1.1 / (ranks ** -1.1).sum()
        adp = (rng.choice(128, b, p=p) + 1).astype(np.int32)
        check_invariants(adp, 129, cu=cu)


def test_edge_cases() -> None:
    r = route(np.zeros(0, np.int32), 4, row_len=1)
    assert r["tok_perm"].size == 0 and r["seg_adapter"].size == 0 and list(r["seg_start"]) == [0]
    r = check_invariants(np.zeros(8, np.int32), 4, row_len=2)               # all base rows: one segment, row 0
    assert list(r["seg_adapter"]) == [0] and list(r["seg_start"]) == [0, 16]
    r = check_invariants(np.full(5, 3, np.int32), 4, row_len=3)             # a single adapter
    assert list(r["seg_adapter"]) == [3] and np.array_equal(r["tok_perm"], np.arange(15))
    r = route(np.array([1, 9, -1, 2], np.int32), 4, row_len=1)             # out of range -> row 0, flagged
    assert r["status"] == STATUS_BAD_ADAPTER and list(r["seg_adapter"]) == [0, 1, 2]
    assert list(r["tok_perm"]) == [1, 2, 0, 3]


def test_brute_force_tiny() -> None:
    """Every adapter assignment of up to 5 rows over 3 pool rows: the sorted order is the (adapter, row) order."""
    for b in range(1, 6):
        for adp in itertools.product(range(3), repeat=b):
            a = np.array(adp, np.int32)
            r = route(a, 3, row_len=1)
            want = sorted(range(b), key=lambda i: (adp[i], i))
            assert r["req_order"].tolist() == want and r["tok_perm"].tolist() == want
