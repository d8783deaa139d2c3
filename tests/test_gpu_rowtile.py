"""The row-tile product (64 sorted rows by 64, 128 or 192 columns per workgroup; each adapter segment's second factor
loaded with the input loop's steps and added in the same accumulators) against the CPU oracle on identical seeded
inputs, every output row: within the forward error bound of exact arithmetic and within rtol 1e-2 / atol 2e-2 of the
fp32 reference. Cases: the decode configuration's group shapes (mixed ranks 8..64, column blocks 1 and 3 per wave),
passes of several row tiles with segments crossing tile boundaries, more segments than input steps (the term of the
segments past the steps added after the loop), symmetric g64 weights, rank capacities of 32, a matrix without LoRA, a
partial last column tile, a single token; each request's last-token row gathered as well; repeated runs and a graph
replay give the same bits (needs a gfx950 GPU; marked gpu)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from jeff_amd import _lib
from jeff_amd.fast_path import DT, Workspace
from jeff_amd.int4_kernels import int4_product
from jeff_amd.int4_tiles import Int4Tiles, int4_plan
from tests.gpu_cases import judge, make_case, token_ids

pytestmark = pytest.mark.gpu

ROWTILE = Int4Tiles("rowtile", "segment")


@pytest.fixture(scope="module", autouse=True)
def gpu() -> None:
    assert torch.cuda.is_available(), "the gpu tests need an AMD GPU"
    _lib.lib()


def mixed(adapters: int, mats: int, caps: tuple[int, ...] = (64,)) -> dict[int, list[int]]:
    """Ranks 8, 16, 32, 64 in turn per adapter and matrix, each at most its matrix's capacity."""
    return {a: [min((8, 16, 32, 64)[(a - 1 + j) % 4], caps[j % len(caps)]) for j in range(mats)]
            for a in range(1, adapters + 1)}


CASES = {
    # name: (matrix widths, inputs, group, zero points, capacities, {adapter: ranks}, adapters drawn (0 = base too),
    #        tokens, tokens per request, column blocks per wave expected)
    "qkv-decode": ([2048, 1024, 1024], 2048, 128, True, [64] * 3, mixed(64, 3), 64, 256, 1, 1),
    "gate-up-decode": ([6144, 6144], 2048, 128, True, [64, 64], mixed(64, 2), 64, 256, 1, 3),
    "down-decode": ([2048], 6144, 128, True, [64], mixed(64, 1), 64, 256, 1, 1),
    "rows-crossing-tiles": ([768, 384], 1024, 128, True, [32, 64], mixed(40, 2, (32, 64)), 40, 1000, 4, 2),
    "more-segments-than-steps": ([256], 256, 64, True, [16], {a: [(8, 16)[a % 2]] for a in range(1, 121)}, 120, 120, 1,
                                 1),
    "symmetric-g64": ([512, 512], 1024, 64, False, [32, 32], mixed(20, 2, (32,)), 20, 300, 1, 1),
    "no-lora-matrix": ([64, 64, 128], 512, 128, True, [16, 0, 32], {1: [16, 0, 32], 2: [8, 0, 8], 3: [0, 0, 24]}, 3,
                       70, 1, 1),
    "partial-last-tile": ([96, 64], 256, 128, True, [32, 16], {a: [(8, 16, 24, 32)[a % 4], (16, 8)[a % 2]]
                                                               for a in range(1, 9)}, 8, 50, 1, 1),
    "one-token": ([128, 64], 128, 64, True, [16, 16], {1: [16, 16], 2: [8, 0]}, 2, 1, 1, 1),
    "base-rows-only": ([256], 512, 128, True, [32], {1: [32]}, 0, 64, 1, 1),
}


@pytest.mark.parametrize("name", list(CASES))
def test_rowtile_products_are_within_the_bound(name: str) -> None:
    sizes, k, group, asym, caps, ranks, drawn, tokens, row_len, nb = CASES[name]
    print(f"rowtile {name}", flush=True)
    case = make_case(sizes, k, group, asym, ranks, caps, len(name) * 31 + k)
    lin = case.lin
    requests = tokens // row_len
    rng = np.random.default_rng(tokens + k)
    if name == "more-segments-than-steps":
        ids = rng.permutation(np.arange(1, drawn + 1))  # every request its own adapter: 64 segments per row tile
    else:
        ids = rng.integers(0 if drawn else 0, drawn + 1, requests)
    adp = torch.tensor(ids.astype(np.int32), device="cuda")
    assert int4_plan(lin.int4.columns, k, tokens, requests, lin.pool.shape[0], lin.rank, lin.out,
                     ROWTILE.flags())[:1] == ("rowtile",)
    x = torch.randn(tokens, k, device="cuda").to(DT)
    ws = Workspace(tokens, row_len, max_rank=lin.rank, max_requests=requests)
    last = torch.zeros(requests, lin.out, dtype=DT, device="cuda")
    got = int4_product(lin, x, ws, adp, tiles=ROWTILE, last_out=last)
    assert torch.equal(last, got[row_len - 1::row_len])
    r = judge(lin, case.w, x, token_ids(adp, lin.pool.shape[0], row_len=row_len), got)
    assert r["finite"] and r["beyond_bound"] == 0 and r["outside_tolerance"] == 0, r
    if name in ("qkv-decode", "gate-up-decode"):
        # the column blocks the library picks for the decode groups
        from jeff_amd.int4_tiles import int4_plan as plan
        assert plan(lin.int4.columns, k, tokens, requests, lin.pool.shape[0], lin.rank, lin.out,
                    ROWTILE.flags())[2] == nb


def test_ragged_requests_with_empty_ones() -> None:
    """Requests of no tokens make empty segments: 200 requests with their own adapters, the odd ones one token, the
    even ones none, so 64 sorted rows span 127 segment indices (more than a wave holds one per lane, more than the 4
    input steps)."""
    n = 200
    ranks = {a: [(8, 16, 24, 32)[a % 4], (16, 8)[a % 2]] for a in range(1, n + 1)}
    case = make_case([96, 64], 256, 128, True, ranks, [32, 16], 17)
    lin = case.lin
    rng = np.random.default_rng(4)
    ids = rng.permutation(np.arange(1, n + 1)).astype(np.int32)
    lengths = (ids % 2).astype(np.int64)
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    tokens = int(cu[-1])
    adp = torch.tensor(ids, device="cuda")
    cu_d = torch.tensor(cu, device="cuda")
    x = torch.randn(tokens, lin.k, device="cuda").to(DT)
    ws = Workspace(tokens, 1, max_rank=lin.rank, max_requests=n)
    ws.route(adp, lin.pool.shape[0], tokens=tokens, cu_seqlens=cu_d)
    got = int4_product(lin, x, ws, adp, tiles=ROWTILE)
    ws.check()
    r = judge(lin, case.w, x, token_ids(adp, lin.pool.shape[0], cu=cu_d), got)
    assert r["finite"] and r["beyond_bound"] == 0 and r["outside_tolerance"] == 0, r


def test_rowtile_runs_and_replays_give_the_same_bits() -> None:
    case = make_case([512, 256], 1024, 128, True, mixed(16, 2, (64, 32)), [64, 32], 23)
    lin = case.lin
    for tokens in (256, 700):
        adp = torch.tensor(np.random.default_rng(tokens).integers(0, 17, tokens).astype(np.int32), device="cuda")
        x = torch.randn(tokens, lin.k, device="cuda").to(DT)
        ws = Workspace(tokens, 1, max_rank=lin.rank)
        first = int4_product(lin, x, ws, adp, tiles=ROWTILE)
        assert torch.equal(first, int4_product(lin, x, ws, adp, tiles=ROWTILE))
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            int4_product(lin, x, ws, adp, tiles=ROWTILE)
        torch.cuda.current_stream().wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = int4_product(lin, x, ws, adp, tiles=ROWTILE)
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, first)
            _ = x.float().sum().item()


def test_rowtile_refusals() -> None:
    """Widths the 16-column wave blocks cannot cut and capacities above 64 are refused when forced, before any
    launch; unforced, such groups take the other kernels."""
    case = make_case([40, 24], 256, 128, True, {1: [16, 8]}, [16, 8], 3)
    x = torch.randn(8, 256, device="cuda").to(DT)
    adp = torch.ones(8, dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="does not run"):
        int4_product(case.lin, x, Workspace(8, 1, max_rank=case.lin.rank), adp, tiles=ROWTILE)
    big = make_case([128], 256, 128, True, {1: [72]}, [72], 4)
    with pytest.raises(RuntimeError, match="does not run"):
        int4_product(big.lin, x, Workspace(8, 1, max_rank=big.lin.rank), adp, tiles=ROWTILE)
    got = int4_product(big.lin, x, Workspace(8, 1, max_rank=big.lin.rank), adp)
    r = judge(big.lin, big.w, x, token_ids(adp, big.lin.pool.shape[0], row_len=1), got)
    assert r["finite"] and r["beyond_bound"] == 0 and r["outside_tolerance"] == 0, r
