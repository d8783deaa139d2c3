"""Routing under the reference's own call patterns (needs a gfx950 GPU; marked gpu).

The reference records each pass once and replays it for every batch (engine/batched_path.py:383-398: the inputs
filled, two warm-up runs of the pass on the recording stream outside the capture, then the capture; each batch then
copies its rows' adapter ids into the same input tensor and replays, :589-603). The products must route the ids the
replay finds, not the ones the warm-up saw. Each replay here, with new adapter ids (and, for ragged rows, new
sequence lengths) copied into the captured tensors, is checked against the oracle on every output row and against
an eager run of the same inputs bit for bit. Also: passes over temporary adp tensors in a row on one workspace, whose
storage the allocator may hand from one to the next."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from jeff_amd import _lib
from jeff_amd.fast_path import DT, Workspace
from jeff_amd.int4_kernels import int4_product
from jeff_amd.int4_tiles import Int4Tiles
from tests.gpu_cases import judge, make_case, token_ids

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu() -> None:
    assert torch.cuda.is_available(), "the gpu tests need an AMD GPU"
    _lib.lib()


def group_case(seed: int):
    """Two fused groups reading the same input (a pass's products share its route), 6 adapters of mixed ranks."""
    ranks = {1: [16, 8], 2: [8, 16], 3: [16, 16], 4: [0, 8], 5: [16, 0], 6: [8, 8]}
    return [make_case([320, 192], 512, 128, True, ranks, [16, 16], seed),
            make_case([256], 512, 64, False, {a: [16] for a in range(1, 7)}, [16], seed + 1)]


@pytest.mark.parametrize("kind", ["uniform-decode", "uniform-prefill", "ragged-prefill", "ragged-narrow"])
def test_capture_after_warm_up_then_replay_new_ids(kind: str) -> None:
    cases = group_case(len(kind))
    pool_rows = cases[0].lin.pool.shape[0]
    assert all(c.lin.pool.shape[0] == pool_rows for c in cases)
    rng = np.random.default_rng(len(kind) * 13)
    ragged = kind.startswith("ragged")
    if kind == "uniform-decode":
        requests, row_len = 64, 1
    elif kind == "uniform-prefill":
        requests, row_len = 8, 64
    else:
        requests, row_len = 24 if kind == "ragged-prefill" else 96, 1
    tokens = 640 if kind == "ragged-prefill" else (96 if kind == "ragged-narrow" else requests * row_len)

    def lengths() -> np.ndarray:  # ragged lengths summing to `tokens`, some requests empty
        cuts = np.sort(rng.choice(np.arange(tokens + 1), requests - 1, replace=True))
        return np.diff(np.concatenate([[0], cuts, [tokens]]))

    # the pass's input tensors, filled as the reference fills them before recording (batched_path.py:383-388)
    adp = torch.zeros(requests, dtype=torch.int32, device="cuda")
    cu = torch.zeros(requests + 1, dtype=torch.int32, device="cuda")
    cu.copy_(torch.arange(requests + 1, dtype=torch.int32) * (tokens // requests))
    cu[-1] = tokens
    x = torch.zeros(tokens, 512, device="cuda", dtype=DT)
    ws = Workspace(tokens, 1 if ragged else row_len, max_rank=32, max_requests=requests)
    tiles = Int4Tiles("narrow", "segment") if kind in ("uniform-decode", "ragged-narrow") else None

    def body() -> list[torch.Tensor]:
        if ragged:
            ws.route(adp, pool_rows, tokens=tokens, cu_seqlens=cu)
        return [int4_product(c.lin, x, ws, adp, tiles=tiles) for c in cases]

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(2):  # warm up outside the capture (batched_path.py:392-395)
            body()
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        outs = body()

    for batch in range(3):
        ids = rng.integers(0, pool_rows, requests).astype(np.int32)
        adp.copy_(torch.from_numpy(ids))  # the new pass's rows, into the recorded tensors (batched_path.py:601)
        lens = lengths() if ragged else np.full(requests, row_len)
        cu_np = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        cu.copy_(torch.from_numpy(cu_np))
        x.copy_(torch.randn(tokens, 512, device="cuda").to(DT))
        graph.replay()
        torch.cuda.synchronize()
        tok = token_ids(adp, pool_rows, cu=cu) if ragged else token_ids(adp, pool_rows, row_len=row_len)
        eager_ws = Workspace(tokens, 1 if ragged else row_len, max_rank=32, max_requests=requests)
        for c, got in zip(cases, outs):
            r = judge(c.lin, c.w, x, tok, got)
            assert r["finite"] and r["beyond_bound"] == 0 and r["outside_tolerance"] == 0, (kind, batch, r)
            if ragged:
                eager_ws.route(adp, pool_rows, tokens=tokens, cu_seqlens=cu)
            eager = int4_product(c.lin, x, eager_ws, adp, tiles=tiles)
            assert torch.equal(eager, got), (kind, batch)
        _ = x.float().sum().item()  # eager work between replays


def test_temporary_adp_tensors_in_a_row() -> None:
    """Each pass builds its adp as a temporary, freed before the next one's is made (the allocator may give the next
    one the same storage): every product routes the ids it is given."""
    case = group_case(3)[0]
    lin = case.lin
    pool_rows = lin.pool.shape[0]
    x = torch.randn(256, lin.k, device="cuda").to(DT)
    ws = Workspace(256, 32, max_rank=lin.rank)
    rng = np.random.default_rng(9)
    for _ in range(4):
        ids = rng.integers(0, pool_rows, 8).astype(np.int32)
        got = int4_product(lin, x, ws, torch.tensor(ids, device="cuda"))
        torch.cuda.synchronize()
        r = judge(lin, case.w, x, np.repeat(ids, 32), got)
        assert r["finite"] and r["beyond_bound"] == 0 and r["outside_tolerance"] == 0, (ids, r)


class PoolOps:
    """Every PyTorch operation, seen from Python, that touches the storage of the adapter pool or its live-rank table
    (the reference's PoolWrites, tests/test_fast_path_cuda.py:138-166)."""

    def __init__(self, pool) -> None:
        self.storages = {t.untyped_storage().data_ptr() for t in (pool.lora_pool, pool.ranks)}
        self.seen: list[str] = []

    def __enter__(self) -> "PoolOps":
        from torch.utils._python_dispatch import TorchDispatchMode

        outer = self

        class Mode(TorchDispatchMode):
            def __torch_dispatch__(self, func, types, args=(), kwargs=None):
                leaves = torch.utils._pytree.tree_leaves((args, kwargs or {}))
                if any(isinstance(t, torch.Tensor) and t.untyped_storage().data_ptr() in outer.storages
                       for t in leaves):
                    outer.seen.append(str(func))
                return func(*args, **(kwargs or {}))

        self.mode = Mode()
        self.mode.__enter__()
        return self

    def __exit__(self, *exc) -> None:
        self.mode.__exit__(*exc)


def test_switching_adapter_touches_the_pool_with_no_pytorch_operation() -> None:
    """As the reference's test_switching_adapter_copies_no_weights (tests/test_fast_path_cuda.py:169-186): adding an
    adapter writes the pool (the spy sees it), while passes that switch adapter on every call, eagerly or as replays of
    a recorded pass, read it in place: no PyTorch operation touches the pool or its rank table."""
    ranks = {1: [16, 8], 2: [8, 16], 3: [16, 16], 4: [0, 8], 5: [16, 0], 6: [8, 8]}
    case = make_case([320, 192], 512, 128, True, ranks, [16, 16], 7, max_adapters=8)
    lin, pool = case.lin, case.pool
    x = torch.randn(64, lin.k, device="cuda").to(DT)
    ws = Workspace(64, 16, max_rank=lin.rank)
    adp = torch.zeros(4, dtype=torch.int32, device="cuda")
    g = torch.Generator().manual_seed(2)
    with PoolOps(pool) as adding:
        pool.add_adapter("late", {lin.names[0]: ((torch.randn(16, lin.k, generator=g) / 32).to(DT).cuda(),
                                                 (torch.randn(lin.sizes[0], 16, generator=g) * 0.02).to(DT).cuda())})
    assert any("copy_" in op for op in adding.seen), adding.seen  # the spy does see writes to the pool
    int4_product(lin, x, ws, adp)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        out = int4_product(lin, x, ws, adp)
    late = pool.index("late")
    with PoolOps(pool) as switching:
        for ids in ([1, 2, 3, 4], [late, 0, 6, late], [5, 5, 0, 2]):
            adp.copy_(torch.tensor(ids, dtype=torch.int32))
            graph.replay()
            eager = int4_product(lin, x, ws, adp)
            torch.cuda.synchronize()
            assert torch.equal(out, eager)
    assert switching.seen == [], switching.seen


def test_two_graphs_on_one_workspace_at_growing_sizes() -> None:
    """A workspace named no shapes, so its float32 partials grow with the products: a graph records a narrow product
    over eight input ranges on the first buffer, an eager product of a wider group then needs a larger one, a tensor
    is allocated after that growth, and a second graph records the wider product. The first graph keeps its buffer
    (the workspace never frees one a graph may hold), so replays of both graphs, new adapter ids each time, match the
    oracle on every row, and the tensor allocated after the growth is never written."""
    ranks = {a: [(8, 16)[a % 2]] for a in range(1, 7)}
    small = make_case([256], 1024, 128, True, ranks, [16], 91)
    wide = make_case([1024], 1024, 128, True, ranks, [16], 92)
    requests = 256
    tiles = Int4Tiles("narrow", "segment", 8)
    rng = np.random.default_rng(5)
    adp = torch.tensor(rng.integers(0, 7, requests).astype(np.int32), device="cuda")
    x = torch.randn(requests, 1024, device="cuda").to(DT)
    ws = Workspace(requests, 1, max_rank=16, max_requests=requests)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        int4_product(small.lin, x, ws, adp, tiles=tiles)
    stream.synchronize()
    g1 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g1, stream=stream):
        y1 = int4_product(small.lin, x, ws, adp, tiles=tiles)
    first = ws._part
    with torch.cuda.stream(stream):
        int4_product(wide.lin, x, ws, adp, tiles=tiles)  # grows the partials
    stream.synchronize()
    assert ws._part is not first and any(t is first for t in ws._retired)
    sentinel = torch.full((4 << 20,), 7.0, device="cuda")
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=stream):
        y2 = int4_product(wide.lin, x, ws, adp, tiles=tiles)
    pool_rows = small.lin.pool.shape[0]
    for rep in range(3):
        adp.copy_(torch.tensor(rng.integers(0, 7, requests).astype(np.int32), device="cuda"))
        x.copy_(torch.randn(requests, 1024, device="cuda").to(DT))
        g1.replay()
        g2.replay()
        torch.cuda.synchronize()
        tok = token_ids(adp, pool_rows, row_len=1)
        for case, y in ((small, y1), (wide, y2)):
            r = judge(case.lin, case.w, x, tok, y)
            assert r["beyond_bound"] == 0 and r["outside_tolerance"] == 0, f"replay {rep}: {r}"
        assert bool((sentinel == 7.0).all()), f"replay {rep} wrote into memory allocated after the growth"
