"""mlora_int4_linear_noalloc, the entry point with its scratch inside the library, against mlora_int4_linear with a
caller's workspace (needs a gfx950 GPU; marked gpu). Both run the same kernels in the same order, so their outputs
must be equal bit for bit: two calls in a row (the second on a smaller pass, over the scratch the first one left),
a replay of a recorded pass, and a pass too large for the scratch refused before any launch."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from jeff_amd import _lib
from jeff_amd.fast_path import DT, Workspace
from jeff_amd.int4_kernels import int4_product
from jeff_amd.int4_tiles import Int4Tiles
from tests.gpu_cases import make_case

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu() -> None:
    assert torch.cuda.is_available(), "the gpu tests need an AMD GPU"
    _lib.lib()


def noalloc(lin, x: torch.Tensor, ws: Workspace, adp: torch.Tensor, y: torch.Tensor, tiles=None,
            last: torch.Tensor | None = None) -> int:
    """One product through the C ABI's no-allocation entry point (the route from the workspace, as int4_product
    takes it); returns the status."""
    r = ws.routed(adp, lin.pool.shape[0], x.shape[0])
    stream = torch.cuda.current_stream().cuda_stream
    return _lib.lib().mlora_int4_linear_noalloc(lin.int4.abi(), lin.lora_abi(), r, x.data_ptr(), x.stride(0),
                                                y.data_ptr(), y.stride(0), 0 if last is None else last.data_ptr(),
                                                0 if tiles is None else tiles.flags(), stream)


def qkv_case():
    """A qkv-shaped group (2048 -> 2048 + 1024 + 1024, g128 asymmetric), 64 adapters of ranks 8/16/32/64."""
    ranks = {a: [(8, 16, 32, 64)[(a - 1) // 16]] * 3 for a in range(1, 65)}
    return make_case([2048, 1024, 1024], 2048, 128, True, ranks, [64, 64, 64], 31)


def test_two_calls_in_a_row_equal_the_workspace_entry_point() -> None:
    case = qkv_case()
    lin = case.lin
    rng = np.random.default_rng(12)
    # first: a decode pass of 256 one-token rows (the narrow product over input ranges: first factors and float32
    # partials in the scratch); second: 96 rows, each request 1 or 0 tokens, over what the first left there
    for tokens, requests, tiles in ((256, 256, None), (96, 160, Int4Tiles("narrow", "segment", 2))):
        adp = torch.tensor(rng.integers(0, 65, requests).astype(np.int32), device="cuda")
        lengths = np.ones(requests, dtype=np.int64) if tokens == requests else np.zeros(requests, dtype=np.int64)
        if tokens != requests:
            lengths[rng.choice(requests, tokens, replace=False)] = 1
        cu = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32), device="cuda")
        x = torch.randn(tokens, lin.k, device="cuda").to(DT)
        ws = Workspace(tokens, 1, max_rank=lin.rank, max_requests=requests)
        ws.route(adp, lin.pool.shape[0], tokens=tokens, cu_seqlens=cu)
        last_ref = torch.zeros(requests, lin.out, dtype=DT, device="cuda")
        want = int4_product(lin, x, ws, adp, tiles=tiles, last_out=last_ref)
        got = torch.full((tokens, lin.out), float("nan"), dtype=DT, device="cuda")
        last = torch.zeros(requests, lin.out, dtype=DT, device="cuda")
        assert noalloc(lin, x, ws, adp, got, tiles, last) == _lib.OK
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{tokens} tokens: the outputs differ"
        assert torch.equal(last, last_ref), f"{tokens} tokens: the gathered rows differ"
        assert bool(torch.isfinite(got.float()).all())


def test_a_recorded_pass_replays_with_new_ids() -> None:
    """A prefill-sized pass (long segments: the fused MFMA product, first factors in the scratch) recorded as a
    graph and replayed after new adapter ids are copied in, against the workspace entry point run eagerly."""
    case = make_case([512, 256], 1024, 128, True, {a: [16, 8] for a in range(1, 9)}, [16, 16], 5)
    lin = case.lin
    rows, row_len = 16, 64
    adp = torch.zeros(rows, dtype=torch.int32, device="cuda")
    x = torch.randn(rows * row_len, lin.k, device="cuda").to(DT)
    ws = Workspace(rows * row_len, row_len, max_rank=lin.rank)
    y = torch.empty(rows * row_len, lin.out, dtype=DT, device="cuda")
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(2):
            assert noalloc(lin, x, ws, adp, y) == _lib.OK
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        noalloc(lin, x, ws, adp, y)
    rng = np.random.default_rng(3)
    for _ in range(3):
        adp.copy_(torch.tensor(rng.integers(0, 9, rows).astype(np.int32)))
        graph.replay()
        torch.cuda.synchronize()
        want = int4_product(lin, x, Workspace(rows * row_len, row_len, max_rank=lin.rank), adp)
        assert torch.equal(y, want)


def test_a_pass_larger_than_the_scratch_is_refused() -> None:
    """A split product of 4096 tokens over 12288 columns needs far more float32 partials than the scratch holds:
    MLORA_EWORKSPACE, and the output is left untouched."""
    case = make_case([6144, 6144], 2048, 128, True, {a: [8, 8] for a in range(1, 5)}, [8, 8], 8)
    lin = case.lin
    tokens = 4096
    adp = torch.tensor(np.random.default_rng(1).integers(0, 5, tokens).astype(np.int32), device="cuda")
    x = torch.zeros(tokens, lin.k, device="cuda", dtype=DT)
    ws = Workspace(tokens, 1, max_rank=lin.rank)
    h = _lib.lib()
    need = h.mlora_int4_partials_bytes(lin.int4.abi(), lin.lora_abi(), ws.routed(adp, lin.pool.shape[0], tokens),
                                       _lib.FORCE_BASE_SPLIT | _lib.FORCE_SHRINK_SEGMENT)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    y = torch.full((tokens, lin.out), 7.0, dtype=DT, device="cuda")
    assert noalloc(lin, x, ws, adp, y, Int4Tiles("split", "segment")) == _lib.EWORKSPACE
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())
