"""The decision head on the GPU, held to the reference's own readout tests (tests/test_batched_kernels.py:399-437)
with the oracle's logits and softmax as the expected values: each row reads its own adapter's readout and
temperature; logits within one bfloat16 step of the exact sum rounded to bfloat16 and at most 0.1% of them not equal;
probabilities within float32 rounding of the softmax of the kernel's own logits, zero past each row's count."""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from jeff_amd.readout import READOUT_ROWS, option_softmax, readout_logits, readout_rows
from oracle.readout import option_softmax as oracle_softmax
from oracle.readout import readout_logits as oracle_logits

pytestmark = pytest.mark.gpu

BATCHES = (1, 3, 16, 64)        # tests/test_batched_kernels.py:29
BF16_STEP = 2.0 ** -7           # one bfloat16 rounding step, relative to the value, at most


def readout_inputs(b: int, seed: int, dim: int = 1024, options: int = READOUT_ROWS, pool_rows: int = 6):
    """As tests/test_batched_kernels.py:399-409: six readouts (row 0 the base), temperatures from 0.5 to 2, each
    row's adapter and option count (1, 2, all, then random)."""
    gen = torch.Generator(device="cuda").manual_seed(seed)
    rng = random.Random(seed)
    counts = [1, 2, options] + [rng.randrange(1, options + 1) for _ in range(b)]
    return {"hidden": torch.randn(b, dim, device="cuda", generator=gen).to(torch.bfloat16),
            "readout_pool": (0.05 * torch.randn(pool_rows, options, dim, device="cuda", generator=gen)).to(
                torch.bfloat16),
            "temp_pool": 0.5 + 1.5 * torch.rand(pool_rows, device="cuda", generator=gen),
            "adapters": torch.tensor([rng.randrange(pool_rows) for _ in range(b)], device="cuda", dtype=torch.int32),
            "counts": torch.tensor(counts[:b], device="cuda", dtype=torch.int32)}


def bits(t: torch.Tensor) -> np.ndarray:
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def expected_logits(x) -> torch.Tensor:
    return torch.from_numpy(oracle_logits(bits(x["hidden"]), bits(x["readout_pool"]), x["adapters"].cpu().numpy()))


def expected_probs(logits: torch.Tensor, x) -> torch.Tensor:
    return torch.from_numpy(oracle_softmax(logits.cpu().numpy(), x["adapters"].cpu().numpy(),
                                           x["counts"].cpu().numpy(), x["temp_pool"].cpu().numpy())).float()


def check_logits(got: torch.Tensor, want: torch.Tensor) -> None:
    got = got.cpu()
    torch.testing.assert_close(got, want, rtol=BF16_STEP, atol=1e-6)
    assert int((got != want).sum()) <= max(1, 0.001 * got.numel())


def check_probs(probs: torch.Tensor, logits: torch.Tensor, x) -> None:
    probs = probs.cpu()
    torch.testing.assert_close(probs, expected_probs(logits, x), rtol=1e-5, atol=1e-7)
    past = torch.arange(probs.shape[1])[None] >= x["counts"].cpu()[:, None]
    assert not probs[past].any()


@pytest.mark.parametrize("b", BATCHES)
def test_readout_rows(b: int) -> None:
    x = readout_inputs(b, seed=b)
    print(f"readout rows={b} dim=1024 options={READOUT_ROWS}", flush=True)
    logits = readout_logits(x["hidden"], x["readout_pool"], x["adapters"])
    check_logits(logits, expected_logits(x))
    probs = readout_rows(x["hidden"], x["readout_pool"], x["temp_pool"], x["adapters"], x["counts"])
    check_probs(probs, logits, x)
    # torch's own float32 mask, temperature and softmax on the kernel's logits (tests/test_batched_kernels.py:413-416)
    masked = logits.masked_fill(torch.arange(READOUT_ROWS, device="cuda")[None] >= x["counts"][:, None].long(), -1e9)
    torch.testing.assert_close(probs, (masked / x["temp_pool"][x["adapters"].long()][:, None]).softmax(-1),
                               rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("b,dim,options", [(5, 8, 1), (7, 2048, 256), (33, 520, 63), (2, 64, 65), (200, 1024, 255)])
def test_readout_shapes(b: int, dim: int, options: int) -> None:
    """Hidden sizes from one 16-byte chunk to the largest, option counts at and either side of the 64-option block."""
    x = readout_inputs(b, seed=100 + b, dim=dim, options=options, pool_rows=3)
    print(f"readout rows={b} dim={dim} options={options}", flush=True)
    logits = readout_logits(x["hidden"], x["readout_pool"], x["adapters"])
    check_logits(logits, expected_logits(x))
    check_probs(option_softmax(logits, x["adapters"], x["counts"], x["temp_pool"]), logits, x)


def test_each_row_reads_its_own_adapter() -> None:
    """Rows that share a hidden vector but not an adapter get their own adapter's logits and temperature."""
    x = readout_inputs(6, seed=7)
    x["hidden"] = x["hidden"][:1].repeat(6, 1).contiguous()
    x["adapters"] = torch.arange(6, device="cuda", dtype=torch.int32)
    x["counts"] = torch.full((6,), READOUT_ROWS, device="cuda", dtype=torch.int32)
    logits = readout_logits(x["hidden"], x["readout_pool"], x["adapters"])
    for a in range(6):
        alone = readout_logits(x["hidden"][:1], x["readout_pool"], x["adapters"][a:a + 1])
        assert torch.equal(logits[a], alone[0])
    assert len({tuple(row.tolist()) for row in logits.cpu()}) == 6
    probs = readout_rows(x["hidden"], x["readout_pool"], x["temp_pool"], x["adapters"], x["counts"])
    check_probs(probs, logits, x)


def test_adapter_outside_the_pool_reads_row_zero() -> None:
    """An adapter index outside [0, pool_rows) reads the base row (0) and its temperature: every read stays inside
    the pool."""
    x = readout_inputs(4, seed=9)
    x["adapters"] = torch.tensor([-1, 6, 1 << 30, 0], device="cuda", dtype=torch.int32)
    probs = readout_rows(x["hidden"], x["readout_pool"], x["temp_pool"], x["adapters"], x["counts"])
    x0 = dict(x, adapters=torch.zeros(4, device="cuda", dtype=torch.int32))
    assert torch.equal(probs, readout_rows(x0["hidden"], x0["readout_pool"], x0["temp_pool"], x0["adapters"],
                                           x0["counts"]))


def test_readout_is_deterministic_and_replays_in_a_graph() -> None:
    """The same inputs give the same bits, eagerly and in every replay of a captured graph (the reference calls
    readout_rows inside its recorded decode graph, engine/batched_path.py:276)."""
    x = readout_inputs(64, seed=11)
    args = (x["hidden"], x["readout_pool"], x["temp_pool"], x["adapters"], x["counts"])
    eager = readout_rows(*args)
    assert torch.equal(eager, readout_rows(*args))
    readout_rows(*args)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = readout_rows(*args)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        assert torch.equal(readout_rows(*args), eager)


def test_readout_refuses_bad_arguments() -> None:
    """tests/test_batched_kernels.py:492-494, plus the library's own limits: ValueError before any launch."""
    x = readout_inputs(1, seed=1)
    with pytest.raises(ValueError, match="temp_pool"):
        readout_rows(x["hidden"], x["readout_pool"], x["temp_pool"].to(torch.bfloat16), x["adapters"], x["counts"])
    with pytest.raises(ValueError, match="adapters"):
        readout_logits(x["hidden"], x["readout_pool"], x["adapters"].long())
    with pytest.raises(ValueError, match="counts"):
        readout_rows(x["hidden"], x["readout_pool"], x["temp_pool"], x["adapters"], x["counts"][:0])
    with pytest.raises(ValueError, match="readout_pool"):
        readout_logits(x["hidden"], x["readout_pool"][:, :, :512].contiguous(), x["adapters"])
    with pytest.raises(ValueError, match="multiple of 8"):
        y = readout_inputs(1, seed=1, dim=12)
        readout_logits(y["hidden"], y["readout_pool"], y["adapters"])
    with pytest.raises(ValueError, match="multiple of 8"):
        y = readout_inputs(1, seed=1, dim=64, options=257)
        readout_logits(y["hidden"], y["readout_pool"], y["adapters"])
