"""The oracle's decision head, pinned on the CPU: logits against a per-element sum in exact rationals rounded by
Python and torch (not by the oracle's own bfloat16 helper), planted mistakes caught, and the softmax against closed
forms and torch's float32 softmax."""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle.readout import option_softmax, readout_exact, readout_logits, readout_rows


def small(seed: int, b: int = 4, options: int = 7, dim: int = 16, pool_rows: int = 3):
    g = torch.Generator().manual_seed(seed)
    hidden = torch.randn(b, dim, generator=g).to(torch.bfloat16)
    pool = (0.3 * torch.randn(pool_rows, options, dim, generator=g)).to(torch.bfloat16)
    adapters = torch.randint(0, pool_rows, (b,), generator=g, dtype=torch.int32)
    return hidden, pool, adapters


def bits(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.int16).numpy().view(np.uint16)


def per_element(hidden, pool, adapters) -> torch.Tensor:
    """Each logit summed in exact rationals, then rounded to float64 (Python), float32 and bfloat16 (torch)."""
    b, dim = hidden.shape
    options = pool.shape[1]
    out = torch.empty(b, options, dtype=torch.float64)
    for i in range(b):
        a = int(adapters[i])
        for o in range(options):
            s = sum(Fraction(float(pool[a, o, d])) * Fraction(float(hidden[i, d])) for d in range(dim))
            out[i, o] = float(s)
    return out.float().to(torch.bfloat16).float()


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_logits_equal_an_exact_per_element_sum(seed: int) -> None:
    hidden, pool, adapters = small(seed)
    got = readout_logits(bits(hidden), bits(pool), adapters.numpy())
    assert np.array_equal(got, per_element(hidden, pool, adapters).numpy())


def test_logits_catch_planted_mistakes() -> None:
    """Another adapter's readout and a transposed readout (options == dim) each change the logits."""
    hidden, pool, adapters = small(3, b=4, options=16, dim=16, pool_rows=3)
    adapters = torch.tensor([0, 1, 2, 1], dtype=torch.int32)
    want = per_element(hidden, pool, adapters).numpy()
    shifted = readout_logits(bits(hidden), bits(pool), ((adapters + 1) % 3).numpy())
    transposed = readout_logits(bits(hidden), bits(pool.transpose(1, 2).contiguous()), adapters.numpy())
    assert not np.array_equal(shifted, want)
    assert not np.array_equal(transposed, want)


def test_exact_sum_is_the_matrix_product_of_each_rows_readout() -> None:
    hidden, pool, adapters = small(4, b=6, options=9, dim=24)
    got = readout_exact(bits(hidden), bits(pool), adapters.numpy())
    want = torch.stack([pool[int(a)].double() @ hidden[i].double() for i, a in enumerate(adapters)])
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-14, atol=1e-14)


def test_softmax_closed_forms() -> None:
    options = 255
    rng = np.random.default_rng(0)
    logits = rng.standard_normal((4, options)).astype(np.float32)
    temps = np.array([1.0, 0.5, 2.0], dtype=np.float32)
    adapters = np.array([0, 1, 2, 0])
    # one option kept: probability 1 on it, 0 elsewhere
    p = option_softmax(logits, adapters, np.ones(4, dtype=np.int32), temps)
    assert np.array_equal(p[:, 0], np.ones(4)) and not p[:, 1:].any()
    # equal logits: 1 / count below the count, 0 from it on, whatever the temperature
    counts = np.array([1, 2, 100, 255])
    p = option_softmax(np.full((4, options), 3.0, np.float32), adapters, counts, temps)
    for i, c in enumerate(counts):
        np.testing.assert_allclose(p[i, :c], 1.0 / c, rtol=1e-12)
        assert not p[i, c:].any()
    # no option kept: every logit is the mask value -1e9, so the probabilities are uniform over all options
    p = option_softmax(logits, adapters, np.zeros(4, dtype=np.int32), temps)
    np.testing.assert_allclose(p, 1.0 / options, rtol=1e-12)
    # a temperature t is a division of the logits by t at temperature 1 (both divisions in float32)
    counts = np.array([10, 255, 1, 77])
    p = option_softmax(logits, adapters, counts, temps)
    scaled = np.where(np.arange(options)[None] < counts[:, None], logits, np.float32(-1e9)) / temps[adapters][:, None]
    q = option_softmax(scaled.astype(np.float32), np.zeros(4, dtype=np.int64), np.full(4, options), np.ones(1, np.float32))
    np.testing.assert_allclose(p, q, rtol=1e-12, atol=1e-300)
    np.testing.assert_allclose(p.sum(axis=1), 1.0, rtol=1e-12)


def test_softmax_matches_torch_float32_softmax() -> None:
    """tests/test_batched_kernels.py:413-416 restated in torch float32 on the CPU."""
    rng = np.random.default_rng(1)
    b, options = 16, 255
    logits = (3 * rng.standard_normal((b, options))).astype(np.float32)
    temps = (0.5 + 1.5 * rng.random(6)).astype(np.float32)
    adapters = rng.integers(0, 6, b)
    counts = np.concatenate([[1, 2, 255], rng.integers(1, 256, b - 3)])
    t = torch.from_numpy(logits)
    masked = t.masked_fill(torch.arange(options)[None] >= torch.from_numpy(counts)[:, None], -1e9)
    want = (masked / torch.from_numpy(temps)[torch.from_numpy(adapters)][:, None]).softmax(-1)
    got = option_softmax(logits, adapters, counts, temps)
    np.testing.assert_allclose(got, want.double().numpy(), rtol=1e-5, atol=1e-7)
    past = np.arange(options)[None] >= counts[:, None]
    assert not got[past].any()


def test_readout_rows_composes_the_two_steps() -> None:
    hidden, pool, adapters = small(5, b=5, options=11, dim=32, pool_rows=4)
    temps = np.array([1.0, 0.7, 1.9, 0.5], dtype=np.float32)
    counts = np.array([1, 11, 4, 7, 2])
    want = option_softmax(readout_logits(bits(hidden), bits(pool), adapters.numpy()), adapters.numpy(), counts, temps)
    assert np.array_equal(readout_rows(bits(hidden), bits(pool), temps, adapters.numpy(), counts), want)
