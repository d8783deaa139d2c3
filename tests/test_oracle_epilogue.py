"""The oracle's residual add + RMSNorm and SiLU(gate) * up, pinned on the CPU against torch's own float32 arithmetic
(the reference's standard-path RMSNorm formula, engine/fast_path.py:295-298), torch's float64 silu, closed forms, and
planted mistakes."""

from __future__ import annotations

import numpy as np
import torch

from oracle.epilogue import EPS, add_rms, silu_mul

BF16_STEP = 2.0 ** -7


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16)


def case(rows: int, n: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    x = (3 * torch.randn(rows, n, generator=g)).to(torch.bfloat16)
    d = torch.randn(rows, n, generator=g).to(torch.bfloat16)
    w1 = (1 + 0.1 * torch.randn(n, generator=g)).float()
    return x, d, w1


def torch_rms(x: torch.Tensor, w1: torch.Tensor) -> torch.Tensor:
    """engine/fast_path.py:295-298 in torch float32 on the CPU."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + EPS) * w1).to(x.dtype)


def test_residual_add_is_torchs_float32_addition_rounded() -> None:
    x, d, w1 = case(16, 1024, 0)
    xo_bits, _, _ = add_rms(bits(x), bits(d), w1.numpy())
    assert torch.equal(from_bits(xo_bits), (x.float() + d.float()).to(torch.bfloat16))
    xo_bits, _, _ = add_rms(bits(x), None, w1.numpy())
    assert np.array_equal(xo_bits, bits(x))


def test_norm_matches_the_reference_formula_in_torch_float32() -> None:
    for rows, n, seed in [(64, 1024, 1), (8, 2048, 2), (3, 8, 3)]:
        x, d, w1 = case(rows, n, seed)
        xo = (x.float() + d.float()).to(torch.bfloat16)
        _, h_exact, h_bits = add_rms(bits(x), bits(d), w1.numpy())
        want = torch_rms(xo, w1)
        got = from_bits(h_bits)
        torch.testing.assert_close(got.float(), want.float(), rtol=BF16_STEP, atol=1e-6)
        assert (got != want).float().mean() < 0.01
        np.testing.assert_allclose(h_exact, want.double().numpy(), rtol=2 ** -8, atol=1e-6)


def test_norm_closed_forms() -> None:
    n = 64
    w1 = np.full(n, 1.5, dtype=np.float32)
    for c in (3.0, -0.25, 100.0):
        x = torch.full((1, n), c).to(torch.bfloat16)
        _, h, _ = add_rms(bits(x), None, w1)
        np.testing.assert_allclose(h, np.sign(c) * 1.5 / np.sqrt(1 + float(np.float32(EPS)) / c ** 2), rtol=1e-12)
    _, h, hb = add_rms(bits(torch.zeros(2, n, dtype=torch.bfloat16)), None, w1)
    assert not h.any() and not hb.any()


def test_norm_catches_planted_mistakes() -> None:
    """No eps, a mean over n - 1, and a missing w1 each move the result by more than a bfloat16 step somewhere."""
    x = (1e-3 * torch.randn(4, 16, generator=torch.Generator().manual_seed(5))).to(torch.bfloat16)
    w1 = np.linspace(0.5, 1.5, 16).astype(np.float32)
    _, h, _ = add_rms(bits(x), None, w1)
    xo = x.double().numpy()
    ms = (xo * xo).mean(axis=1, keepdims=True)
    no_eps = xo / np.sqrt(ms) * w1
    n_minus_1 = xo / np.sqrt((xo * xo).sum(axis=1, keepdims=True) / 15 + EPS) * w1
    no_w1 = xo / np.sqrt(ms + EPS)
    for wrong in (no_eps, n_minus_1, no_w1):
        assert np.abs(wrong - h).max() > BF16_STEP * np.abs(h).max()


def test_silu_matches_torch_float64() -> None:
    g = torch.Generator().manual_seed(7)
    gu = (4 * torch.randn(32, 256, generator=g)).to(torch.bfloat16)
    y, y_bits, s_bits = silu_mul(bits(gu))
    gate, up = gu[:, :128].double(), gu[:, 128:].double()
    s = torch.nn.functional.silu(gate).float().to(torch.bfloat16)
    assert torch.equal(from_bits(s_bits), s)
    assert torch.equal(from_bits(y_bits), (s.float() * up.float()).to(torch.bfloat16))
    np.testing.assert_array_equal(y, s.double().numpy() * up.numpy())


def test_silu_limits() -> None:
    vals = torch.tensor([[0.0, 40.0, -40.0, 1.0, 0.0, 1.0, 1.0, -1.0]]).to(torch.bfloat16)  # gates, then ups
    _, y_bits, s_bits = silu_mul(bits(vals))
    s = from_bits(s_bits).float()[0]
    assert s[0] == 0 and s[1] == 40.0 and abs(float(s[2])) < 1e-15
    np.testing.assert_allclose(float(s[3]), 1 / (1 + np.exp(-1.0)), rtol=BF16_STEP)
    assert float(from_bits(y_bits).float()[0, 3]) == -float(s[3])
