"""Residual add + RMSNorm and SiLU(gate) * up on the GPU against the oracle: x + d bit for bit; the norm and the
gated activation within one bfloat16 step of the exact result, equal to the oracle's rounding on all but the values
that lie within float32 rounding of a bfloat16 boundary (at most 0.5%), and within one step of the reference's
standard-path formula in torch (engine/fast_path.py:295-298)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from jeff_amd.epilogues import EPS, add_rms, rms, silu_mul
from oracle.epilogue import add_rms as oracle_add_rms
from oracle.epilogue import silu_mul as oracle_silu_mul

pytestmark = pytest.mark.gpu

BF16_STEP = 2.0 ** -7


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def from_bits(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16)


def case(rows: int, n: int, seed: int):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = (3 * torch.randn(rows, n, device="cuda", generator=g)).to(torch.bfloat16)
    d = torch.randn(rows, n, device="cuda", generator=g).to(torch.bfloat16)
    w1 = (1 + 0.1 * torch.randn(n, device="cuda", generator=g)).float()
    return x, d, w1


def check_close(got: torch.Tensor, exact: np.ndarray, rounded: np.ndarray, what: str) -> None:
    got = got.float().cpu()
    torch.testing.assert_close(got.double(), torch.from_numpy(exact), rtol=BF16_STEP, atol=1e-6, msg=what)
    unequal = int((got != from_bits(rounded).float()).sum())
    assert unequal <= max(1, 0.005 * got.numel()), f"{what}: {unequal} of {got.numel()} differ from the oracle"


@pytest.mark.parametrize("rows,n", [(1, 8), (256, 2048), (300, 1024), (7, 8192), (64, 520)])
def test_add_rms(rows: int, n: int) -> None:
    print(f"add_rms rows={rows} n={n}", flush=True)
    x, d, w1 = case(rows, n, rows + n)
    xo, h = add_rms(x, d, w1)
    xo_bits, h_exact, h_bits = oracle_add_rms(bits(x), bits(d), w1.cpu().numpy())
    assert np.array_equal(bits(xo), xo_bits)
    check_close(h, h_exact, h_bits, "add_rms h")
    xf = xo.float()  # the reference's standard-path RMSNorm in torch
    want = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + EPS) * w1).to(torch.bfloat16)
    torch.testing.assert_close(h.float(), want.float(), rtol=BF16_STEP, atol=1e-6)


def test_rms_without_residual_returns_x_itself() -> None:
    x, _, w1 = case(33, 2048, 3)
    xo, h = add_rms(x, None, w1)
    assert xo is x
    _, h_exact, h_bits = oracle_add_rms(bits(x), None, w1.cpu().numpy())
    check_close(h, h_exact, h_bits, "rms")
    assert torch.equal(rms(x, w1), h)


def test_add_rms_on_strided_rows_and_zero_rows() -> None:
    """Rows of a wider buffer (row stride above the row length), and all-zero rows (the norm of zero is zero)."""
    big = torch.randn(40, 4096, device="cuda").to(torch.bfloat16)
    x = big[:, :2048]
    x[5].zero_()
    d = torch.zeros(40, 2048, device="cuda", dtype=torch.bfloat16)
    w1 = torch.ones(2048, device="cuda")
    xo, h = add_rms(x, d, w1)
    assert torch.equal(xo, x) and not h[5].any()
    _, h_exact, h_bits = oracle_add_rms(bits(x), bits(d), w1.cpu().numpy())
    check_close(h, h_exact, h_bits, "strided add_rms")


@pytest.mark.parametrize("rows,inter", [(256, 6144), (3, 8), (1000, 3584)])
def test_silu_mul(rows: int, inter: int) -> None:
    print(f"silu_mul rows={rows} inter={inter}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(rows + inter)
    gu = (4 * torch.randn(rows, 2 * inter, device="cuda", generator=g)).to(torch.bfloat16)
    y = silu_mul(gu)
    y_exact, y_bits, _ = oracle_silu_mul(bits(gu))
    check_close(y, y_exact, y_bits, "silu_mul")
    # the reference's formula in torch float32 on the GPU
    gf, uf = gu[:, :inter].float(), gu[:, inter:].float()
    want = ((gf / (1.0 + torch.exp(-gf))).to(torch.bfloat16).float() * uf).to(torch.bfloat16)
    torch.testing.assert_close(y.float(), want.float(), rtol=BF16_STEP, atol=1e-6)


def test_epilogues_are_deterministic_and_replay_in_a_graph() -> None:
    x, d, w1 = case(256, 2048, 9)
    gu = torch.randn(256, 12288, device="cuda").to(torch.bfloat16)
    xo, h = add_rms(x, d, w1)
    y = silu_mul(gu)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gxo, gh = add_rms(x, d, w1)
        gy = silu_mul(gu)
    for _ in range(3):
        gh.zero_()
        gy.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gxo, xo) and torch.equal(gh, h) and torch.equal(gy, y)
        assert torch.equal(silu_mul(gu), y)


def test_epilogues_refuse_bad_arguments() -> None:
    x, d, w1 = case(4, 64, 1)
    with pytest.raises(ValueError, match="w1"):
        add_rms(x, d, w1.to(torch.bfloat16))
    with pytest.raises(ValueError, match="shape"):
        add_rms(x, d[:, :32].contiguous(), w1)
    with pytest.raises(ValueError, match="multiple of 8"):
        y = torch.zeros(4, 12, device="cuda", dtype=torch.bfloat16)
        add_rms(y, None, torch.ones(12, device="cuda"))
    with pytest.raises(ValueError, match="twice a multiple of 8"):
        silu_mul(torch.zeros(4, 24, device="cuda", dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="bfloat16"):
        silu_mul(torch.zeros(4, 32, device="cuda"))
