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


def test_silu_mul_over_every_bf16_gate() -> None:
    """All 65536 bf16 gate values (with up = 1, then random ups): bit for bit the oracle's rounding wherever exp(-g)
    is finite in float32; below g of about -88.7, where the reference's float32 formula overflows exp and gives
    g / inf = -0, bit for bit that formula (the float64 oracle keeps a tiny nonzero value there). Signed zeros and
    infinities included: g = -0 gives -0 * u and g = +inf gives inf * u, as the formula does."""
    g = np.arange(65536, dtype=np.uint32).astype(np.uint16).reshape(256, 256)
    gf = from_bits(g).float()
    with np.errstate(over="ignore", invalid="ignore"):
        overflow = np.isinf(np.exp(-gf.numpy()))
    overflow &= gf.numpy() < 0  # exp(-g) overflows: g below about -88.7 (and g = -inf)
    ups = [np.full((256, 256), 0x3F80, np.uint16),
           bits(torch.randn(256, 256, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16))]
    for u in ups:
        gu = np.concatenate([g, u], 1)
        y = bits(silu_mul(from_bits(gu).cuda()))
        with np.errstate(invalid="ignore"):  # the NaN and infinite gates
            _, want, _ = oracle_silu_mul(gu)
        uf = from_bits(u).float()
        f32 = bits(((gf / (1.0 + torch.exp(-gf))).to(torch.bfloat16).float() * uf).to(torch.bfloat16))
        want = np.where(overflow, f32, want)
        nan_got, nan_want = np.isnan(from_bits(y).float().numpy()), np.isnan(from_bits(want).float().numpy())
        assert np.array_equal(nan_got, nan_want)
        differ = (y != want) & ~nan_got
        assert not differ.any(), f"{int(differ.sum())} gates differ, e.g. {[hex(v) for v in g[differ][:8]]}"
        assert y[128, 0] == (0x8000 if u[128, 0] < 0x8000 else 0)  # g = -0 (row 128, column 0): -0 * u


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


# name: (tokens per request, requests, adapters, gate/up width, inputs, tiles, the kernel chosen, rank capacity of gate
# and of up). At capacity c the adapters' live ranks cycle through RANKS[c]: c itself among them, so the sB rows at
# the capacity's own stride are read (64: finish_gated_columns<8>, the gated 256 x 256 kernel's second staged buffer,
# the narrow kernel's ranks 33..64; 40 and 48: up's ranks across both staged buffers of the 256 x 256 kernel).
RANKS = {32: (8, 16, 32), 40: (40, 8, 24), 48: (16, 48, 40), 64: (8, 16, 32, 64, 40, 56)}
FUSED_CASES = {
    "decode-narrow": (1, 160, 12, 512, 2048, None, "narrow", 32),
    "decode-narrow-cap64": (1, 256, 64, 512, 2048, None, "narrow", 64),  # decode-28l's gate_up, narrower
    "decode-narrow-cap48": (1, 200, 24, 256, 1024, None, "narrow", 48),
    "decode-narrow-ranges": (1, 96, 12, 256, 1024, "narrow-4", "narrow", 32),
    "decode-narrow-ranges-cap64": (1, 96, 12, 256, 1024, "narrow-4", "narrow", 64),
    "decode-narrow-one-range-cap64": (1, 256, 64, 512, 2048, "narrow-1", "narrow", 64),  # as decode-28l's gate_up
    "decode-few-tokens": (1, 5, 12, 256, 512, "narrow", "narrow", 32),
    "decode-split": (1, 600, 48, 256, 1024, None, "split", 32),
    "decode-split-cap64": (1, 600, 48, 256, 1024, None, "split", 64),
    # 1536 one-token rows over 300 adapters: the 256 x 256 tiles with ~50 segments each (lane tables, 64 at a time)
    "decode-tiles-cap64": (1, 1536, 300, 256, 1024, None, "mfma", 64),  # decode-pool-28l's gate_up, narrower
    "prefill-fused": (64, 24, 12, 384, 1024, None, "mfma", 32),  # 1536 tokens: 224-row tiles
    "prefill-fused-cap64": (64, 24, 12, 384, 1024, None, "mfma", 64),
    "prefill-fused-cap48": (64, 24, 12, 384, 1024, None, "mfma", 48),
    "prefill-fused-cap40": (80, 20, 12, 256, 512, None, "mfma", 40),
    "prefill-tail": (40, 26, 12, 128, 512, "mfma", "mfma", 32),  # 1040 tokens: the last 256-row tile holds 16
}


@pytest.mark.parametrize("name", list(FUSED_CASES))
def test_silu_mul_in_the_product_tile_equals_silu_mul_of_the_product(name: str) -> None:
    """int4_product(..., epilogue="silu_mul") on a gate_up group (gate then up, one width) against silu_mul of the
    plain product (the same tiles), bit for bit, for every kernel family that takes it (narrow with and without input
    ranges, few tokens, split, the 256 x 256 tiles of 224 and 256 rows with a partial last tile) at rank capacities
    32, 40, 48 and 64, with the last-token rows gathered; against the oracle's silu_mul of the plain product; and the
    plain product against the oracle's exact result and bound on every row."""
    from jeff_amd.fast_path import Workspace
    from jeff_amd.int4_kernels import int4_product
    from jeff_amd.int4_tiles import Int4Tiles
    from tests.gpu_cases import judge, make_case, token_ids

    from jeff_amd import _lib
    from jeff_amd.int4_tiles import int4_plan

    row_len, requests, adapters, width, k, forced, kernel, cap = FUSED_CASES[name]
    print(f"fused silu_mul {name}", flush=True)
    cyc = RANKS[cap]
    ranks = {a: [cyc[a % len(cyc)], cyc[(a + 1) % len(cyc)]] for a in range(1, adapters + 1)}
    case = make_case([width, width], k, 128, True, ranks, [cap, cap], width + k)
    lin = case.lin
    tokens = row_len * requests
    rng = np.random.default_rng(tokens)
    adp = torch.tensor(rng.integers(0, adapters + 1, requests).astype(np.int32), device="cuda")
    x = torch.randn(tokens, k, device="cuda").to(torch.bfloat16)
    ws = Workspace(tokens, row_len, max_rank=lin.rank)
    tiles = {None: None, "narrow": Int4Tiles("narrow", "segment"), "narrow-1": Int4Tiles("narrow", "segment", 1),
             "narrow-4": Int4Tiles("narrow", "segment", 4), "split": Int4Tiles("split", "segment"),
             "mfma": Int4Tiles("mfma", "mfma")}[forced]
    flags = (0 if tiles is None else tiles.flags()) | _lib.EPILOGUE_SILU_MUL
    assert int4_plan(lin.int4.columns, k, tokens, requests, adapters + 1, lin.rank, lin.out, flags)[0] == kernel
    # the plain product on the same kernels (unforced, a few tokens would take the GEMV, which sums in another order)
    plan = int4_plan(lin.int4.columns, k, tokens, requests, adapters + 1, lin.rank, lin.out, flags)
    plain = int4_product(lin, x, ws, adp, tiles=tiles if tiles is not None else Int4Tiles(plan[0], plan[1]))
    last = torch.zeros(requests, width, dtype=torch.bfloat16, device="cuda")
    fused = int4_product(lin, x, ws, adp, tiles=tiles, last_out=last, epilogue="silu_mul")
    assert fused.shape == (tokens, width)
    assert torch.equal(fused, silu_mul(plain))
    assert torch.equal(last, fused[row_len - 1::row_len])
    y_exact, y_bits, _ = oracle_silu_mul(bits(plain))
    check_close(fused, y_exact, y_bits, f"fused silu_mul {name}")
    r = judge(lin, case.w, x, token_ids(adp, adapters + 1, row_len=row_len), plain)
    assert r["beyond_bound"] == 0 and r["outside_tolerance"] == 0, f"{name}: {r}"


def test_silu_mul_epilogue_refusals() -> None:
    from jeff_amd.fast_path import Workspace
    from jeff_amd.int4_kernels import int4_product
    from tests.gpu_cases import make_case

    case = make_case([256, 128], 512, 128, True, {1: [8, 8]}, [8, 8], 3)
    x = torch.randn(8, 512, device="cuda").to(torch.bfloat16)
    adp = torch.ones(8, dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="gate and an up matrix of one width"):
        int4_product(case.lin, x, Workspace(8, 1, max_rank=16), adp, epilogue="silu_mul")
    with pytest.raises(ValueError, match="Unknown epilogue"):
        int4_product(case.lin, x, Workspace(8, 1, max_rank=16), adp, epilogue="gelu")


RESIDUAL_CASES = {  # name: (tokens per request, requests, adapters, matrix widths, inputs, tiles, the kernel chosen,
    # rank capacity of every matrix; the live ranks cycle through RANKS[capacity])
    "decode-narrow": (1, 160, 12, [512], 2048, None, "narrow", 32),
    "decode-narrow-ranges": (1, 96, 12, [256], 1024, "narrow-4", "narrow", 32),
    "decode-o-cap64": (1, 256, 64, [2048], 2048, None, "narrow", 64),  # decode-28l's o product
    "decode-down-cap64": (1, 256, 64, [2048], 6144, None, "narrow", 64),  # decode-28l's down product
    "decode-one-range-cap64": (1, 256, 64, [1024], 2048, "narrow-1", "narrow", 64),
    "decode-few-tokens": (1, 5, 12, [256], 512, None, "narrow", 32),  # 5 tokens: the narrow product, not the GEMV
    "decode-split": (1, 600, 48, [256], 1024, None, "split", 32),
    "decode-split-cap64": (1, 600, 48, [256, 128], 1024, None, "split", 64),  # finish_columns<8>
    # the 256 x 256 tiles on a decode-shaped pass (each tile's segments from lane tables, 64 at a time)
    "decode-tiles-cap64": (1, 1536, 300, [384, 128], 1024, None, "mfma", 64),
    "decode-tiles-many-segments": (1, 2048, 900, [256], 512, None, "mfma", 32),  # > 64 segments in a tile
    "prefill-fused": (64, 24, 12, [384, 128], 1024, None, "mfma", 32),
    "prefill-fused-cap64": (64, 24, 12, [384, 128], 1024, None, "mfma", 64),
    "prefill-small": (20, 6, 12, [256], 512, "mfma", "mfma", 32),  # 120 tokens: still the 256 x 256 kernel
    "prefill-tail": (40, 26, 12, [128], 512, "mfma", "mfma", 32),  # 1040 tokens: the last 256-row tile holds 16
}


@pytest.mark.parametrize("name", list(RESIDUAL_CASES))
def test_residual_add_in_the_product_tile_equals_add_rms_of_the_product(name: str) -> None:
    """int4_product(..., epilogue="residual", residual=r) against the x that add_rms(r, product, w) gives on the plain
    product (the same tiles), bit for bit, for every kernel family that takes it, with the last-token rows gathered;
    and against the oracle's residual add."""
    from jeff_amd import _lib
    from jeff_amd.fast_path import Workspace
    from jeff_amd.int4_kernels import int4_product
    from jeff_amd.int4_tiles import Int4Tiles, int4_plan
    from tests.gpu_cases import judge, make_case, token_ids

    row_len, requests, adapters, widths, k, forced, kernel, cap = RESIDUAL_CASES[name]
    print(f"fused residual add {name}", flush=True)
    cyc = RANKS[cap]
    ranks = {a: [cyc[(a + j) % len(cyc)] for j in range(len(widths))] for a in range(1, adapters + 1)}
    case = make_case(widths, k, 128, True, ranks, [cap] * len(widths), sum(widths) + k + 7)
    lin = case.lin
    tokens = row_len * requests
    rng = np.random.default_rng(tokens + 1)
    adp = torch.tensor(rng.integers(0, adapters + 1, requests).astype(np.int32), device="cuda")
    x = torch.randn(tokens, k, device="cuda").to(torch.bfloat16)
    ws = Workspace(tokens, row_len, max_rank=lin.rank)
    tiles = {None: None, "narrow": Int4Tiles("narrow", "segment"), "narrow-1": Int4Tiles("narrow", "segment", 1),
             "narrow-4": Int4Tiles("narrow", "segment", 4), "split": Int4Tiles("split", "segment"),
             "mfma": Int4Tiles("mfma", "mfma")}[forced]
    flags = (0 if tiles is None else tiles.flags()) | _lib.EPILOGUE_RESIDUAL
    plan = int4_plan(lin.int4.columns, k, tokens, requests, adapters + 1, lin.rank, lin.out, flags)
    assert plan[0] == kernel
    # the plain product on the same kernels (unforced, a few tokens would take the GEMV, which sums in another order)
    same = Int4Tiles(plan[0], plan[1], plan[2] if plan[0] == "narrow" else None)
    plain = int4_product(lin, x, ws, adp, tiles=tiles if tiles is not None else same)
    r0 = (3 * torch.randn(tokens, lin.out, device="cuda")).to(torch.bfloat16)
    res = r0.clone()
    last = torch.zeros(requests, lin.out, dtype=torch.bfloat16, device="cuda")
    got = int4_product(lin, x, ws, adp, tiles=tiles, last_out=last, epilogue="residual", residual=res)
    assert got is res
    xo, _ = add_rms(r0, plain, torch.ones(lin.out, device="cuda"))
    assert torch.equal(res, xo)
    assert torch.equal(last, res[row_len - 1::row_len])
    xo_bits, _, _ = oracle_add_rms(bits(r0), bits(plain), np.ones(lin.out, np.float32))
    assert np.array_equal(bits(res), xo_bits)
    r = judge(lin, case.w, x, token_ids(adp, adapters + 1, row_len=row_len), plain)
    assert r["beyond_bound"] == 0 and r["outside_tolerance"] == 0, f"{name}: {r}"


def test_residual_epilogue_refusals() -> None:
    from jeff_amd import _lib
    from jeff_amd.fast_path import Workspace
    from jeff_amd.int4_kernels import int4_product
    from jeff_amd.int4_tiles import Int4Tiles
    from tests.gpu_cases import make_case

    case = make_case([256], 512, 128, True, {1: [8]}, [8], 5)
    lin = case.lin
    x = torch.randn(8, 512, device="cuda").to(torch.bfloat16)
    adp = torch.ones(8, dtype=torch.int32, device="cuda")
    ws = Workspace(8, 1, max_rank=16)
    r = torch.zeros(8, 256, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="takes the residual rows"):
        int4_product(lin, x, ws, adp, epilogue="residual")
    with pytest.raises(ValueError, match="takes the residual rows"):
        int4_product(lin, x, ws, adp, residual=r)
    with pytest.raises(ValueError, match="residual must be a bfloat16"):
        int4_product(lin, x, ws, adp, epilogue="residual", residual=r[:, :128])
    flat = torch.zeros(8 * 512 + 8 * 256, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="must not overlap x"):  # rows of x and of the residual in one buffer
        int4_product(lin, flat[:4096].view(8, 512), ws, adp, epilogue="residual",
                     residual=flat[2048:4096].view(8, 256))
    with pytest.raises(_lib.HipError, match="does not run"):  # the GEMV kernel has no epilogue
        int4_product(lin, x, ws, adp, tiles=Int4Tiles("gemv", "segment"), epilogue="residual", residual=r)
    h = _lib.lib()
    rc = h.mlora_lora_add(lin.lora_abi(), ws.routed(adp, lin.pool.shape[0], 8), x.data_ptr(), x.stride(0), 512,
                          r.data_ptr(), r.stride(0), 256, ws.mid.data_ptr(), ws.mid.numel() * 2,
                          _lib.EPILOGUE_RESIDUAL, torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.EUNSUPPORTED
    assert not r.any()  # nothing ran
