"""The HIP library against the CPU oracle on identical seeded inputs (needs a gfx950 GPU; marked gpu).

- routing: bit-exact against the stable segment sort, including empty rows, the base row, out-of-range ids, unusable
  cu_seqlens and the largest pass the routing kernel takes;
- dequantisation: bit-exact, g64 and g128, symmetric and asymmetric, every code x zero point x scale exponent;
- LoRA first factor (both kernels): each bf16 value within one rounding of the float64 exact value plus the float32
  accumulation slack;
- the fused product (every kernel combination) and lora_add: within the forward error bound of exact arithmetic and
  within rtol 1e-2 / atol 2e-2 of the fp32 reference, on the reference's own test pattern (adapters cycling 1, 2, 0,
  3 over rows, a tail pass of 48 tokens in rows of 16) and on the configurations' shapes;
- two runs and a HIP graph replay give the same bits; freed pool rows are never read."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from jeff_amd import _lib
from jeff_amd.fast_path import DT, Workspace, lora_add
from jeff_amd.int4 import dequantize_kernel, pack_kernel_asym
from jeff_amd.int4_kernels import int4_product, shrink
from jeff_amd.int4_tiles import Int4Tiles
from oracle import codec
from oracle.layer import step
from oracle.routing import route as oracle_route
from tests.gpu_cases import bf16_bits, judge, make_case, mean_abs_error, oracle_adapters, token_ids

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu() -> None:
    assert torch.cuda.is_available(), "the gpu tests need an AMD GPU"
    _lib.lib()  # fails loudly when the HIP library is missing


def run_route(adp: np.ndarray, pool_rows: int, row_len: int | None, cu: np.ndarray | None):
    tokens = int(cu[-1]) if cu is not None else len(adp) * row_len
    ws = Workspace(max(tokens, 1), 1, max_requests=max(len(adp), 1))
    adp_d = torch.tensor(adp.astype(np.int32), device="cuda")
    if cu is None:
        ws.row_len = row_len
        ws.route(adp_d, pool_rows, tokens=tokens)
    else:
        ws.route(adp_d, pool_rows, tokens=tokens, cu_seqlens=torch.tensor(cu.astype(np.int32), device="cuda"))
    torch.cuda.synchronize()
    return ws, tokens


def assert_route_equal(ws: Workspace, tokens: int, want: dict, requests: int) -> None:
    s = int(ws.num_segs.item())
    assert s == want["seg_adapter"].size
    assert np.array_equal(ws.seg_start[:s + 1].cpu().numpy(), want["seg_start"])
    assert np.array_equal(ws.seg_adapter[:s].cpu().numpy(), want["seg_adapter"])
    assert np.array_equal(ws.req_order[:requests].cpu().numpy(), want["req_order"])
    assert np.array_equal(ws.tok_perm[:tokens].cpu().numpy(), want["tok_perm"])
    assert np.array_equal(ws.last_of[:tokens].cpu().numpy(), want["last_of"])
    assert np.array_equal(ws.seg_of[:tokens].cpu().numpy(), want["seg_of"])
    assert int(ws.status.item()) == want["status"]


@pytest.mark.parametrize("case", ["uniform-32", "decode-256", "one-row", "ragged-64", "ragged-65", "zipf-512",
                                  "empty-rows", "all-base", "single-adapter", "out-of-range", "long-rows",
                                  "max-requests"])
def test_route_is_bit_exact(case: str) -> None:
    rng = np.random.default_rng(hash(case) % 2**32)
    cu = None
    row_len = 1
    pool_rows = 65
    if case == "uniform-32":
        adp, row_len, pool_rows = rng.integers(0, 5, 8), 32, 5
    elif case == "decode-256":
        adp = rng.integers(1, 65, 256)
    elif case == "one-row":
        adp, row_len = np.array([3]), 16
    elif case in ("ragged-64", "ragged-65"):  # the one-wave and the block routing kernels
        n = int(case[-2:])
        adp = rng.integers(1, 17, n)
        cu = np.concatenate([[0], np.cumsum(rng.integers(16, 257, n))])
    elif case == "zipf-512":
        p = np.arange(1, 129) ** -1.1
        adp = rng.choice(128, 512, p=p / p.sum()) + 1
        cu = np.concatenate([[0], np.cumsum(np.clip(rng.lognormal(np.log(200), 1, 512), 16, 2048).astype(int))])
        pool_rows = 129
    elif case == "empty-rows":
        adp = rng.integers(0, 4, 40)
        lengths = rng.integers(0, 5, 40)
        lengths[[0, 7, 39]] = 0
        cu = np.concatenate([[0], np.cumsum(lengths)])
        pool_rows = 4
    elif case == "all-base":
        adp, row_len = np.zeros(16, dtype=int), 4
    elif case == "single-adapter":
        adp, row_len = np.full(33, 7), 3
    elif case == "out-of-range":
        adp = np.array([1, 70, -1, 2, 64, 65])
    elif case == "long-rows":  # requests longer than a routing workgroup's threads
        adp = rng.integers(0, 6, 9)
        cu = np.concatenate([[0], np.cumsum([1, 700, 255, 256, 257, 2049, 0, 513, 3])])
        pool_rows = 6
    else:  # the largest pass the routing kernel sorts
        adp = rng.integers(0, 1025, _lib.MAX_REQUESTS)
        pool_rows = 1025
    ws, tokens = run_route(adp, pool_rows, row_len if cu is None else None, cu)
    want = oracle_route(adp, pool_rows, row_len=row_len if cu is None else None, cu_seqlens=cu)
    assert_route_equal(ws, tokens, want, len(adp))


@pytest.mark.parametrize("cu", [[0, 5, 3, 9], [0, 1500, 700, 3000]])  # decreasing offsets; few and many tokens
def test_route_flags_unusable_seqlens_and_falls_back_to_identity(cu: list) -> None:
    cu = np.array(cu)
    ws, tokens = run_route(np.array([1, 2, 3]), 4, None, cu)
    assert int(ws.status.item()) == _lib.ROUTE_BAD_SEQLENS
    assert np.array_equal(ws.tok_perm[:tokens].cpu().numpy(), np.arange(tokens))
    assert not ws.seg_of[:tokens].cpu().numpy().any()
    assert int(ws.num_segs.item()) == 1 and int(ws.seg_adapter[0].item()) == 0
    with pytest.raises(ValueError, match="cu_seqlens"):
        ws.check()


@pytest.mark.parametrize("group,asym", [(64, False), (128, False), (64, True), (128, True)])
def test_dequant_is_bit_exact(group: int, asym: bool) -> None:
    g = torch.Generator().manual_seed(group + asym)
    out, k = 200, 1024  # 200 outputs: padded to 256 kernel columns
    codes = torch.randint(0, 16, (out, k), generator=g, dtype=torch.uint8)
    scales = (torch.rand(out, k // group, generator=g) * 0.015 + 0.005).to(torch.bfloat16)
    zeros = torch.randint(0, 16, (out, k // group), generator=g, dtype=torch.uint8) if asym else None
    if asym:
        packed = pack_kernel_asym(codes.cuda(), scales.cuda(), zeros.cuda(), group)
    else:
        from jeff_amd.int4 import pack_kernel
        packed = pack_kernel((codes.to(torch.int16) - 8).to(torch.int8).cuda(), scales.cuda(), group)
    got = bf16_bits(dequantize_kernel(packed))
    want = codec.dequantize(codes.numpy(), bf16_bits(scales), None if zeros is None else zeros.numpy(), group)
    assert np.array_equal(got, want)


def test_dequant_every_code_zero_and_scale() -> None:
    """Every code x every zero point x every finite positive bf16 scale below 2^120 (pack_kernel refuses larger)."""
    bits = np.arange(1, 0x7F80, dtype=np.uint16)
    bits = bits[codec.bf16_bits_to_f32(bits) < 2.0 ** 120]
    pairs_s = np.repeat(bits, 16)
    pairs_z = np.tile(np.arange(16, dtype=np.uint8), bits.size)
    groups = 64
    rows = -(-pairs_s.size // groups)
    pad = rows * groups - pairs_s.size
    s = np.concatenate([pairs_s, np.full(pad, 0x3F80, np.uint16)]).reshape(rows, groups)
    z = np.concatenate([pairs_z, np.full(pad, 8, np.uint8)]).reshape(rows, groups)
    k = 64 * groups
    codes = np.tile(np.arange(16, dtype=np.uint8), (rows, k // 16))
    scales_t = torch.from_numpy(s.view(np.int16)).view(torch.bfloat16)
    packed = pack_kernel_asym(torch.from_numpy(codes).cuda(), scales_t.cuda(), torch.from_numpy(z).cuda(), 64)
    got = bf16_bits(dequantize_kernel(packed))
    want = codec.dequantize(codes, s, z, 64)
    assert np.array_equal(got, want)


def mid_bound_check(lin, x, tok_adp, perm, mid) -> tuple[int, float]:
    """Each first factor against exact: |mid - m| <= k u32 (|x| |A|) + half a bf16 step of the largest value."""
    adapters = oracle_adapters(lin, np.unique(tok_adp))
    xd = x.cpu().double()
    bad, worst = 0, 0.0
    for p, t in enumerate(perm):
        a = int(tok_adp[t])
        if a == 0:
            continue
        for j, upd in enumerate(adapters[a]):
            if upd is None:
                continue
            am = upd[0].double()
            exact = am @ xd[t]
            slack = lin.k * 2.0 ** -23 * (am.abs() @ xd[t].abs())
            bound = slack + step(exact.abs() + slack) / 2
            got = mid[p, lin.rho[j]:lin.rho[j] + am.shape[0]].double()
            err = (got - exact).abs()
            bad += int((err > bound).sum())
            worst = max(worst, float((err / bound).max()))
    return bad, worst


@pytest.mark.parametrize("mfma", [False, True])
def test_shrink_within_one_rounding_of_exact(mfma: bool) -> None:
    case = make_case([512, 256], 1024, 64, True, {1: [8, 16], 2: [16, 0], 3: [32, 32], 5: [24, 8]}, [32, 32], 11)
    rng = np.random.default_rng(3)
    requests, row_len = 24, 5
    adp = torch.tensor(rng.integers(0, 6, requests).astype(np.int32), device="cuda")
    x = torch.randn(requests * row_len, 1024, device="cuda").to(DT)
    ws = Workspace(requests * row_len, row_len, max_rank=case.lin.rank)
    mid = shrink(case.lin, x, ws, adp, mfma=mfma).clone()
    torch.cuda.synchronize()
    perm = ws.tok_perm[:x.shape[0]].cpu().numpy()
    tok = token_ids(adp, case.lin.pool.shape[0], row_len=row_len)
    bad, worst = mid_bound_check(case.lin, x, tok, perm, mid.cpu())
    assert bad == 0, f"{bad} first factors beyond one rounding (worst {worst:.3g} x the bound)"


@pytest.mark.parametrize("k", [64, 192, 448, 1600])
@pytest.mark.parametrize("mfma", [False, True])
def test_shrink_input_chunk_counts(k: int, mfma: bool) -> None:
    """Input sizes whose 64-input chunks split unevenly over a workgroup's waves (none, one or a few each, past the
    prefetch depth or not), with segments that cross 32-row blocks."""
    case = make_case([192, 64], k, 64, True, {1: [8, 16], 2: [32, 0], 3: [16, 24]}, [32, 32], 5 + k)
    rng = np.random.default_rng(k)
    requests, row_len = 12, 13
    adp = torch.tensor(rng.integers(0, 4, requests).astype(np.int32), device="cuda")
    x = torch.randn(requests * row_len, k, device="cuda").to(DT)
    ws = Workspace(requests * row_len, row_len, max_rank=case.lin.rank)
    mid = shrink(case.lin, x, ws, adp, mfma=mfma).clone()
    torch.cuda.synchronize()
    perm = ws.tok_perm[:x.shape[0]].cpu().numpy()
    tok = token_ids(adp, case.lin.pool.shape[0], row_len=row_len)
    bad, worst = mid_bound_check(case.lin, x, tok, perm, mid.cpu())
    assert bad == 0, f"{bad} first factors beyond one rounding (worst {worst:.3g} x the bound)"


CYCLE = (1, 2, 0, 3)  # the reference's adapter pattern over request rows (tests/test_int4_kernels_cuda.py:58)


def reference_pattern_case(seed: int, group: int, asym: bool):
    return make_case([1024, 512, 16, 16], 1024, group, asym, {1: [16, 16, 16, 16], 2: [16, 8, 16, 0],
                                                             3: [8, 16, 16, 16]}, [16, 16, 16, 16], seed)


@pytest.mark.parametrize("tokens,row_len", [(32, 32), (64, 64), (128, 128), (48, 16), (256, 32), (1024, 64), (4, 1),
                                            (8, 1)])
@pytest.mark.parametrize("tiles", [None, Int4Tiles("mfma", "segment"), Int4Tiles("mfma", "mfma"),
                                   Int4Tiles("split", "segment"), Int4Tiles("split", "mfma"),
                                   Int4Tiles("narrow", "segment"), Int4Tiles("narrow", "mfma", 2)])
def test_reference_pattern_products_are_within_the_bound(tokens: int, row_len: int, tiles) -> None:
    if tiles is not None and tiles.base == "narrow" and tokens > 256:
        pytest.skip("the narrow product takes at most 256 tokens")
    case = reference_pattern_case(tokens + row_len, 64, False)
    lin = case.lin
    rows = tokens // row_len
    adp = torch.tensor([CYCLE[r % 4] for r in range(rows)], dtype=torch.int32, device="cuda")
    gen = torch.Generator(device="cuda").manual_seed(tokens * 7919 + row_len * 31 + lin.k)
    x = torch.randn(tokens, lin.k, device="cuda", generator=gen).to(DT)
    ws = Workspace(tokens, row_len, max_rank=lin.rank)
    got = int4_product(lin, x, ws, adp, tiles=tiles)
    assert got.shape == (tokens, lin.out) and got.dtype == DT
    r = judge(lin, case.w, x, token_ids(adp, lin.pool.shape[0], row_len=row_len), got)
    assert r["finite"] and r["beyond_bound"] == 0 and r["outside_tolerance"] == 0, r
    # the reference's accuracy gate (tests/test_int4_kernels_cuda.py:196-198): the kernel's mean absolute error
    # against exact is no larger than the library GEMM's on the dequantised weights plus lora_add
    lin.W = case.w.cuda()
    library = lin(x, ws, adp)
    assert r["mean_abs_err"] <= mean_abs_error(lin, case.w, x, token_ids(adp, lin.pool.shape[0], row_len=row_len),
                                               library), r


@pytest.mark.parametrize("tokens", [1, 3, 8])
@pytest.mark.parametrize("shrink_kind", ["segment", "mfma"])
def test_decode_gemv_products(tokens: int, shrink_kind: str) -> None:
    case = make_case([2048, 1024, 1024], 2048, 128, True, {a: [r, r, r] for a, r in
                                                            zip(range(1, 9), (8, 16, 32, 64, 8, 16, 32, 64))},
                     [64, 64, 64], 5)
    lin = case.lin
    adp = torch.tensor(np.random.default_rng(tokens).integers(0, 9, tokens).astype(np.int32), device="cuda")
    x = torch.randn(tokens, lin.k, device="cuda").to(DT)
    ws = Workspace(tokens, 1, max_rank=lin.rank)
    got = int4_product(lin, x, ws, adp, tiles=Int4Tiles("gemv", shrink_kind))
    r = judge(lin, case.w, x, token_ids(adp, lin.pool.shape[0], row_len=1), got)
    assert r["finite"] and r["beyond_bound"] == 0 and r["outside_tolerance"] == 0, r


@pytest.mark.parametrize("tiles", [None, Int4Tiles("mfma", "mfma"), Int4Tiles("mfma", "segment"),
                                   Int4Tiles("split", "mfma"), Int4Tiles("split", "segment"),
                                   Int4Tiles("narrow", "segment", 1), Int4Tiles("narrow", "segment", 8)])
def test_mixed_rank_decode_batch(tiles) -> None:
    """256 one-token rows, 64 adapters of ranks 8/16/32/64, a qkv-shaped group (2048 -> 2048 + 1024 + 1024)."""
    ranks = {a: [(8, 16, 32, 64)[(a - 1) // 16]] * 3 for a in range(1, 65)}
    case = make_case([2048, 1024, 1024], 2048, 128, True, ranks, [64, 64, 64], 7)
    lin = case.lin
    adp = torch.tensor(np.random.default_rng(1).integers(1, 65, 256).astype(np.int32), device="cuda")
    x = torch.randn(256, lin.k, device="cuda").to(DT)
    ws = Workspace(256, 1, max_rank=lin.rank)
    got = int4_product(lin, x, ws, adp, tiles=tiles)
    r = judge(lin, case.w, x, token_ids(adp, lin.pool.shape[0], row_len=1), got)
    assert r["finite"] and r["beyond_bound"] == 0 and r["outside_tolerance"] == 0, r


NARROW_CASES = {
    # matrices straddling 32-column groups, a matrix without LoRA, a non-power-of-two capacity, odd ranks
    "straddle": ([40, 24, 200], 256, [16, 24, 0], {1: [16, 24, 0], 2: [3, 17, 0], 3: [0, 9, 0], 4: [8, 0, 0]}, 37),
    # capacities above one 64-rank pass (128 and 72), segments longer than a wave's 64 rows
    "big-cap": ([128, 96], 128, [128, 72], {1: [128, 72], 2: [65, 40], 3: [100, 8]}, 200),
    # the most tokens, 64 columns only, every token its own request
    "one-tile": ([64], 512, [32], {a: [(8, 16, 24, 32)[a % 4]] for a in range(1, 33)}, 256),
    "one-token": ([96, 32], 192, [16, 16], {1: [16, 16], 2: [8, 0]}, 1),
}


@pytest.mark.parametrize("name", list(NARROW_CASES))
@pytest.mark.parametrize("ranges", [None, 1, 2, 4])
def test_narrow_products(name: str, ranges) -> None:
    """The narrow product (every token in one row tile of 64 columns, the LoRA term fused) on awkward groups, with
    the input dimension in 1, 2 and 4 ranges; each request's last-token row gathered as well."""
    sizes, k, caps, ranks, tokens = NARROW_CASES[name]
    if ranges is not None and (k // 64) % ranges:
        pytest.skip(f"{k // 64} input steps do not split into {ranges} ranges")
    case = make_case(sizes, k, 128 if k % 128 == 0 else 64, True, ranks, caps, 11)
    lin = case.lin
    rng = np.random.default_rng(tokens + k)
    row_len = 4 if name == "big-cap" else 1
    requests = tokens // row_len
    adp = torch.tensor(rng.integers(0, max(ranks) + 1, requests).astype(np.int32), device="cuda")
    x = torch.randn(tokens, lin.k, device="cuda").to(DT)
    ws = Workspace(tokens, row_len, max_rank=lin.rank)
    last = torch.empty(requests, lin.out, dtype=DT, device="cuda")
    got = int4_product(lin, x, ws, adp, tiles=Int4Tiles("narrow", "segment", ranges), last_out=last)
    assert torch.equal(last, got[row_len - 1::row_len])
    r = judge(lin, case.w, x, token_ids(adp, lin.pool.shape[0], row_len=row_len), got)
    assert r["finite"] and r["beyond_bound"] == 0 and r["outside_tolerance"] == 0, r


@pytest.mark.parametrize("tiles", [None, Int4Tiles("narrow", "segment", 1), Int4Tiles("narrow", "segment", 2),
                                   Int4Tiles("split", "segment"), Int4Tiles("mfma", "segment")])
def test_more_segments_than_a_wave_has_lanes(tiles) -> None:
    """Requests of no tokens still make adapter segments (empty ones). 200 requests, each with its own adapter, in
    shuffled order; the odd adapters' requests have one token and the even ones' none, so in sorted order every 64
    rows span 127 segment indices, more than a wave holds one per lane."""
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
    last = torch.empty(n, lin.out, dtype=DT, device="cuda")
    got = int4_product(lin, x, ws, adp, tiles=tiles, last_out=last)
    ws.check()
    assert int(ws.num_segs.item()) == n
    ends = np.flatnonzero(lengths)
    assert torch.equal(last[torch.as_tensor(ends, device="cuda")], got[torch.as_tensor(cu[1:][ends] - 1,
                                                                                    device="cuda").long()])
    r = judge(lin, case.w, x, token_ids(adp, lin.pool.shape[0], cu=cu_d), got)
    assert r["finite"] and r["beyond_bound"] == 0 and r["outside_tolerance"] == 0, r


@pytest.mark.parametrize("tiles", [None, Int4Tiles("mfma", "segment"), Int4Tiles("split", "mfma")])
def test_ragged_prefill_with_last_token_gather(tiles) -> None:
    """64 requests of U{16..256} tokens, 16 adapters rank 16 on a 1024 -> 3072 g128 asymmetric group; each request's
    last-token row gathered as well."""
    case = make_case([3072], 1024, 128, True, {a: [16] for a in range(1, 17)}, [16], 9)
    lin = case.lin
    rng = np.random.default_rng(2)
    lengths = rng.integers(16, 257, 64)
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    tokens = int(cu[-1])
    adp = torch.tensor(rng.integers(1, 17, 64).astype(np.int32), device="cuda")
    cu_d = torch.tensor(cu, device="cuda")
    x = torch.randn(tokens, lin.k, device="cuda").to(DT)
    ws = Workspace(tokens, 1, max_rank=lin.rank, max_requests=64)
    ws.route(adp, lin.pool.shape[0], tokens=tokens, cu_seqlens=cu_d)
    last = torch.empty(64, lin.out, dtype=DT, device="cuda")
    got = int4_product(lin, x, ws, adp, tiles=tiles, last_out=last)
    ws.check()
    assert torch.equal(last, got[torch.as_tensor(cu[1:] - 1, device="cuda").long()])
    tok = token_ids(adp, lin.pool.shape[0], cu=cu_d)
    sample = np.unique(np.concatenate([cu[:-1], cu[1:] - 1, rng.integers(0, tokens, 64)]))
    r = judge(lin, case.w, x, tok, got, rows=sample)
    assert r["finite"] and r["beyond_bound"] == 0 and r["outside_tolerance"] == 0, r


def test_lora_add_on_the_library_gemm_is_within_the_uncut_bound() -> None:
    """Lin.__call__ (torch's GEMM on the bf16 W, then lora_add), the reference's "cublas" product, against exact."""
    from oracle.layer import exact_and_bound, reference_f32, uncut_bound, within_tolerance
    case = reference_pattern_case(4, 64, False)
    lin = case.lin
    lin.W = case.w.cuda()
    adp = torch.tensor([CYCLE[r % 4] for r in range(8)], dtype=torch.int32, device="cuda")
    x = torch.randn(256, lin.k, device="cuda").to(DT)
    ws = Workspace(256, 32, max_rank=lin.rank)
    base = x @ lin.W.T
    got = lora_add(base.clone(), x, lin, adp, ws).cpu()
    tok = token_ids(adp, lin.pool.shape[0], row_len=32)
    adapters = oracle_adapters(lin, np.unique(tok))
    exact, bound = exact_and_bound(x.cpu(), case.w, tok, adapters, lin.sizes, lin.rank)
    # torch's GEMM splits and orders its sums its own way: allow its bf16 rounding of the base as the uncut bound
    # does, plus one more step for its reduction order
    allowed = uncut_bound(x.cpu(), case.w, exact, bound) + step(exact.abs())
    assert int(((got.double() - exact).abs() > allowed).sum()) == 0
    assert bool(within_tolerance(got, reference_f32(x.cpu(), case.w, tok, adapters, lin.sizes)).all())
    again = lin(x, ws, adp)
    assert torch.equal(again.cpu(), got)


def test_two_runs_and_a_graph_replay_give_the_same_bits() -> None:
    case = reference_pattern_case(21, 128, True)
    lin = case.lin
    for tokens, row_len, tiles in ((32, 32, None), (1024, 64, None), (6, 1, None), (64, 1, Int4Tiles("mfma", "segment")),
                                   (64, 1, None), (1024, 64, Int4Tiles("split", "mfma")),
                                   (64, 1, Int4Tiles("narrow", "segment", 4)), (256, 4, Int4Tiles("split", "segment"))):
        adp = torch.tensor([CYCLE[r % 4] for r in range(tokens // row_len)], dtype=torch.int32, device="cuda")
        x = torch.randn(tokens, lin.k, device="cuda").to(DT)
        ws = Workspace(tokens, row_len, max_rank=lin.rank)
        first = int4_product(lin, x, ws, adp, tiles=tiles)
        second = int4_product(lin, x, ws, adp, tiles=tiles)
        assert torch.equal(first, second)
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            int4_product(lin, x, ws, adp, tiles=tiles)
        torch.cuda.current_stream().wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = int4_product(lin, x, ws, adp, tiles=tiles)
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, first)
            _ = x.float().sum().item()  # eager work between replays


def test_a_freed_row_is_never_read() -> None:
    """Freed rows are NaN-poisoned; a pass naming one reads no LoRA from it (its live ranks are 0), and a pass that
    does not name it is unchanged."""
    case = reference_pattern_case(5, 64, False)
    lin, pool = case.lin, case.pool
    adp = torch.tensor([1, 2, 3, 2], dtype=torch.int32, device="cuda")
    x = torch.randn(64, lin.k, device="cuda").to(DT)
    ws = Workspace(64, 16, max_rank=lin.rank)
    before = int4_product(lin, x, ws, adp)
    pool.remove_adapter("a3", poison=True)
    after = int4_product(lin, x, ws, torch.tensor([1, 2, 3, 2], dtype=torch.int32, device="cuda"))
    assert bool(torch.isfinite(after.float()).all())
    assert torch.equal(after[:32], before[:32]) and torch.equal(after[48:], before[48:])
    base_only = int4_product(lin, x, ws, torch.tensor([0, 0, 0, 0], dtype=torch.int32, device="cuda"))
    assert torch.equal(after[32:48], base_only[32:48])
