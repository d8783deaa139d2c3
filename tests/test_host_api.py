"""The host-side mirror of the reference's interface, checked without a GPU: the pool layout Lin.pack writes, the
pool's row management, the refusals int4_product makes before any allocation or launch, the kernel choice rule and
the product registry (the reference's tests/test_product_choice.py expectations)."""

from __future__ import annotations

import pytest
import torch

from jeff_amd.fast_path import DT, AdapterPool, Lin, Workspace, fold_scale, sb_stride
from jeff_amd.int4 import Int4Error, pack_kernel, pack_kernel_asym, unpack_kernel, unpack_kernel_asym
from jeff_amd.int4_kernels import int4_product
from jeff_amd.int4_tiles import Int4Tiles, int4_tiles
from jeff_amd.product_choice import (CUBLAS, INT4, PAIRS, PRODUCTS, ProductChoice, choose_product,
                                     product_candidates)
from oracle import pool_view


def test_pack_writes_a_rows_and_per_matrix_second_factors() -> None:
    lin = Lin(["l.q_proj", "l.k_proj"], sizes=[24, 16], k=32, ranks=[16, 8])
    assert lin.rank == 24 and lin.numel() == 24 * 32 + 24 * 16 + 16 * 8
    pool = AdapterPool([lin], 2, device="cpu")
    a0, b0 = torch.randn(8, 32).to(DT), torch.randn(24, 8).to(DT)
    a1, b1 = torch.randn(8, 32).to(DT), torch.randn(16, 8).to(DT)
    row = pool.add_adapter("x", {"l.q_proj": (a0, b0), "l.k_proj": (a1, b1)})
    assert row == 1 and pool.ranks[1, :2].tolist() == [8, 8]
    flat = pool.lora_pool[1]
    a = flat[:24 * 32].view(24, 32)
    assert torch.equal(a[0:8], a0) and bool((a[8:16] == 0).all()) and torch.equal(a[16:24], a1)
    # sB rows at the live rank's stride (rank 8 in a rank-16 block: 8 elements per row, the rest of the block zero)
    bq = flat[lin.off_bj[0]:lin.off_bj[0] + 24 * 8].view(24, 8)
    assert torch.equal(bq, b0) and bool((flat[lin.off_bj[0] + 24 * 8:lin.off_bj[1]] == 0).all())
    bk = flat[lin.off_bj[1]:lin.off_bj[1] + 16 * 8].view(16, 8)
    assert torch.equal(bk, b1)
    with pytest.raises(ValueError, match="does not fit the fast path's rank-8 buffer"):
        pool.add_adapter("big", {"l.k_proj": (torch.zeros(16, 32, dtype=DT), torch.zeros(16, 16, dtype=DT))})


def test_second_factor_stride_follows_the_live_rank() -> None:
    """sB rows are stored at the live rank rounded up to a power of two (at least 8, at most the capacity), and the
    oracle's pool reader applies the same rule: adapters of every rank read back exactly what was packed."""
    assert [sb_stride(r, 64) for r in (0, 1, 8, 9, 16, 17, 33, 64)] == [8, 8, 8, 16, 16, 32, 64, 64]
    assert [sb_stride(r, 48) for r in (0, 33, 48)] == [8, 48, 48] and sb_stride(0, 0) == 0
    lin = Lin(["l.q_proj", "l.k_proj"], sizes=[40, 24], k=16, ranks=[64, 48])
    pool = AdapterPool([lin], 8, device="cpu")
    g = torch.Generator().manual_seed(3)

    def update(r: int, n: int):
        return torch.randn(r, 16, generator=g).to(DT), torch.randn(n, r, generator=g).to(DT)

    packed = {}
    for i, (rq, rk) in enumerate([(1, 33), (8, 48), (9, 1), (17, 24), (33, 0), (64, 47)]):
        ups = {"l.q_proj": update(rq, 40)}
        if rk:
            ups["l.k_proj"] = update(rk, 24)
        packed[pool.add_adapter(f"a{i}", ups)] = ups
    got = pool_view.adapters_of(lin, packed)
    for row, ups in packed.items():
        for j, name in enumerate(lin.names):
            if name not in ups:
                assert got[row][j] is None
                continue
            assert torch.equal(got[row][j][0], ups[name][0]) and torch.equal(got[row][j][1], ups[name][1])


def test_pool_rows_lowest_free_first_base_row_zero_and_refusals() -> None:
    lin = Lin(["l.o_proj"], sizes=[16], k=16)
    pool = AdapterPool([lin], 3, device="cpu")
    up = {"l.o_proj": (torch.ones(4, 16, dtype=DT), torch.ones(16, 4, dtype=DT))}
    assert [pool.add_adapter(n, up) for n in "abc"] == [1, 2, 3]
    assert pool.index(None) == 0 and bool((pool.lora_pool[0] == 0).all()) and int(pool.ranks[0].abs().sum()) == 0
    with pytest.raises(ValueError, match="at most 3 adapters"):
        pool.add_adapter("d", up)
    with pytest.raises(ValueError, match="already"):
        pool.add_adapter("a", up)
    pool.remove_adapter("b", poison=True)
    assert int(pool.ranks[2].abs().sum()) == 0 and bool(torch.isnan(pool.lora_pool[2].float()).all())
    assert pool.add_adapter("d", up) == 2 and bool(torch.isfinite(pool.lora_pool[2].float()).all())
    with pytest.raises(ValueError, match="not loaded"):
        pool.index("b")
    pool.remove_adapter("a")
    with pytest.raises(ValueError, match="does not support"):
        pool.add_adapter("e", {"l.mlp.gate_proj": up["l.o_proj"]})


def test_scale_is_folded_in_float32_then_cast() -> None:
    b = torch.tensor([[1.0 + 2 ** -7]], dtype=DT)
    assert float(fold_scale(b, 3.0)) == float(torch.tensor((1.0 + 2 ** -7) * 3.0).to(DT))


def test_int4_product_refusals_before_any_launch() -> None:
    plain = Lin(["layers.0.mlp.down_proj"], [torch.zeros(64, 128, dtype=DT)])
    ws = Workspace(32, 32, {(128, 64)}, device="cpu")
    adp = torch.zeros(1, dtype=torch.int32)
    with pytest.raises(ValueError, match="no INT4 weights"):
        int4_product(plain, torch.zeros(32, 128, dtype=DT), ws, adp)
    plain.int4 = pack_kernel(torch.zeros(64, 128, dtype=torch.int8), torch.ones(64, 2, dtype=DT))
    with pytest.raises(ValueError, match="bfloat16"):
        int4_product(plain, torch.zeros(32, 128), ws, adp)
    with pytest.raises(ValueError, match="contiguous rows"):
        int4_product(plain, torch.zeros(128, 32, dtype=DT).T, ws, adp)
    with pytest.raises(ValueError, match="cannot hold whole rows"):
        Workspace(30, 32)


def test_kernel_layout_round_trips_and_refuses() -> None:
    q = torch.randint(-8, 8, (70, 256), dtype=torch.int8)
    s = (torch.rand(70, 2) + 0.01).to(DT)
    p = pack_kernel(q, s, 128)
    assert tuple(p.words.shape) == (32, 128) and tuple(p.scales.shape) == (2, 128) and p.k == 256
    back_q, back_s = unpack_kernel(p)
    assert torch.equal(back_q, q) and torch.equal(back_s, s)
    codes = torch.randint(0, 16, (70, 256), dtype=torch.uint8)
    z = torch.randint(0, 16, (70, 2), dtype=torch.uint8)
    pa = pack_kernel_asym(codes, s, z, 128)
    c2, s2, z2 = unpack_kernel_asym(pa)
    assert torch.equal(c2, codes) and torch.equal(s2, s) and torch.equal(z2, z)
    assert bool((pa.zeros[:, 70:] == 8).all())
    with pytest.raises(Int4Error, match="finite, positive"):
        pack_kernel(q, torch.full((70, 2), 2.0 ** 121).to(DT), 128)
    with pytest.raises(Int4Error, match=r"\[-8, 7\]"):
        pack_kernel(q.to(torch.int16) + 8, s, 128)
    with pytest.raises(Int4Error):
        pack_kernel(q, s, 96)


def test_kernel_choice_rule() -> None:
    assert int4_tiles(4096, 2048, 1) == Int4Tiles("gemv", "segment")
    assert int4_tiles(4096, 2048, 8) == Int4Tiles("gemv", "segment")
    assert int4_tiles(4096, 2048, 256, 256, 65) == Int4Tiles("narrow", "segment")
    assert int4_tiles(4096, 2048, 257, 257, 65) == Int4Tiles("split", "segment")
    assert int4_tiles(12288, 2048, 1023, 1023, 1025) == Int4Tiles("split", "segment")
    # from 1024 tokens on, short segments take the 256 x 256 tiles with the LoRA term fused (segment-form first factor)
    assert int4_tiles(12288, 2048, 4096, 4096, 1025) == Int4Tiles("mfma", "segment")
    assert int4_tiles(3072, 1024, 8704, 64, 17) == Int4Tiles("mfma", "mfma")
    with pytest.raises(ValueError):
        int4_tiles(100, 1024, 4)


def test_kernel_choice_with_epilogues() -> None:
    """The residual and gated epilogues never take the GEMV kernel (it has no epilogue): few tokens run the narrow
    product; forcing the GEMV, or both epilogues at once, is refused."""
    from jeff_amd import _lib
    from jeff_amd.int4_tiles import int4_plan

    assert int4_plan(2048, 2048, 5)[0] == "gemv"
    assert int4_plan(2048, 2048, 5, flags=_lib.EPILOGUE_RESIDUAL)[0] == "narrow"
    assert int4_plan(12288, 2048, 5, flags=_lib.EPILOGUE_SILU_MUL)[0] == "narrow"
    assert int4_plan(2048, 6144, 159488, 512, 129, 32, flags=_lib.EPILOGUE_RESIDUAL)[0] == "mfma"
    assert int4_plan(2048, 6144, 1000, 1000, 1025, 64, flags=_lib.EPILOGUE_RESIDUAL)[0] == "split"
    assert int4_plan(2048, 6144, 4096, 4096, 1025, 64, flags=_lib.EPILOGUE_RESIDUAL)[0] == "mfma"
    with pytest.raises(ValueError, match="does not run"):
        int4_plan(2048, 2048, 5, flags=_lib.EPILOGUE_RESIDUAL | _lib.FORCE_BASE_GEMV)
    with pytest.raises(ValueError, match="invalid|argument"):
        int4_plan(12288, 2048, 64, flags=_lib.EPILOGUE_RESIDUAL | _lib.EPILOGUE_SILU_MUL)


GROUPS = ("layers.0.mlp.gate_proj, layers.0.mlp.up_proj", "layers.0.mlp.down_proj")


def test_product_registry_follows_the_reference_rules() -> None:
    assert product_candidates(dict.fromkeys(GROUPS, False)) == (CUBLAS,)
    assert product_candidates(dict.fromkeys(GROUPS, True)) == PRODUCTS == (CUBLAS, INT4) and PAIRS == 3
    times = {CUBLAS: [2.4, 9.0, 2.3], INT4: [1.7, 1.6, 8.0]}
    calls = []

    def timer(kernel: str) -> float:
        calls.append(kernel)
        return times[kernel].pop(0)

    assert choose_product(PRODUCTS, timer) == ProductChoice(INT4, {CUBLAS: 2.4, INT4: 1.7})
    assert calls == [CUBLAS, INT4] * PAIRS
    assert choose_product(PRODUCTS, lambda k: 1.0) == ProductChoice(CUBLAS, {CUBLAS: 1.0, INT4: 1.0})
    with pytest.raises(ValueError, match="Unknown product kernel"):
        product_candidates(dict.fromkeys(GROUPS, True), ["hip"])
    with pytest.raises(ValueError, match="need an INT4 base"):
        product_candidates(dict.fromkeys(GROUPS, False), [INT4])
    with pytest.raises(ValueError, match="hold no INT4 weights"):
        product_candidates({GROUPS[0]: True, GROUPS[1]: False})


def test_a_route_is_shared_only_inside_the_capture_that_launched_it() -> None:
    """Workspace.routed's rule (reusable): a product reads the last routing launch instead of routing again only
    inside the same graph capture, on the same stream, for the same adp tensor unchanged since, and the same pass."""
    import weakref

    from jeff_amd.fast_path import RouteRecord, reusable

    adp = torch.zeros(4, dtype=torch.int32)
    cu = torch.tensor([0, 1, 3, 3, 9], dtype=torch.int32)

    def record(capture: int, stream: int = 7, with_cu: bool = False) -> RouteRecord:
        return RouteRecord(weakref.ref(adp), adp._version, 4, 9 if with_cu else 4, 5,
                           weakref.ref(cu) if with_cu else None, cu._version if with_cu else -1, stream, capture)

    assert reusable(record(11), adp, 4, 5, 7, 11)
    assert not reusable(record(0), adp, 4, 5, 7, 0)          # eager: always route again
    assert not reusable(record(0), adp, 4, 5, 7, 11)         # routed before the capture (the warm-up)
    assert not reusable(record(11), adp, 4, 5, 7, 12)        # another capture
    assert not reusable(record(11), adp, 4, 5, 8, 11)        # another stream
    assert not reusable(record(11), adp, 8, 5, 7, 11)        # another token count
    assert not reusable(record(11), adp, 4, 6, 7, 11)        # another pool
    other = torch.zeros(4, dtype=torch.int32)
    assert not reusable(record(11), other, 4, 5, 7, 11)      # an equal tensor that is another object
    rec = record(11)
    adp.copy_(torch.tensor([1, 2, 3, 4]))                    # new ids in the same tensor
    assert not reusable(rec, adp, 4, 5, 7, 11)
    rec = record(11, with_cu=True)
    assert reusable(rec, adp, 9, 5, 7, 11)
    cu[1] = 2                                                # new sequence lengths
    assert not reusable(rec, adp, 9, 5, 7, 11)
    rec = record(11)
    del adp                                                  # the recorded tensor is gone
    assert not reusable(rec, torch.zeros(4, dtype=torch.int32), 4, 5, 7, 11)


def test_partials_bound_covers_every_automatic_product() -> None:
    """mlora_int4_partials_bound (a workspace's up-front size for its shapes) is at least the float32 partials of the
    kernels the library picks for every token count up to the bound's own, on the decoder's groups (host only)."""
    from jeff_amd import _lib
    from jeff_amd.int4_tiles import int4_plan

    h = _lib.lib()
    for k, out in ((2048, 4096), (2048, 2048), (2048, 12288), (6144, 2048), (1024, 3072), (512, 320)):
        cols = -(-out // 64) * 64
        for tokens in (1, 9, 200, 256, 257, 1000, 4096, 20000):
            bound = h.mlora_int4_partials_bound(k, cols, out, tokens)
            for t in sorted({1, 2, 9, 255, 256, 257, 511, 512, 513, 1024, tokens // 2 + 1, tokens}):
                if t > tokens:
                    continue
                for requests in (min(t, 8192), max(1, t // 40)):
                    base, _, ranges = int4_plan(cols, k, t, requests, 1025, 64, out)
                    need = {"narrow": ranges * (cols // 64) * 256 * 64 * 4 if ranges > 1 else 0,
                            "split": (ranges * t * cols * 4 + 255) // 256 * 256}.get(base, 0)
                    assert bound >= need, (k, out, tokens, t, requests, base, ranges, need, bound)
    assert h.mlora_int4_partials_bound(100, 64, 64, 8) == 0
    assert h.mlora_int4_partials_bound(2048, 4096, 4096, 0) == 0
