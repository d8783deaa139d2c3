"""The five benchmark configurations at their real shapes on the GPU, checked against the CPU oracle.

Each output row depends only on its own input row, the group's weights and its adapter, so checking a sample of rows
(every request's first and last token among them) with the oracle is an exact check of those rows; the whole output
is checked for finiteness. Where the oracle's float64 sums take seconds (every group of decode-28l, gate_up of
prefill-1layer and of decode-pool-28l: all 4096 rows, about 1000 adapters), every row is checked. The decoder
configurations run one of their 28 identical layers (all four fused groups).
- cpu-1024: bf16 base 1024 -> 1024 (torch's GEMM, the reference's "cublas" product) plus lora_add, 256 tokens in 8
  segments of 32, 4 adapters of rank 16;
- prefill-1layer, decode-28l, prefill-skewed-28l (with the last-token gather), decode-pool-28l: int4_product."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from jeff_amd import workloads
from jeff_amd.fast_path import DT, AdapterPool, Lin, Workspace, fold_scale, lora_add
from jeff_amd.int4_kernels import int4_product
from oracle.layer import exact_and_bound, reference_f32, step, uncut_bound, within_tolerance
from oracle.pool_view import adapters_of, weights_of
from tests.gpu_cases import judge

pytestmark = pytest.mark.gpu


def test_cpu_reference_config_bf16_base() -> None:
    g = torch.Generator().manual_seed(0)
    x = torch.randn(256, 1024, generator=g).to(DT)
    w = (torch.randn(1024, 1024, generator=g) * 0.02).to(DT)
    lin = Lin(["layers.0.self_attn.o_proj"], [w.cuda()])
    pool = AdapterPool([lin], 4)
    for a in range(1, 5):
        am = (torch.randn(16, 1024, generator=g) / 32).to(DT)
        b = torch.randn(1024, 16, generator=g) * 0.02
        pool.add_adapter(f"a{a}", {lin.names[0]: (am.cuda(), fold_scale(b, 2.0).cuda())})
    ids = torch.randint(1, 5, (8,), generator=g).to(torch.int32)
    ws = Workspace(256, 32, max_rank=lin.rank)
    got = lin(x.cuda(), ws, ids.cuda()).cpu()
    tok = np.repeat(ids.numpy(), 32)
    adapters = adapters_of(lin, np.unique(tok))
    exact, bound = exact_and_bound(x, w, tok, adapters, lin.sizes, lin.rank)
    allowed = uncut_bound(x, w, exact, bound) + step(exact.abs())  # torch's GEMM orders its sums its own way
    assert int(((got.double() - exact).abs() > allowed).sum()) == 0
    assert bool(within_tolerance(got, reference_f32(x, w, tok, adapters, lin.sizes)).all())


def sample_rows(w: workloads.Workload, n_random: int = 48) -> np.ndarray:
    cu = np.concatenate([[0], np.cumsum(w.lengths)])
    rng = np.random.default_rng(7)
    firsts = cu[:-1][w.lengths > 0]
    lasts = cu[1:][w.lengths > 0] - 1
    picks = rng.choice(len(firsts), min(24, len(firsts)), replace=False)
    rows = np.concatenate([firsts[picks], lasts[picks], rng.integers(0, w.tokens, n_random)])
    return np.unique(rows)


# groups checked on every output row against the oracle; the others on sampled rows and on whole row tiles, plus
# every row against the fp32 reference on the GPU
EVERY_ROW = {"prefill-1layer": ("gate_up",), "decode-28l": ("qkv", "o", "gate_up", "down"),
             "prefill-skewed-28l": (), "decode-pool-28l": ("qkv", "o", "gate_up", "down")}


def whole_tiles(ws: Workspace, tokens: int, height: int = 256) -> np.ndarray:
    """The original token indices of the first, a middle and the last row tile of `height` sorted rows (every 32-row
    block of those tiles' accumulators), read from the route."""
    perm = ws.tok_perm[:tokens].cpu().numpy()
    n = (tokens + height - 1) // height
    picks = sorted({0, n // 2, n - 1})
    return np.concatenate([perm[m * height:min((m + 1) * height, tokens)] for m in picks])


@pytest.mark.parametrize("name", ["prefill-1layer", "decode-28l", "prefill-skewed-28l", "decode-pool-28l"])
def test_config_at_full_shape(name: str) -> None:
    """One layer of each configuration at its full token and adapter shape, the products the benchmark times among
    them: every group's plain product against the oracle (every row, or sampled rows and whole row tiles, with every
    row against the fp32 reference on the GPU); on the decoder configurations gate_up with SiLU(gate) * up in its
    output tile and o and down with the residual add in theirs, each bit for bit against silu_mul / add_rms of the
    plain product (and, on the decode passes, against the oracle's epilogue of it), at the rank capacities the
    benchmark runs (64 on the decode passes: adapters of ranks up to 64)."""
    from jeff_amd.epilogues import add_rms, silu_mul
    from oracle.epilogue import add_rms as oracle_add_rms
    from oracle.epilogue import silu_mul as oracle_silu_mul
    from tests.gpu_cases import bf16_bits, reference_f32_gpu

    print(f"config {name}", flush=True)
    w = workloads.make(name, n_layers=1)
    layer = w.layers[0]
    gen = torch.Generator(device="cuda").manual_seed(5)
    ws = Workspace(w.tokens, 1, max_rank=max(lin.rank for lin in layer.values()), max_requests=w.requests)
    ws.route(w.adp, w.pool.lora_pool.shape[0], tokens=w.tokens, cu_seqlens=w.cu_seqlens)
    tok = workloads.token_ids(w)
    rows = np.unique(np.concatenate([sample_rows(w), whole_tiles(ws, w.tokens)]))
    decode = name.startswith("decode")
    for label, lin in layer.items():
        print(f"config {name} {label}", flush=True)
        x = workloads.inputs(w, label, gen)
        last = torch.empty(w.requests, lin.out, dtype=DT, device="cuda") if w.gather_last else None
        y = int4_product(lin, x, ws, w.adp, last_out=last)
        torch.cuda.synchronize()
        assert bool(torch.isfinite(y.float()).all()), f"{name} {label}: non-finite outputs"
        if last is not None:
            ends = torch.as_tensor(np.cumsum(w.lengths) - 1, device="cuda")
            assert torch.equal(last, y[ends]), f"{name} {label}: gathered rows differ"
        wt = weights_of(lin.int4)
        every = label in EVERY_ROW[name]
        r = judge(lin, wt, x, tok, y, rows=None if every else rows)
        assert r["beyond_bound"] == 0 and r["outside_tolerance"] == 0, f"{name} {label}: {r}"
        if not every:  # every row against the fp32 reference, on the GPU
            ref = reference_f32_gpu(lin, wt, x, tok)
            bad = int((~within_tolerance(y, ref)).sum())
            assert bad == 0, f"{name} {label}: {bad} outputs outside rtol 1e-2 / atol 2e-2 of the fp32 reference"
            del ref
        if w.gated and label == "gate_up":
            inter = lin.out // 2
            glast = torch.empty(w.requests, inter, dtype=DT, device="cuda") if w.gather_last else None
            fused = int4_product(lin, x, ws, w.adp, last_out=glast, epilogue="silu_mul")
            assert torch.equal(fused, silu_mul(y)), f"{name} gate_up: the gated tile differs from silu_mul"
            if glast is not None:
                assert torch.equal(glast, fused[ends])
            if decode:
                y_exact, y_bits, _ = oracle_silu_mul(bf16_bits(y))
                unequal = int((bf16_bits(fused) != y_bits).sum())
                assert unequal <= max(1, 0.005 * fused.numel()), f"{name}: {unequal} SiLU outputs off the oracle's"
                torch.testing.assert_close(fused.float().cpu().double(), torch.from_numpy(y_exact), rtol=2.0 ** -7,
                                           atol=1e-6)
            del fused
        if w.gated and label in ("o", "down"):
            r0 = (3 * torch.randn(w.tokens, lin.out, device="cuda", generator=gen)).to(DT)
            res = r0.clone()
            rlast = torch.empty(w.requests, lin.out, dtype=DT, device="cuda") if w.gather_last else None
            int4_product(lin, x, ws, w.adp, last_out=rlast, epilogue="residual", residual=res)
            xo, _ = add_rms(r0, y, torch.ones(lin.out, device="cuda"))
            assert torch.equal(res, xo), f"{name} {label}: the residual tile differs from add_rms"
            if rlast is not None:
                assert torch.equal(rlast, res[ends])
            if decode:
                xo_bits, _, _ = oracle_add_rms(bf16_bits(r0), bf16_bits(y), np.ones(lin.out, np.float32))
                assert np.array_equal(bf16_bits(res), xo_bits)
            del r0, res, xo
        del x, y, last
    ws.check()
