"""A whole decoder pass recorded as one HIP graph (jeff_amd.passes) and replayed for new batches (needs a gfx950 GPU;
marked gpu): two layers of qkv, o + residual add + RMSNorm, gate_up with SiLU(gate) * up, down + residual add +
RMSNorm, the last-token gather and the decision head, with ragged requests over a pool of adapters of mixed ranks,
the residual adds and the gated activation in the products' output tiles. Each replay, after new adapter ids,
sequence lengths, inputs and option counts are copied into the recorded tensors (engine/batched_path.py:589-603),
must give the bits an eager run of the same body gives, and so must the reference's sequence of separate launches
(add_rms, silu_mul); every kernel it runs is checked against the oracle in its own tests."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from jeff_amd import _lib
from jeff_amd.fast_path import DT, AdapterPool, Lin, Workspace
from jeff_amd.int4 import pack_kernel_asym
from jeff_amd.passes import DecoderInputs, RecordedPass, decoder_pass

pytestmark = pytest.mark.gpu

HIDDEN, INTER, Q, KV, OPTIONS = 512, 1024, 512, 256, 40


@pytest.fixture(scope="module", autouse=True)
def gpu() -> None:
    assert torch.cuda.is_available(), "the gpu tests need an AMD GPU"
    _lib.lib()


def int4(out: int, k: int, g: torch.Generator):
    codes = torch.randint(0, 16, (out, k), generator=g, device="cuda", dtype=torch.uint8)
    zeros = torch.randint(0, 16, (out, k // 128), generator=g, device="cuda", dtype=torch.uint8)
    scales = (torch.rand(out, k // 128, generator=g, device="cuda") * 0.015 + 0.005).to(DT)
    return pack_kernel_asym(codes, scales, zeros, 128)


def test_a_recorded_decoder_pass_replays_new_batches_as_an_eager_run() -> None:
    g = torch.Generator(device="cuda").manual_seed(11)
    groups = {"qkv": (["q_proj", "k_proj", "v_proj"], [Q, KV, KV], HIDDEN), "o": (["o_proj"], [HIDDEN], Q),
              "gate_up": (["gate_proj", "up_proj"], [INTER, INTER], HIDDEN), "down": (["down_proj"], [HIDDEN], INTER)}
    layers = []
    for i in range(2):
        layer = {}
        for label, (names, sizes, k) in groups.items():
            lin = Lin([f"layers.{i}.{n}" for n in names], sizes=sizes, k=k, ranks=[32] * len(names))
            lin.int4 = int4(lin.out, k, g)
            layer[label] = lin
        layers.append(layer)
    lins = [lin for layer in layers for lin in layer.values()]
    pool = AdapterPool(lins, 8)
    for a in range(1, 9):
        r = (8, 16, 32)[a % 3]
        updates = {}
        for lin in lins:
            for name, n in zip(lin.names, lin.sizes):
                updates[name] = ((torch.randn(r, lin.k, generator=g, device="cuda") / 32).to(DT),
                                 (torch.randn(n, r, generator=g, device="cuda") * 0.04).to(DT))
        pool.add_adapter(f"a{a}", updates)
    norms = [tuple((1 + 0.1 * torch.randn(HIDDEN, generator=g, device="cuda")).float() for _ in range(2))
             for _ in layers]
    final_norm = (1 + 0.1 * torch.randn(HIDDEN, generator=g, device="cuda")).float()
    readout_pool = (0.05 * torch.randn(9, OPTIONS, HIDDEN, generator=g, device="cuda")).to(DT)
    temp_pool = 0.5 + 1.5 * torch.rand(9, generator=g, device="cuda")

    requests, tokens = 12, 600
    rng = np.random.default_rng(5)

    def batch():
        cuts = np.sort(rng.choice(np.arange(1, tokens), requests - 1, replace=False))
        cu = np.concatenate([[0], cuts, [tokens]]).astype(np.int32)
        return (rng.integers(0, 9, requests).astype(np.int32), cu, rng.integers(1, OPTIONS + 1, requests))

    ids, cu, counts = batch()
    inputs = DecoderInputs(x=torch.randn(tokens, HIDDEN, generator=g, device="cuda").to(DT),
                           adp=torch.tensor(ids, device="cuda"), cu_seqlens=torch.tensor(cu, device="cuda"),
                           ends=torch.tensor(cu[1:] - 1, device="cuda").long(),
                           counts=torch.tensor(counts.astype(np.int32), device="cuda"))
    ws = Workspace(tokens, 1, max_rank=max(lin.rank for lin in lins), max_requests=requests)
    body = decoder_pass(layers, norms, final_norm, ws, inputs, tokens, readout_pool, temp_pool)
    unfused = decoder_pass(layers, norms, final_norm, ws, inputs, tokens, readout_pool, temp_pool, fused=False)
    recorded = RecordedPass(body)
    seen = []
    for _ in range(3):
        ids, cu, counts = batch()
        inputs.adp.copy_(torch.from_numpy(ids))
        inputs.cu_seqlens.copy_(torch.from_numpy(cu))
        inputs.ends.copy_(torch.from_numpy(cu[1:] - 1))
        inputs.counts.copy_(torch.from_numpy(counts.astype(np.int32)))
        inputs.x.copy_(torch.randn(tokens, HIDDEN, generator=g, device="cuda").to(DT))
        probs = recorded.replay().clone()
        torch.cuda.synchronize()
        eager = body()
        torch.cuda.synchronize()
        assert torch.equal(probs, eager)
        assert torch.equal(unfused(), eager)  # the epilogues in the output tiles give the separate launches' bits
        assert bool(torch.isfinite(probs).all())
        sums = probs.sum(1)
        assert bool(((sums - 1).abs() < 1e-4).all())
        assert not probs[torch.arange(requests), torch.as_tensor(counts, device="cuda") - 1].eq(0).any()
        seen.append(probs)
    assert not torch.equal(seen[0], seen[1])  # new batches give new answers
