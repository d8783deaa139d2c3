"""Pass-level recording: a whole pass (routing, every fused group's product, the element-wise steps between them, the
decision head) recorded once as a HIP graph and replayed for every batch, the way the reference's BatchedPath records
its passes (engine/batched_path.py:353-417: the inputs filled, two warm-up runs on the recording stream outside the
capture, the capture into a graph memory pool; engine/batched_path.py:589-609: each batch copies its rows into the
recorded input tensors and replays).

The products of a pass share one routing launch only inside the capture that recorded it (Workspace.routed), so a
replay routes the adapter ids and sequence lengths it finds in the recorded tensors, whatever the warm-up saw.
`decoder_pass` is the layer body of the configurations' decoder (per layer: qkv, o with the residual add and
RMSNorm, gate_up with SiLU(gate) * up, down with the residual add and RMSNorm; the last token of each request
gathered; the decision head), written with this package's calls, either as the reference's sequence of products and
element-wise launches (engine/fast_path.py:80-156) or with those element-wise steps in the products' output tiles
(the residual add in o's and down's, SiLU(gate) * up in gate_up's), which give the same bits; attention, which this
build does not cover, is stood in for by the qkv product's first hidden-size columns."""

from __future__ import annotations

from collections.abc import Callable, Sequence
from dataclasses import dataclass
from typing import Any

import torch

from jeff_amd.epilogues import add_rms, rms, silu_mul
from jeff_amd.fast_path import Lin, Workspace
from jeff_amd.int4_kernels import int4_product
from jeff_amd.readout import readout_rows


class RecordedPass:
    """`body()` recorded as a HIP graph: run `warmups` times on the recording stream outside the capture, then
    captured once (into `pool`, a graph memory pool handle, or a private one). `outputs` are the tensors the captured
    body returned; `replay()` runs the graph on the current stream and returns them."""

    def __init__(self, body: Callable[[], Any], *, warmups: int = 2, stream: torch.cuda.Stream | None = None,
                 pool: Any = None) -> None:
        if warmups < 1:
            raise ValueError("a pass is run at least once before it is recorded (its first run sizes its buffers)")
        self.stream = stream if stream is not None else torch.cuda.Stream()
        self.stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(self.stream):
            for _ in range(warmups):
                body()
        self.stream.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, pool=pool, stream=self.stream):
            self.outputs = body()
        torch.cuda.current_stream().wait_stream(self.stream)

    def replay(self) -> Any:
        self.graph.replay()
        return self.outputs


@dataclass
class DecoderInputs:
    """The tensors a recorded decoder pass reads: each batch copies its rows into them before a replay."""
    x: torch.Tensor              # (tokens, hidden) bf16: the residual stream entering the first layer
    adp: torch.Tensor            # (requests,) int32 pool rows
    cu_seqlens: torch.Tensor     # (requests + 1,) int32 token offsets
    ends: torch.Tensor           # (requests,) int64: each request's last token (cu_seqlens[1:] - 1)
    counts: torch.Tensor         # (requests,) int32 answer options per request


def decoder_pass(layers: Sequence[dict[str, Lin]], norms: Sequence[tuple[torch.Tensor, torch.Tensor]],
                 final_norm: torch.Tensor, ws: Workspace, inputs: DecoderInputs, tokens: int,
                 readout_pool: torch.Tensor, temp_pool: torch.Tensor, fused: bool = True) -> Callable[[], torch.Tensor]:
    """The body of one decoder pass over `layers` ({"qkv", "o", "gate_up", "down"} per layer, gate_up a gate and an
    up matrix of one width) with their RMSNorm weights (1 + weight, float32) before attention and before the MLP;
    returns a callable that runs the pass and returns the decision head's option probabilities (requests, options).
    `tokens` is cu_seqlens' last value (the pass size the graph is recorded at). fused: the residual adds and
    SiLU(gate) * up in the products' output tiles (the residual stream a copy of inputs.x that the o and down
    products update in place); else the reference's separate add_rms and silu_mul launches."""
    pool_rows = layers[0]["qkv"].pool.shape[0]
    hidden = layers[0]["o"].out

    def body_fused() -> torch.Tensor:
        ws.route(inputs.adp, pool_rows, tokens=tokens, cu_seqlens=inputs.cu_seqlens)
        x = inputs.x.clone()  # the residual stream
        for layer, (attn_norm, mlp_norm) in zip(layers, norms):
            qkv = int4_product(layer["qkv"], rms(x, attn_norm), ws, inputs.adp)
            # qkv's columns stand in for attention
            int4_product(layer["o"], qkv[:, :hidden], ws, inputs.adp, epilogue="residual", residual=x)
            act = int4_product(layer["gate_up"], rms(x, mlp_norm), ws, inputs.adp, epilogue="silu_mul")
            int4_product(layer["down"], act, ws, inputs.adp, epilogue="residual", residual=x)
        # the decision head reads each request's last token after the last residual add and the final norm
        # (engine/batched_path.py:274-276)
        hl = rms(x.index_select(0, inputs.ends), final_norm)
        return readout_rows(hl, readout_pool, temp_pool, inputs.adp, inputs.counts)

    def body_unfused() -> torch.Tensor:
        ws.route(inputs.adp, pool_rows, tokens=tokens, cu_seqlens=inputs.cu_seqlens)
        x = inputs.x
        _, h = add_rms(x, None, norms[0][0])
        d = None
        for i, (layer, (_, mlp_norm)) in enumerate(zip(layers, norms)):
            if i > 0:
                x, h = add_rms(x, d, norms[i][0])
            qkv = int4_product(layer["qkv"], h, ws, inputs.adp)
            d = int4_product(layer["o"], qkv[:, :hidden], ws, inputs.adp)
            x, h = add_rms(x, d, mlp_norm)
            act = silu_mul(int4_product(layer["gate_up"], h, ws, inputs.adp))
            d = int4_product(layer["down"], act, ws, inputs.adp)
        _, hl = add_rms(x.index_select(0, inputs.ends), d.index_select(0, inputs.ends), final_norm)
        return readout_rows(hl, readout_pool, temp_pool, inputs.adp, inputs.counts)

    return body_fused if fused else body_unfused
