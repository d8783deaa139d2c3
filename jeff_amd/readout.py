"""The decision head on the HIP library: each request row's option probabilities from its own adapter's readout.

Mirrors the reference's engine/batched_kernels.py:492-559: `readout_logits(hidden, readout_pool, adapters)`,
`option_softmax(logits, adapters, counts, temp_pool)` and `readout_rows(hidden, readout_pool, temp_pool, adapters,
counts)`, with the same arguments, results and ValueError before any launch. The reference's readout has
READOUT_ROWS = 255 options; here the option count is the readout pool's second dimension (at most 256) and the
hidden size at most 2048. Logits are summed in float32 and rounded to bfloat16, as a bfloat16 product rounds its
output; the probabilities follow DecisionModel.forward (options past the row's count get -1e9, division by the
adapter's temperature, softmax)."""

from __future__ import annotations

import torch

from jeff_amd import _lib

READOUT_ROWS = 255  # the reference's option count (engine/batched_kernels.py)


def _check_rows(name: str, t: torch.Tensor, b: int) -> None:
    if t.dtype != torch.int32 or t.dim() != 1 or t.shape[0] != b or not t.is_contiguous() or t.device.type != "cuda":
        raise ValueError(f"{name} must be a contiguous int32 vector of {b} rows on the GPU, got {t.dtype} "
                         f"{tuple(t.shape)} on {t.device}")


def _check_pool(hidden: torch.Tensor, readout_pool: torch.Tensor, what: str) -> None:
    if hidden.dim() != 2 or hidden.dtype != torch.bfloat16 or not hidden.is_contiguous():
        raise ValueError(f"{what}: expected contiguous bfloat16 hidden (B, dim), got {hidden.dtype} "
                         f"{tuple(hidden.shape)}")
    dim = hidden.shape[1]
    if (readout_pool.dim() != 3 or readout_pool.shape[2] != dim or readout_pool.dtype != torch.bfloat16
            or not readout_pool.is_contiguous()):
        raise ValueError(f"{what}: expected contiguous bfloat16 readout_pool (adapters + 1, options, {dim}), got "
                         f"{readout_pool.dtype} {tuple(readout_pool.shape)}")
    if dim % 8 or dim > _lib.READOUT_MAX_DIM or readout_pool.shape[1] > _lib.READOUT_MAX_OPTIONS:
        raise ValueError(f"{what}: the HIP readout takes a hidden size that is a multiple of 8 up to "
                         f"{_lib.READOUT_MAX_DIM} and up to {_lib.READOUT_MAX_OPTIONS} options; got {dim} and "
                         f"{readout_pool.shape[1]}")


def readout_logits(hidden: torch.Tensor, readout_pool: torch.Tensor, adapters: torch.Tensor) -> torch.Tensor:
    """engine/batched_kernels.py:522-536: each row's option logits from its own adapter's readout: hidden (B, dim)
    bf16, readout_pool (adapters + 1, options, dim) bf16. Summed in float32 and rounded to bfloat16. Returns
    (B, options) float32."""
    b = hidden.shape[0] if hidden.dim() == 2 else -1
    _check_rows("adapters", adapters, b)
    _check_pool(hidden, readout_pool, "readout_logits")
    logits = torch.empty(b, readout_pool.shape[1], device=hidden.device, dtype=torch.float32)
    h = _lib.lib()
    stream = torch.cuda.current_stream(hidden.device).cuda_stream
    _lib.check(h.mlora_readout_logits(hidden.data_ptr(), hidden.stride(0), hidden.shape[1], readout_pool.data_ptr(),
                                      readout_pool.stride(0), readout_pool.shape[1], readout_pool.shape[0],
                                      adapters.data_ptr(), b, logits.data_ptr(), stream), "mlora_readout_logits")
    return logits


def option_softmax(logits: torch.Tensor, adapters: torch.Tensor, counts: torch.Tensor,
                   temp_pool: torch.Tensor) -> torch.Tensor:
    """engine/batched_kernels.py:539-553: each row's option probabilities from its logits (B, options) float32:
    options past counts[row] masked, divided by temp_pool[adapters[row]], softmax. Returns (B, options) float32
    (zero past the row's count)."""
    b = logits.shape[0] if logits.dim() == 2 else -1
    _check_rows("adapters", adapters, b)
    _check_rows("counts", counts, b)
    if temp_pool.dim() != 1 or temp_pool.dtype != torch.float32 or not temp_pool.is_contiguous():
        raise ValueError(f"option_softmax: temp_pool must be a contiguous float32 vector (one temperature per adapter "
                         f"row), got shape {tuple(temp_pool.shape)}, {temp_pool.dtype}")
    if (logits.dim() != 2 or logits.dtype != torch.float32 or not logits.is_contiguous()
            or logits.shape[1] > _lib.READOUT_MAX_OPTIONS):
        raise ValueError(f"option_softmax: expected contiguous float32 logits (B, options) with at most "
                         f"{_lib.READOUT_MAX_OPTIONS} options, got {logits.dtype} {tuple(logits.shape)}")
    out = torch.empty_like(logits)
    h = _lib.lib()
    stream = torch.cuda.current_stream(logits.device).cuda_stream
    _lib.check(h.mlora_option_softmax(logits.data_ptr(), logits.shape[1], adapters.data_ptr(), counts.data_ptr(),
                                      temp_pool.data_ptr(), temp_pool.shape[0], b, out.data_ptr(), stream),
               "mlora_option_softmax")
    return out


def readout_rows(hidden: torch.Tensor, readout_pool: torch.Tensor, temp_pool: torch.Tensor, adapters: torch.Tensor,
                 counts: torch.Tensor) -> torch.Tensor:
    """engine/batched_kernels.py:556-559: each row's option probabilities (B, options) float32 (zero past its
    count): its own adapter's readout (readout_logits), its option mask, its adapter's temperature and the softmax
    (option_softmax). Two launches; no copy of any readout."""
    return option_softmax(readout_logits(hidden, readout_pool, adapters), adapters, counts, temp_pool)
