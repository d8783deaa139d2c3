"""INT4 weights of a fused group in the layout the HIP kernels read, and the codec they come from.

Mirrors the kernel part of the reference's engine/int4.py (paths relative to runtime/python/src/jeff_runtime/):
- pack_int4 / unpack_int4: the folder's uint8 (out, in/2), low nibble first, q + 8 (engine/int4.py:183-200);
- dequantize: bf16(q * s), formed in float32 and rounded once (engine/int4.py:203-208);
- KernelInt4, pack_kernel, unpack_kernel: words int32 (in/8, columns), scales bf16 (in/group, columns)
  (engine/int4.py:211-262);
- pack_group: a fused group's matrices stacked along the output, checked against their bf16 copy
  (engine/int4.py:265-277).
Extensions, each opt-in: a group of 128 inputs per scale (g128) and asymmetric zero points (codes c in [0, 15] with a
zero point z in [0, 15] per (group, output): w = bf16((c - z) s)); the symmetric format is z = 8.

These are load-time transforms in torch (as in the reference). The device-side dequantisation export
(`dequantize_kernel`) runs the HIP library."""

from __future__ import annotations

from collections.abc import Mapping, Sequence
from dataclasses import dataclass

import torch

from jeff_amd import _lib

GROUP = 64            # the reference format's inputs per scale (engine/int4.py:39)
GROUPS = (64, 128)    # what the kernels run
LOW, HIGH = -8, 7     # engine/int4.py:40
KERNEL_COLUMNS = 64   # engine/int4.py:211
WORD = 8              # engine/int4.py:212
SYMMETRIC_ZERO = 8
MAX_SCALE = 2.0 ** 120  # above it z * s could overflow float32 inside the kernels' exact dequantisation


class Int4Error(ValueError):
    """A tensor the INT4 layout cannot hold (the reference raises EngineError for these)."""


def pack_int4(q: torch.Tensor) -> torch.Tensor:
    """engine/int4.py:183-193: integers in [-8, 7] (out, in) as uint8 (out, in/2), q + 8, low nibble first."""
    if q.dtype.is_floating_point or q.dtype == torch.bool or q.dim() != 2 or q.shape[1] % 2:
        raise Int4Error(f"pack_int4 takes a 2-D integer tensor with an even number of columns; got {q.dtype} "
                        f"{tuple(q.shape)}")
    low, high = int(q.min()), int(q.max())
    if low < LOW or high > HIGH:
        raise Int4Error(f"Integers from {low} to {high}; int4 holds integers in [{LOW}, {HIGH}] only")
    stored = (q.to(torch.int16) - LOW).to(torch.uint8)
    return (stored[:, 0::2] | (stored[:, 1::2] << 4)).contiguous()


def unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    """engine/int4.py:196-200: uint8 (out, in/2) -> int8 (out, in) in [-8, 7]."""
    low = (packed & 0xF).to(torch.int8) + LOW
    high = (packed >> 4).to(torch.int8) + LOW
    return torch.stack((low, high), dim=-1).reshape(packed.shape[0], packed.shape[1] * 2)


def dequantize(q: torch.Tensor, scales: torch.Tensor, group: int = GROUP,
               zeros: torch.Tensor | None = None) -> torch.Tensor:
    """engine/int4.py:203-208: bf16((q - z) * s) per weight, the product exact in float32, rounded once.
    q: (out, in) integers, in [-8, 7] when zeros is None (z = 0 on q, i.e. the stored nibble minus 8), else the
    codes in [0, 15] with zeros (out, in/group) in [0, 15]."""
    out, inputs = q.shape
    diff = q.to(torch.float32).reshape(out, inputs // group, group)
    if zeros is not None:
        diff = diff - zeros.to(torch.float32)[..., None]
    return (diff * scales.to(torch.float32)[..., None]).reshape(out, inputs).to(torch.bfloat16)


@dataclass(frozen=True)
class KernelInt4:
    """engine/int4.py:215-230: a fused group's integers in the kernel layout.
    words int32 (in/8, columns): word i of column c holds inputs 8i..8i+7, input 8i+j as its code in bits 4j..4j+3;
    scales bf16 (in/group, columns); zeros uint8 (in/group, columns) or None (symmetric: z = 8);
    columns = out rounded up to 64, padding columns hold code 8 (zero 8) and scale 1: zero weights."""
    words: torch.Tensor
    scales: torch.Tensor
    out: int
    zeros: torch.Tensor | None = None
    group: int = GROUP

    def nbytes(self) -> int:
        n = self.words.numel() * self.words.element_size() + self.scales.numel() * self.scales.element_size()
        return n + (0 if self.zeros is None else self.zeros.numel())

    @property
    def columns(self) -> int:
        return int(self.words.shape[1])

    @property
    def k(self) -> int:
        return int(self.words.shape[0]) * WORD

    def abi(self) -> _lib.Int4:
        """The C description of these weights (pointers stay valid while this object lives)."""
        return _lib.Int4(self.words.data_ptr(), self.scales.data_ptr(),
                         0 if self.zeros is None else self.zeros.data_ptr(), self.k, self.columns, self.out,
                         self.group)


def _check_scales(scales: torch.Tensor, out: int, inputs: int, group: int) -> None:
    if scales.dtype != torch.bfloat16 or tuple(scales.shape) != (out, inputs // group):
        raise Int4Error(f"pack_kernel: the scales must be bfloat16 ({out}, {inputs // group}); got {scales.dtype} "
                        f"{tuple(scales.shape)}")
    f = scales.float()
    if not bool(torch.isfinite(f).all()) or not bool((f > 0).all()) or not bool((f < MAX_SCALE).all()):
        raise Int4Error("pack_kernel: every scale must be finite, positive and below 2^120")


def _pack_codes(codes: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor | None, group: int) -> KernelInt4:
    out, inputs = codes.shape
    columns = -(-out // KERNEL_COLUMNS) * KERNEL_COLUMNS
    stored = torch.full((columns, inputs), SYMMETRIC_ZERO, dtype=torch.int32, device=codes.device)
    stored[:out] = codes.to(torch.int32)
    stored = stored.T.contiguous()  # (in, columns)
    words = torch.zeros(inputs // WORD, columns, dtype=torch.int32, device=codes.device)
    for j in range(WORD):
        words |= stored[j::WORD] << (4 * j)  # j = 7 sets the sign bit for codes >= 8; the kernels mask each nibble
    padded = torch.ones(columns, inputs // group, dtype=torch.bfloat16, device=codes.device)
    padded[:out] = scales
    z = None
    if zeros is not None:
        zp = torch.full((columns, inputs // group), SYMMETRIC_ZERO, dtype=torch.uint8, device=codes.device)
        zp[:out] = zeros.to(torch.uint8)
        z = zp.T.contiguous()
    return KernelInt4(words, padded.T.contiguous(), out, z, group)


def pack_kernel(q: torch.Tensor, scales: torch.Tensor, group: int = GROUP) -> KernelInt4:
    """engine/int4.py:233-255: integers (out, in) in [-8, 7] and bf16 scales (out, in/group), symmetric."""
    if q.dtype.is_floating_point or q.dtype == torch.bool or q.dim() != 2 or group not in GROUPS or q.shape[1] % group:
        raise Int4Error(f"pack_kernel takes a 2-D integer tensor whose inputs are a multiple of {group} (a group of "
                        f"{GROUPS}); got {q.dtype} {tuple(q.shape)}")
    out, inputs = q.shape
    _check_scales(scales, out, inputs, group)
    low, high = int(q.min()), int(q.max())
    if low < LOW or high > HIGH:
        raise Int4Error(f"Integers from {low} to {high}; int4 holds integers in [{LOW}, {HIGH}] only")
    return _pack_codes((q.to(torch.int16) - LOW).to(torch.uint8), scales, None, group)


def pack_kernel_asym(codes: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor,
                     group: int = 128) -> KernelInt4:
    """Asymmetric weights: codes (out, in) in [0, 15], bf16 scales and uint8 zero points (out, in/group) in [0, 15];
    w = bf16((c - z) s)."""
    if codes.dtype.is_floating_point or codes.dim() != 2 or group not in GROUPS or codes.shape[1] % group:
        raise Int4Error(f"pack_kernel_asym takes 2-D integer codes whose inputs are a multiple of {group} (a group "
                        f"of {GROUPS}); got {codes.dtype} {tuple(codes.shape)}")
    out, inputs = codes.shape
    _check_scales(scales, out, inputs, group)
    if tuple(zeros.shape) != (out, inputs // group) or zeros.dtype.is_floating_point:
        raise Int4Error(f"pack_kernel_asym: the zero points must be integers ({out}, {inputs // group})")
    for name, t in (("codes", codes), ("zero points", zeros)):
        if int(t.min()) < 0 or int(t.max()) > 15:
            raise Int4Error(f"pack_kernel_asym: {name} must lie in [0, 15]")
    return _pack_codes(codes, scales, zeros, group)


def _codes(packed: KernelInt4) -> torch.Tensor:
    nibbles = torch.stack([(packed.words >> (4 * j)) & 0xF for j in range(WORD)], dim=1)  # (in/8, 8, columns)
    return nibbles.reshape(-1, packed.columns).T[:packed.out]


def unpack_kernel(packed: KernelInt4) -> tuple[torch.Tensor, torch.Tensor]:
    """engine/int4.py:258-262: (q int8 (out, in), scales (out, in/group)) of a symmetric layout."""
    if packed.zeros is not None:
        raise Int4Error("unpack_kernel reads a symmetric layout; this one has zero points (unpack_kernel_asym)")
    q = (_codes(packed) + LOW).to(torch.int8)
    return q.contiguous(), packed.scales.T[:packed.out].contiguous()


def unpack_kernel_asym(packed: KernelInt4) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(codes uint8 (out, in), scales, zero points (out, in/group)); a symmetric layout reports zero points 8."""
    codes = _codes(packed).to(torch.uint8).contiguous()
    scales = packed.scales.T[:packed.out].contiguous()
    if packed.zeros is None:
        zeros = torch.full_like(scales, SYMMETRIC_ZERO, dtype=torch.uint8)
    else:
        zeros = packed.zeros.T[:packed.out].contiguous()
    return codes, scales, zeros


def pack_group(stored: Mapping[str, tuple[torch.Tensor, torch.Tensor]], names: Sequence[str],
               dequantised: torch.Tensor) -> KernelInt4:
    """engine/int4.py:265-277: the kernel layout of the fused group `names` from the folder's stored matrices
    ({name: (qweight uint8 (out, in/2), scales bf16 (out, in/G))}, as read_int4_file gives them), packed on the
    device of `dequantised`, the group's bfloat16 weights; those must be bf16(q * s) of the same integers and scales
    bit for bit (Int4Error naming the group otherwise). The packing itself is int4_file.pack_stored_group's."""
    from jeff_amd.int4_file import StoredInt4, pack_stored_group
    return pack_stored_group({name: StoredInt4(*stored[name]) for name in names}, names, dequantised.device,
                             dequantised)


def dequantize_kernel(packed: KernelInt4) -> torch.Tensor:
    """bf16((c - z) s) of a kernel layout as (out, in), computed by the HIP library on the layout's device (the
    export the bit-exactness tests read)."""
    h = _lib.lib()
    if packed.words.device.type != "cuda":
        raise ValueError("dequantize_kernel runs on the GPU: the packed weights must be on a cuda device")
    out = torch.empty(packed.out, packed.k, dtype=torch.bfloat16, device=packed.words.device)
    desc = packed.abi()
    stream = torch.cuda.current_stream(packed.words.device).cuda_stream
    _lib.check(h.mlora_dequant(desc, out.data_ptr(), stream), "mlora_dequant")
    return out
