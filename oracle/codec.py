"""INT4 codec, kernel word layout and dequantisation, restated in numpy (test infrastructure; see oracle/__init__.py).

Integers are handled as 4-bit codes c in [0, 15]. The reference's symmetric format stores q in [-8, 7] as the nibble
q + 8 (`engine/int4.py:183-193`), i.e. c = q + 8 with the zero point z = 8. The asymmetric variant keeps one integer
zero point z in [0, 15] per (group, output) and the same nibbles. bfloat16 values are uint16 bit patterns."""

from __future__ import annotations

import numpy as np

from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

SYMMETRIC_ZERO = 8     # engine/int4.py:40,192 (LOW = -8: stored = q - LOW)
KERNEL_COLUMNS = 64    # engine/int4.py:211
WORD = 8               # engine/int4.py:212
BF16_ONE = 0x3F80


def pack_int4(q: np.ndarray) -> np.ndarray:
    """engine/int4.py:183-193: integers in [-8, 7], shape (out, in), as uint8 (out, in/2), q + 8 per nibble, low
    nibble = even input."""
    q = np.asarray(q)
    if q.ndim != 2 or q.shape[1] % 2 or q.min() < -8 or q.max() > 7:
        raise ValueError("pack_int4 takes integers in [-8, 7] with an even number of columns")
    stored = (q.astype(np.int16) + 8).astype(np.uint8)
    return (stored[:, 0::2] | (stored[:, 1::2] << 4)).astype(np.uint8)


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    """engine/int4.py:196-200: uint8 (out, in/2) -> int8 (out, in) in [-8, 7]."""
    low = (packed & 0xF).astype(np.int8) - 8
    high = (packed >> 4).astype(np.int8) - 8
    return np.stack((low, high), axis=-1).reshape(packed.shape[0], packed.shape[1] * 2)


def pack_kernel(codes: np.ndarray, scales: np.ndarray, zeros: np.ndarray | None = None,
                group: int = 64) -> tuple[np.ndarray, np.ndarray, np.ndarray | None, int]:
    """engine/int4.py:233-255, generalised to a group of 64 or 128 inputs and optional zero points.

    codes uint8 (out, in) in [0, 15]; scales bf16 bits (out, in/group); zeros uint8 (out, in/group) or None (z = 8).
    Returns (words int32 (in/8, columns), scales bf16 bits (in/group, columns), zeros uint8 (in/group, columns) or
    None, out): word i of column c holds inputs 8i..8i+7, input 8i+j in bits 4j..4j+3; columns = out rounded up to 64;
    padding columns hold code 8, zero 8 (when zeros are given) and scale 1.0, i.e. weight 0."""
    codes = np.asarray(codes)
    out, inputs = codes.shape
    if inputs % group or codes.min() < 0 or codes.max() > 15:
        raise ValueError("codes must be in [0, 15] with inputs a multiple of the group")
    columns = -(-out // KERNEL_COLUMNS) * KERNEL_COLUMNS
    stored = np.full((columns, inputs), SYMMETRIC_ZERO, dtype=np.uint32)
    stored[:out] = codes
    stored = stored.T  # (in, columns)
    words = np.zeros((inputs // WORD, columns), dtype=np.uint32)
    for j in range(WORD):
        words |= stored[j::WORD] << np.uint32(4 * j)
    padded_scales = np.full((columns, inputs // group), BF16_ONE, dtype=np.uint16)
    padded_scales[:out] = scales
    padded_zeros = None
    if zeros is not None:
        padded_zeros = np.full((columns, inputs // group), SYMMETRIC_ZERO, dtype=np.uint8)
        padded_zeros[:out] = zeros
        padded_zeros = np.ascontiguousarray(padded_zeros.T)
    return words.view(np.int32), np.ascontiguousarray(padded_scales.T), padded_zeros, out


def unpack_kernel(words: np.ndarray, scales: np.ndarray, zeros: np.ndarray | None,
                  out: int) -> tuple[np.ndarray, np.ndarray, np.ndarray | None]:
    """engine/int4.py:258-262: the inverse of pack_kernel, padding columns dropped."""
    u = np.asarray(words).view(np.uint32)
    nibbles = np.stack([(u >> np.uint32(4 * j)) & 0xF for j in range(WORD)], axis=1)  # (in/8, 8, columns)
    codes = nibbles.reshape(-1, u.shape[1]).T[:out].astype(np.uint8)
    z = None if zeros is None else np.ascontiguousarray(zeros.T[:out])
    return np.ascontiguousarray(codes), np.ascontiguousarray(scales.T[:out]), z


def dequantize(codes: np.ndarray, scales: np.ndarray, zeros: np.ndarray | None = None,
               group: int = 64) -> np.ndarray:
    """engine/int4.py:203-208 with zero points: bf16((c - z) * s) per weight, the product formed in float32 (exact:
    a 5-bit signed integer times an 8-bit-significand bfloat16) and rounded once to nearest even.
    codes (out, in) in [0, 15]; scales bf16 bits (out, in/group); zeros (out, in/group) or None (z = 8).
    Returns bf16 bits (out, in)."""
    out, inputs = codes.shape
    z = np.full(scales.shape, SYMMETRIC_ZERO, dtype=np.int32) if zeros is None else zeros.astype(np.int32)
    diff = (codes.astype(np.int32).reshape(out, inputs // group, group) - z[..., None]).astype(np.float32)
    with np.errstate(over="ignore"):  # scales near the bfloat16 maximum overflow to inf, as float32 does
        product = diff * bf16_bits_to_f32(scales)[..., None]
    return f32_to_bf16_bits(product.reshape(out, inputs))


def dequantize_kernel(words: np.ndarray, scales: np.ndarray, zeros: np.ndarray | None, out: int,
                      group: int) -> np.ndarray:
    """The dequantised weights bf16 bits (out, in) of a kernel-layout group (what the HIP dequant export returns)."""
    codes, s, z = unpack_kernel(words, scales, zeros, out)
    return dequantize(codes, s, z, group)
