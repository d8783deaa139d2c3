"""The oracle's bfloat16 rounding, INT4 codec, kernel layout and dequantisation, pinned without importing the
reference: its tests' golden vectors (tests/golden/reference_vectors.json), an independent rounding of exact float64
products, and brute force over every code, zero point and finite positive bfloat16 scale."""

from __future__ import annotations

import json
import os
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits
from oracle.codec import dequantize, pack_int4, pack_kernel, unpack_int4, unpack_kernel

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.json")))
BF16_MAX = float.fromhex("0x1.fep127")


def test_rne_matches_torch_on_ties_random_bits_and_specials() -> None:
    rng = np.random.default_rng(0)
    upper = rng.integers(0, 1 << 16, 200_000, dtype=np.uint32)
    ties = (upper << 16) | 0x8000                                   # exactly half way: even rule decides
    near = (upper << 16) | rng.integers(0, 1 << 16, 200_000, dtype=np.uint32)
    specials = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x00000001, 0x007FFFFF, 0x7F7FFFFF, 0x7F7F8000,
                         0x3F808000, 0x3F818000], dtype=np.uint32)
    bits = np.concatenate([ties, near, specials])
    vals = bits.view(np.float32)
    keep = ~np.isnan(vals)
    ours = f32_to_bf16_bits(vals[keep])
    theirs = torch.from_numpy(vals[keep].copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    assert np.isnan(bf16_bits_to_f32(f32_to_bf16_bits(np.array([np.nan], dtype=np.float32)))).all()


def test_rne_matches_exact_rational_rounding_on_a_sample() -> None:
    rng = np.random.default_rng(1)
    vals = (rng.standard_normal(2000) * 10.0 ** rng.integers(-6, 6, 2000)).astype(np.float32)
    got = bf16_bits_to_f32(f32_to_bf16_bits(vals)).astype(np.float64)
    for v, g in zip(vals.tolist(), got.tolist()):
        exact = Fraction(v)
        m, e = np.frexp(abs(v))
        quantum = Fraction(2) ** (int(e) - 8)
        q, r = divmod(abs(exact), quantum)
        if r > quantum / 2 or (r == quantum / 2 and q % 2 == 1):
            q += 1
        want = float(q * quantum) * (1 if v >= 0 else -1)
        assert g == want, (v, g, want)


def test_folder_codec_golden_byte_and_round_trip() -> None:
    g = GOLDEN["folder_byte"]
    q = np.tile(np.arange(-8, 8, dtype=np.int8), (3, 8))
    packed = pack_int4(q)
    assert packed.dtype == np.uint8 and packed.shape == (3, 64)
    assert int(packed[0, 0]) == g["byte"]
    assert np.array_equal(unpack_int4(packed), q)
    with pytest.raises(ValueError):
        pack_int4(np.full((2, 64), 8))


def _words_by_definition(codes: np.ndarray) -> np.ndarray:
    """Scalar construction of the kernel words straight from the layout's definition (input 8i+j in bits 4j..4j+3
    of word i, column c = output c)."""
    out, inputs = codes.shape
    words = np.zeros((inputs // 8, out), dtype=np.uint64)
    for i in range(inputs // 8):
        for c in range(out):
            w = 0
            for j in range(8):
                w |= int(codes[c, 8 * i + j]) << (4 * j)
            words[i, c] = w
    return words.astype(np.uint32)


def test_kernel_layout_golden_word_and_round_trip() -> None:
    g = GOLDEN["kernel_word"]
    rng = np.random.default_rng(0)
    q = rng.integers(-8, 8, (g["rows"], g["inputs"]))
    q[0, :8] = g["q_inputs_0_to_7_of_column_0"]
    scales = f32_to_bf16_bits((rng.random((g["rows"], g["inputs"] // 64)) + 0.01).astype(np.float32))
    codes = (q + 8).astype(np.uint8)
    words, s, z, out = pack_kernel(codes, scales, None, 64)
    assert list(words.shape) == g["words_shape"] and list(s.shape) == g["scales_shape"] and z is None
    assert int(words.view(np.uint32)[0, 0]) == int(g["word_0_0"], 16)
    assert words.nbytes + s.nbytes == g["nbytes"]
    assert np.array_equal(words.view(np.uint32), _words_by_definition(codes))
    back_c, back_s, _ = unpack_kernel(words, s, None, out)
    assert np.array_equal(back_c, codes) and np.array_equal(back_s, scales)


def test_kernel_layout_pads_outputs_with_zero_weights() -> None:
    g = GOLDEN["kernel_padding"]
    rng = np.random.default_rng(1)
    codes = rng.integers(0, 16, (g["out"], g["inputs"])).astype(np.uint8)
    scales = f32_to_bf16_bits(rng.random((g["out"], g["inputs"] // 64)).astype(np.float32) + 0.01)
    words, s, _, out = pack_kernel(codes, scales, None, 64)
    assert list(words.shape) == g["words_shape"] and list(s.shape) == g["scales_shape"]
    assert (words.view(np.uint32)[:, out:] == int(g["padding_word"], 16)).all()
    assert (bf16_bits_to_f32(s[:, out:]) == g["padding_scale"]).all()
    zeros = rng.integers(0, 16, (g["out"], g["inputs"] // 64)).astype(np.uint8)
    _, _, z, _ = pack_kernel(codes, scales, zeros, 64)
    assert (z[:, out:] == 8).all() and np.array_equal(z[:, :out].T, zeros)


def test_group_128_is_group_64_with_each_scale_duplicated() -> None:
    rng = np.random.default_rng(2)
    codes = rng.integers(0, 16, (64, 512)).astype(np.uint8)
    s128 = f32_to_bf16_bits((rng.random((64, 4)) * 0.015 + 0.005).astype(np.float32))
    z128 = rng.integers(0, 16, (64, 4)).astype(np.uint8)
    w128 = dequantize(codes, s128, z128, 128)
    w64 = dequantize(codes, np.repeat(s128, 2, axis=1), np.repeat(z128, 2, axis=1), 64)
    assert np.array_equal(w128, w64)


def test_dequant_golden_rounding() -> None:
    g = GOLDEN["dequant_rounding"]
    codes = np.full((1, 64), g["q"] + 8, dtype=np.uint8)
    scales = f32_to_bf16_bits(np.array([[g["scale"]]], dtype=np.float32))
    assert float(bf16_bits_to_f32(scales)[0, 0]) == g["scale"]
    assert float(bf16_bits_to_f32(dequantize(codes, scales))[0, 0]) == g["bf16_result"]


def _rne_float64(v: np.ndarray) -> np.ndarray:
    """Round exact float64 values to bfloat16 by exponent/quantum arithmetic (independent of the bit trick)."""
    _, e = np.frexp(np.abs(v))
    quantum = np.ldexp(1.0, np.maximum(e - 8, -133))       # bfloat16 subnormals: quantum 2^-133
    r = np.rint(v / quantum) * quantum                       # np.rint: halves to even
    return np.where(np.abs(r) > BF16_MAX, np.copysign(np.inf, v), r)


def test_dequant_brute_force_every_code_zero_and_positive_scale() -> None:
    """16 codes x 16 zero points x every finite positive bfloat16 scale (32,640): about 8.4 million weights."""
    all_bits = np.arange(1, 0x7F80, dtype=np.uint16)         # +min subnormal .. +max finite
    scales = bf16_bits_to_f32(all_bits).astype(np.float64)
    diffs = np.arange(-15, 16, dtype=np.float64)             # every (c - z)
    exact = diffs[:, None] * scales[None, :]                 # exact in float64 (13 significant bits at most)
    f32 = (diffs[:, None].astype(np.float32) * scales[None, :].astype(np.float32))
    finite = np.isfinite(f32)
    assert np.array_equal(f32[finite].astype(np.float64), exact[finite])   # the float32 product is exact
    want = _rne_float64(exact)
    codes = np.arange(16, dtype=np.uint8)[:, None].repeat(64, axis=1)       # (16 rows = codes, 64 inputs)
    for z in range(16):
        for start in range(0, all_bits.size, 4096):
            chunk = all_bits[start:start + 4096]
            c = np.repeat(codes[None], chunk.size, axis=0).reshape(-1, 64)
            s = np.repeat(chunk, 16)[:, None]
            zz = np.full_like(s, z, dtype=np.uint8)
            w = bf16_bits_to_f32(dequantize(c, s, zz, 64)[:, 0]).astype(np.float64).reshape(chunk.size, 16)
            for code in range(16):
                assert np.array_equal(w[:, code], want[code - z + 15, start:start + chunk.size]), (code, z, start)
