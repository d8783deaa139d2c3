"""INT4 checkpoint ingestion (jeff_amd.int4_file): the reference's int4.safetensors (engine/int4.py:280-325) read
strictly into the kernel layout, plus the zero-point / group-128 extension. CPU only."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from jeff_amd.int4 import Int4Error, pack_int4, pack_kernel, pack_kernel_asym, unpack_kernel, unpack_kernel_asym
from jeff_amd.int4_file import (StoredInt4, attach_int4_file, dequantize_stored, file_sha256, pack_stored_group,
                                read_int4_file, stored_from_codes, write_int4_file)
from oracle.codec import dequantize as oracle_dequantize


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> its bit patterns (uint16), the oracle's representation."""
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(b.astype(np.uint16).view(np.int16)).view(torch.bfloat16)


def sym_matrix(out: int, inputs: int, seed: int) -> tuple[torch.Tensor, torch.Tensor, StoredInt4]:
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(-8, 8, (out, inputs), generator=g, dtype=torch.int8)
    s = (torch.rand(out, inputs // 64, generator=g) * 0.02 + 0.001).to(torch.bfloat16)
    return q, s, StoredInt4(pack_int4(q), s)


def test_reference_format_round_trip_and_golden_byte(tmp_path) -> None:
    q, s, m = sym_matrix(96, 256, 0)
    q[0, :2] = torch.tensor([-8, -7], dtype=torch.int8)  # the reference's golden byte (tests/test_int4.py:211-219)
    m = StoredInt4(pack_int4(q), s)
    assert int(m.qweight[0, 0]) == (-8 + 8) | ((-7 + 8) << 4)
    sha = write_int4_file(tmp_path / "int4.safetensors", {"layers.0.mlp.down_proj": m})
    assert sha == file_sha256(tmp_path / "int4.safetensors")
    got = read_int4_file(tmp_path / "int4.safetensors", sha, {"layers.0.mlp.down_proj": (96, 256)})
    back = got["layers.0.mlp.down_proj"]
    assert torch.equal(back.qweight, m.qweight) and torch.equal(back.scales, s) and back.zeros is None
    assert back.group == 64
    packed = pack_stored_group(got, ["layers.0.mlp.down_proj"], "cpu")
    q2, s2 = unpack_kernel(packed)
    assert torch.equal(q2, q) and torch.equal(s2, s)
    assert torch.equal(packed.words, pack_kernel(q, s).words)


def test_group_is_packed_with_its_bf16_weights_checked_bit_for_bit(tmp_path) -> None:
    names = ["layers.0.self_attn.q_proj", "layers.0.self_attn.k_proj"]
    mats = {names[0]: sym_matrix(128, 128, 1), names[1]: sym_matrix(64, 128, 2)}
    sha = write_int4_file(tmp_path / "int4.safetensors", {n: m[2] for n, m in mats.items()})
    stored = read_int4_file(tmp_path / "int4.safetensors", sha, {names[0]: (128, 128), names[1]: (64, 128)})
    w = torch.cat([from_bits(oracle_dequantize((mats[n][0].numpy() + 8).astype(np.uint8), bits(mats[n][1]), None, 64))
                   for n in names])
    packed = pack_stored_group(stored, names, "cpu", w)
    assert packed.out == 192 and packed.columns == 192
    bad = w.clone()
    bad[5, 7] = bad[5, 7] * 2 if float(bad[5, 7]) != 0 else 1.0
    with pytest.raises(Int4Error, match="not bf16"):
        pack_stored_group(stored, names, "cpu", bad)


def test_zero_point_group_128_extension(tmp_path) -> None:
    g = torch.Generator().manual_seed(3)
    codes = torch.randint(0, 16, (64, 256), generator=g, dtype=torch.uint8)
    zeros = torch.randint(0, 16, (64, 2), generator=g, dtype=torch.uint8)
    s = (torch.rand(64, 2, generator=g) * 0.015 + 0.005).to(torch.bfloat16)
    m = stored_from_codes(codes, s, zeros)
    sha = write_int4_file(tmp_path / "int4.safetensors", {"m": m})
    got = read_int4_file(tmp_path / "int4.safetensors", sha, {"m": (64, 256)})["m"]
    assert got.group == 128 and torch.equal(got.zeros, zeros)
    packed = pack_stored_group({"m": got}, ["m"], "cpu", dequantize_stored(got))
    want = pack_kernel_asym(codes, s, zeros, 128)
    assert torch.equal(packed.words, want.words) and torch.equal(packed.zeros, want.zeros)
    c2, s2, z2 = unpack_kernel_asym(packed)
    assert torch.equal(c2.to(torch.uint8), codes) and torch.equal(z2.to(torch.uint8), zeros)
    # the oracle's dequantisation of the same codes
    ref = from_bits(oracle_dequantize(codes.numpy(), bits(s), zeros.numpy(), 128))
    assert torch.equal(dequantize_stored(got), ref)


@pytest.mark.parametrize("fault", ["sha", "missing", "surplus", "dtype", "shape", "scale", "zeros"])
def test_refusals_name_the_problem(tmp_path, fault: str) -> None:
    q, s, m = sym_matrix(32, 128, 4)
    tensors = {"m": m}
    if fault == "dtype":
        tensors = {"m": StoredInt4(m.qweight.to(torch.int16), s)}
    elif fault == "scale":
        bad = s.clone()
        bad[0, 0] = float("nan")
        tensors = {"m": StoredInt4(m.qweight, bad)}
    elif fault == "zeros":
        tensors = {"m": StoredInt4(m.qweight, s, torch.full((32, 2), 16, dtype=torch.uint8))}
    path = tmp_path / "int4.safetensors"
    if fault in ("dtype", "scale", "zeros"):
        with pytest.raises(Int4Error):  # the writer checks too
            write_int4_file(path, tensors)
        from safetensors.torch import save_file
        t = tensors["m"]
        raw = {"m.qweight": t.qweight, "m.scales": t.scales}
        if t.zeros is not None:
            raw["m.zeros"] = t.zeros
        save_file(raw, str(path))
        sha = file_sha256(path)
    else:
        sha = write_int4_file(path, tensors)
    matrices = {"m": (32, 128)}
    if fault == "sha":
        sha = "0" * 64
    elif fault == "missing":
        matrices["n"] = (32, 128)
    elif fault == "surplus":
        from safetensors.torch import save_file
        save_file({"m.qweight": m.qweight, "m.scales": s, "extra": torch.zeros(1)}, str(path))
        sha = file_sha256(path)
    elif fault == "shape":
        matrices = {"m": (32, 256)}
    expect = {"sha": "sha256", "missing": "lacks", "surplus": "not an INT4", "dtype": "uint8", "shape": "shape",
              "scale": "finite", "zeros": "zero point"}[fault]
    with pytest.raises(Int4Error, match=expect):
        read_int4_file(path, sha, matrices)


def test_attach_gives_every_group_its_layout(tmp_path) -> None:
    from jeff_amd.fast_path import Lin
    lin = Lin(["a.q_proj", "a.k_proj"], sizes=[128, 64], k=128, ranks=[16, 16])
    mats = {"a.q_proj": sym_matrix(128, 128, 5)[2], "a.k_proj": sym_matrix(64, 128, 6)[2]}
    sha = write_int4_file(tmp_path / "int4.safetensors", mats)
    attach_int4_file([lin], tmp_path / "int4.safetensors", sha, device="cpu")
    assert lin.int4 is not None and lin.int4.out == 192 and lin.int4.k == 128


def test_pack_group_from_the_folder_tuples_checks_the_bf16_copy(tmp_path) -> None:
    """int4.pack_group, the reference's form (engine/int4.py:265-277; its test tests/test_int4.py:282-307): the stored
    {name: (qweight, scales)} of a fused group stacked along the output, whose integers and scales unpack to the
    originals, after a bit-for-bit check of the group's bfloat16 copy; a copy one step off or in float32 is refused."""
    from jeff_amd.int4 import pack_group
    names = [f"layers.0.linear_attn.{n}" for n in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a")]
    mats = {n: sym_matrix(size, 128, 10 + i) for i, (n, size) in enumerate(zip(names, (192, 64, 16, 16)))}
    sha = write_int4_file(tmp_path / "int4.safetensors", {n: m[2] for n, m in mats.items()})
    stored = read_int4_file(tmp_path / "int4.safetensors", sha, {n: (m[0].shape[0], 128) for n, m in mats.items()})
    folder_tuples = {n: (m.qweight, m.scales) for n, m in stored.items()}
    copy = torch.cat([from_bits(oracle_dequantize((mats[n][0].numpy() + 8).astype(np.uint8), bits(mats[n][1]), None,
                                                  64)) for n in names])
    packed = pack_group(folder_tuples, names, copy)
    assert packed.out == copy.shape[0] == 288 and packed.words.shape[1] % 64 == 0
    q, scales = unpack_kernel(packed)
    assert torch.equal(q, torch.cat([mats[n][0] for n in names]))
    assert torch.equal(scales, torch.cat([mats[n][1] for n in names]))
    changed = copy.clone()
    changed[1, 2] += 1
    with pytest.raises(Int4Error, match=r"The bfloat16 weights of layers.0.linear_attn.in_proj_qkv, "
                                        r".*in_proj_a are not bf16\(q \* s\) of their integers and scales"):
        pack_group(folder_tuples, names, changed)
    with pytest.raises(Int4Error, match=r"are not bf16\(q \* s\)"):
        pack_group(folder_tuples, names, copy.float())


def test_attach_int4_reads_the_folder_the_record_names(tmp_path) -> None:
    """fast_path.attach_int4(lins, quantization) (fast_path.py:352-363): every Lin gets the layout of its matrices
    from the folder's int4.safetensors, checked against the record's sha256 and the Lin's bfloat16 W; the packed
    bytes are returned; a missing matrix or another file is refused."""
    from jeff_amd.fast_path import Lin, attach_int4
    from jeff_amd.int4_file import INT4_FILE, Quantization
    groups = {"qkv": (["l.q_proj", "l.k_proj", "l.v_proj"], [128, 64, 64]), "o": (["l.o_proj"], [128])}
    mats = {}
    for i, (names, sizes) in enumerate(groups.values()):
        for j, (n, size) in enumerate(zip(names, sizes)):
            mats[n] = sym_matrix(size, 128, 20 + 4 * i + j)
    sha = write_int4_file(tmp_path / INT4_FILE, {n: m[2] for n, m in mats.items()})

    def copy_of(names):
        return torch.cat([from_bits(oracle_dequantize((mats[n][0].numpy() + 8).astype(np.uint8), bits(mats[n][1]),
                                                      None, 64)) for n in names])

    lins = [Lin(names, [copy_of([n]) for n in names]) for names, _ in groups.values()]
    record = Quantization("int4-g64", "base@v1+int4-g64-rtn." + sha[:8], "rtn", {}, {"int4_sha256": sha}, tmp_path)
    total = attach_int4(lins, record)
    assert total == sum(lin.int4.nbytes() for lin in lins)
    for lin, (names, _) in zip(lins, groups.values()):
        q, s = unpack_kernel(lin.int4)
        assert torch.equal(q, torch.cat([mats[n][0] for n in names]))
        assert torch.equal(s, torch.cat([mats[n][1] for n in names]))
        assert torch.equal(lin.int4.words, pack_kernel(q, s).words)
    extra = Lin(["l.gate_proj"], [copy_of(["l.o_proj"])])
    with pytest.raises(Int4Error, match="lacks 2 tensors"):
        attach_int4(lins + [extra], record)
    with pytest.raises(Int4Error, match="has sha256"):
        attach_int4(lins, Quantization("int4-g64", "x", "rtn", {}, {"int4_sha256": "0" * 64}, tmp_path))
