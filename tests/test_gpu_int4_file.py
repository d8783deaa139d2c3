"""INT4 checkpoint ingestion on the GPU: weights read from an int4.safetensors (the reference's format, and the
zero-point / group-128 extension) give the same kernel layout, and so the same product bits, as the weights packed
directly, and the product is within the oracle's bound."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from jeff_amd.fast_path import DT, Workspace
from jeff_amd.int4_file import attach_int4_file, stored_from_codes, write_int4_file
from jeff_amd.int4_kernels import int4_product
from tests.gpu_cases import judge, make_case, token_ids

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("asym,group", [(False, 64), (True, 128)])
def test_products_from_an_int4_file_equal_the_directly_packed_ones(tmp_path, asym: bool, group: int) -> None:
    case = make_case([256, 128], 512, group, asym, {1: [16, 16], 2: [8, 16], 3: [16, 0]}, [16, 16], 11)
    lin = case.lin
    direct = lin.int4
    sizes = np.cumsum([0] + lin.sizes)
    gs = group
    mats = {}
    for j, name in enumerate(lin.names):
        rows = slice(int(sizes[j]), int(sizes[j + 1]))
        zeros = None if case.zeros is None else case.zeros[rows]
        mats[name] = stored_from_codes(case.codes[rows], case.scales[rows], zeros)
    sha = write_int4_file(tmp_path / "int4.safetensors", mats)
    lin.W = case.w.cuda()  # the standard path's bf16 copy: the reader checks it bit for bit
    attach_int4_file([lin], tmp_path / "int4.safetensors", sha, device="cuda")
    assert lin.int4.group == gs and torch.equal(lin.int4.words, direct.words)
    assert torch.equal(lin.int4.scales, direct.scales)
    assert (lin.int4.zeros is None) == (direct.zeros is None)
    adp = torch.tensor([1, 2, 0, 3, 2, 1, 3, 0], dtype=torch.int32, device="cuda")
    x = torch.randn(8 * 16, lin.k, device="cuda").to(DT)
    ws = Workspace(8 * 16, 16, max_rank=lin.rank)
    got = int4_product(lin, x, ws, adp)
    lin_direct = lin.int4
    lin.int4 = direct
    again = int4_product(lin, x, ws, adp)
    lin.int4 = lin_direct
    assert torch.equal(got, again)
    r = judge(lin, case.w, x, token_ids(adp, lin.pool.shape[0], row_len=16), got)
    assert r["finite"] and r["beyond_bound"] == 0 and r["outside_tolerance"] == 0, r
