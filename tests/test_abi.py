"""The C-ABI library without a GPU: it loads, exports every entry point include/jeff_mlora.h declares (and nothing
else), its constants match the header, and its host-only calls answer (no kernel runs here)."""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

from jeff_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "jeff_mlora.h"


def declared() -> set[str]:
    """The entry points the header declares (its static inline helpers are not exported)."""
    return set(re.findall(r"^(?!static)\w[\w\s\*]*?\b(mlora_\w+)\(", HEADER.read_text(), flags=re.M))


def test_every_declared_entry_point_is_exported() -> None:
    names = declared()
    assert names == set(_lib.EXPORTS)
    h = _lib.lib()
    for name in names:
        assert isinstance(getattr(h, name), ctypes._CFuncPtr)
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIBRARY)], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert {n for n in exported if "mlora" in n} == names  # internal launchers stay hidden


def test_header_constants_match_the_binding() -> None:
    text = HEADER.read_text()

    def const(name: str) -> int:
        return int(re.search(rf"#define {name} (\d+)", text).group(1))

    assert const("MLORA_ABI_VERSION") == _lib.ABI_VERSION == _lib.lib().mlora_abi_version()
    assert const("MLORA_MAX_MATS") == _lib.MAX_MATS
    assert const("MLORA_MAX_REQUESTS") == _lib.MAX_REQUESTS
    assert const("MLORA_MAX_POOL_ROWS") == _lib.MAX_POOL_ROWS
    assert const("MLORA_READOUT_MAX_DIM") == _lib.READOUT_MAX_DIM
    assert const("MLORA_READOUT_MAX_OPTIONS") == _lib.READOUT_MAX_OPTIONS
    assert const("MLORA_EPILOGUE_MAX_N") == _lib.EPILOGUE_MAX_N
    assert re.search(r"#define MLORA_NOALLOC_SCRATCH_BYTES \(64u << 20\)", text)
    assert _lib.NOALLOC_SCRATCH_BYTES == 64 << 20
    assert const("MLORA_ROUTE_BAD_ADAPTER") == _lib.ROUTE_BAD_ADAPTER
    assert const("MLORA_ROUTE_BAD_SEQLENS") == _lib.ROUTE_BAD_SEQLENS
    for name, value in (("MLORA_FORCE_BASE_GEMV", _lib.FORCE_BASE_GEMV), ("MLORA_FORCE_BASE_MFMA", _lib.FORCE_BASE_MFMA),
                        ("MLORA_FORCE_SHRINK_SEGMENT", _lib.FORCE_SHRINK_SEGMENT),
                        ("MLORA_FORCE_SHRINK_MFMA", _lib.FORCE_SHRINK_MFMA),
                        ("MLORA_FORCE_BASE_SPLIT", _lib.FORCE_BASE_SPLIT),
                        ("MLORA_FORCE_BASE_NARROW", _lib.FORCE_BASE_NARROW),
                        ("MLORA_EPILOGUE_SILU_MUL", _lib.EPILOGUE_SILU_MUL),
                        ("MLORA_EPILOGUE_RESIDUAL", _lib.EPILOGUE_RESIDUAL)):
        assert const(name) == value
    assert re.search(r"#define MLORA_FORCE_RANGES\(s\) \(\(s\) << 8\)", text) and _lib.force_ranges(4) == 4 << 8
    assert ctypes.sizeof(_lib.Int4) == 8 * 3 + 4 * 4
    assert ctypes.sizeof(_lib.Lora) == 8 * 4 + 8 * 8 + 4 * 4 + 4 * 16


def test_workspace_bytes_and_refusals_before_any_launch() -> None:
    h = _lib.lib()
    assert h.mlora_workspace_bytes(100, 48) == 9728 and h.mlora_workspace_bytes(0, 16) == 256
    # null descriptors and unsupported shapes are refused on the host: nothing reaches a GPU
    assert h.mlora_dequant(None, None, None) == _lib.EINVAL
    w = _lib.Int4(16, 16, None, 1024, 3072, 3072, 96)
    assert h.mlora_dequant(ctypes.byref(w), 16, None) == _lib.EUNSUPPORTED
    w = _lib.Int4(16, 16, None, 1000, 3072, 3072, 64)
    assert h.mlora_dequant(ctypes.byref(w), 16, None) == _lib.EINVAL
    r = _lib.Route(0, 0, 0, 0, 0, 0, 0, 0, 10, _lib.MAX_REQUESTS + 1, 1)
    assert h.mlora_route(16, None, 1, ctypes.byref(r), 4, None) == _lib.EUNSUPPORTED
    r = _lib.Route(16, 16, 16, 16, 16, 16, 16, 16, 10, 10, 1)
    assert h.mlora_route(16, None, 1, ctypes.byref(r), 4, None) == _lib.EINVAL  # max_segs < min(requests, rows)
    assert h.mlora_route(16, None, 2, ctypes.byref(_lib.Route(16, 16, 16, 16, 16, 16, 16, 16, 10, 10, 4)), 4,
                         None) == _lib.EINVAL  # 10 rows of 2 tokens are not 10 tokens


def test_header_stride_helper_matches_the_package(tmp_path: Path) -> None:
    """mlora_sb_stride (the header's rule for an adapter's sB row stride) gives what Lin.pack uses."""
    from jeff_amd.fast_path import sb_stride

    src = tmp_path / "s.c"
    src.write_text('#include "jeff_mlora.h"\n#include <stdio.h>\nint main(void) {\n'
                   '  for (int c = 0; c <= 128; c += 8)\n    for (int r = 0; r <= c; ++r)\n'
                   '      printf("%d %d %d\\n", r, c, mlora_sb_stride(r, c));\n  return 0;\n}\n')
    exe = tmp_path / "s"
    subprocess.run(["gcc", "-std=c99", "-I", str(HEADER.parent), str(src), "-o", str(exe)], check=True)
    rows = [tuple(map(int, line.split())) for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                                      check=True).stdout.splitlines()]
    assert len(rows) == sum(c + 1 for c in range(0, 129, 8))
    assert all(s == sb_stride(r, c) for r, c, s in rows)


def test_first_factor_extent_past_32_bits_is_refused() -> None:
    """The first factors (tokens x stacked rank, bf16) are addressed with 32-bit buffer offsets: a pass whose first
    factors reach 2^31 bytes is refused with MLORA_EOVERFLOW before any launch, one token fewer is not."""
    h = _lib.lib()
    mats = (_lib.c_i64 * _lib.MAX_MATS)(64 * 64, *([0] * (_lib.MAX_MATS - 1)))
    caps = (_lib.c_i32 * _lib.MAX_MATS)(64, *([0] * (_lib.MAX_MATS - 1)))
    cols = (_lib.c_i32 * _lib.MAX_MATS)(64, *([0] * (_lib.MAX_MATS - 1)))
    lora = _lib.Lora(16, 16, 2 * 64 * 64, 0, mats, 1, 2, 1, 64, caps, cols)
    w = _lib.Int4(16, 16, None, 64, 64, 64, 64)
    for tokens, want in ((1 << 24, _lib.EOVERFLOW), ((1 << 24) - 1, _lib.EINVAL)):
        r = _lib.Route(16, 16, 16, 16, 16, 16, 16, 16, tokens, 1, 1)
        # with y missing, a pass that fits stops at the y check (EINVAL); none of these calls launches anything
        assert h.mlora_int4_linear(ctypes.byref(w), ctypes.byref(lora), ctypes.byref(r), 16, 64, None, 64, None, 16,
                                   1 << 40, None, 0, 0, None) == want
        assert h.mlora_lora_add(ctypes.byref(lora), ctypes.byref(r), 16, 64, 64, None, 64, 64, 16, 1 << 40, 0,
                                None) == want
    r = _lib.Route(16, 16, 16, 16, 16, 16, 16, 16, 1 << 24, 1, 1)
    assert h.mlora_shrink(ctypes.byref(lora), ctypes.byref(r), 16, 64, 64, 16, 0, None) == _lib.EOVERFLOW
    assert h.mlora_int4_base_expand(ctypes.byref(w), ctypes.byref(lora), ctypes.byref(r), 16, 64, 16, 64, None, 16,
                                    None, 0, 0, None) == _lib.EOVERFLOW
