"""Every HIP kernel of the library keeps its state in registers and LDS: compiled for gfx950 with the compiler's
resource remarks, no kernel may use scratch (per-lane private) memory. Scratch comes from register spills and from
small arrays indexed at run time; either one turns into memory traffic that every thread of every workgroup writes
and reads back (a 20-byte array in the 256 x 256 prefill kernel wrote 245 MB per gate_up launch at 159,488 tokens).
Runs on the CPU: hipcc cross-compiles the device code."""

from __future__ import annotations

import re
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

from jeff_amd import build

REMARK = re.compile(r"(Function Name|ScratchSize \[bytes/lane\]|VGPRs Spill|SGPRs Spill): (\S+)")


def resources(source: str, out: Path) -> list[dict[str, str]]:
    """The compiler's resource remarks for each kernel of one source file."""
    cmd = [build.HIPCC, *build.FLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", str(build.CSRC / source), "-o",
           str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr
    kernels: list[dict[str, str]] = []
    for key, value in REMARK.findall(proc.stderr):
        if key == "Function Name":
            kernels.append({"name": value})
        elif kernels:
            kernels[-1][key] = value
    return kernels


@pytest.mark.skipif(not Path(build.HIPCC).exists(), reason="needs hipcc")
def test_no_kernel_uses_scratch_memory(tmp_path: Path) -> None:
    with ThreadPoolExecutor(max_workers=4) as pool:
        found = dict(zip(build.SOURCES, pool.map(lambda s: resources(s, tmp_path / (s + ".o")), build.SOURCES)))
    kernels = [(src, k) for src, ks in found.items() for k in ks]
    assert len(kernels) >= 20, found  # every source's kernels were reported
    bad = [(src, k) for src, k in kernels
           if k.get("ScratchSize [bytes/lane]") != "0" or k.get("VGPRs Spill", "0") != "0"]
    assert not bad, bad
