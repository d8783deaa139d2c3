"""Build recipe of the HIP library: every csrc/*.hip compiled for gfx950 with hipcc and linked into
jeff_amd/libjeff_mlora.so (in-tree, so it travels with the repository to the GPU machine).

Run as `python -m jeff_amd.build`; `__graft_entry__.build()` calls `build()`."""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
INCLUDE = ROOT / "include"
OBJ_DIR = PACKAGE / "_build"
LIBRARY = PACKAGE / "libjeff_mlora.so"
SOURCES = ("route.hip", "shrink.hip", "base.hip", "gemm256.hip", "decode.hip", "finish.hip", "readout.hip",
           "epilogue.hip", "api.hip")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Packed float32 instructions are disabled in device code (-packed-fp32-ops); hipcc's host pass warns that it does not
# know the feature, which is harmless.
FLAGS = ["-std=c++17", "-O3", "-fPIC", f"--offload-arch={ARCH}", f"-I{INCLUDE}", f"-I{CSRC}",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wall", "-Wno-unused-function", "-fvisibility=hidden"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build(jobs: int = 4) -> Path:
    """Compile every source and link the shared library; returns its path. Always rebuilds."""
    OBJ_DIR.mkdir(exist_ok=True)
    objects = [OBJ_DIR / (name.rsplit(".", 1)[0] + ".o") for name in SOURCES]
    cmds = [[HIPCC, *FLAGS, "-c", str(CSRC / name), "-o", str(obj)] for name, obj in zip(SOURCES, objects)]
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        list(pool.map(_run, cmds))
    tmp = LIBRARY.with_suffix(".so.tmp")
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objects), "-o", str(tmp)])
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build())
