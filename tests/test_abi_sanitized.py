"""The C ABI's host-side argument checks under AddressSanitizer and UndefinedBehaviorSanitizer, on a machine without a
GPU: api.hip (every check and the kernel choice) is compiled with the sanitizers on its host code only, linked with the
library's other objects into tests/abi_sanitize.cpp's driver, and the driver's calls (null, misaligned, inconsistent
and extreme arguments, none of which may launch anything) must return the expected statuses with no sanitizer report.
"""

from __future__ import annotations

import os
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
ROCM = Path("/opt/rocm")
HIPCC = ROCM / "bin" / "hipcc"
CLANG = ROCM / "llvm" / "bin" / "clang++"


@pytest.mark.skipif(not HIPCC.exists() or not CLANG.exists(), reason="needs the ROCm compilers")
def test_argument_checks_are_clean_under_asan_and_ubsan(tmp_path: Path) -> None:
    from jeff_amd import build

    others = [build.OBJ_DIR / (n.rsplit(".", 1)[0] + ".o") for n in build.SOURCES if n != "api.hip"]
    if not all(o.exists() for o in others):
        build.build()
    inc = [f"-I{ROOT / 'include'}", f"-I{ROOT / 'jeff_amd' / 'csrc'}"]
    api = tmp_path / "api_sanitized.o"
    # the sanitizers on the host code only: each -fsanitize= behind -Xarch_host
    subprocess.run([str(HIPCC), "-std=c++17", "-O1", "-g", "-fPIC", f"--offload-arch={build.ARCH}", *inc,
                    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                    "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                    "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer",
                    "-c", str(ROOT / "jeff_amd" / "csrc" / "api.hip"), "-o", str(api)],
                   check=True, capture_output=True, text=True)
    driver = tmp_path / "abi_sanitize"
    host_flags = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-g"]
    subprocess.run([str(CLANG), "-std=c++17", *host_flags, *inc, str(ROOT / "tests" / "abi_sanitize.cpp"),
                    str(api), *map(str, others), f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}",
                    "-o", str(driver)], check=True, capture_output=True, text=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", HIP_VISIBLE_DEVICES="")
    run = subprocess.run([str(driver)], capture_output=True, text=True, env=env, timeout=120)
    report = run.stdout + run.stderr
    assert run.returncode == 0, report
    assert "runtime error" not in report and "AddressSanitizer" not in report, report
    assert "ok: 0 mismatches" in run.stdout, report
