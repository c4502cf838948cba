"""Builds the native test programs:

* tests/native/libdkz_checks.so (test-only helpers, see dkz_checks.hip), with
  the product's hipcc flags so the device header compiles exactly as it does
  inside libdkz.so; the host half is built for x86-64-v3 (AVX2 + FMA);
* tests/native/gputest, gputest.zig's CPU-vs-GPU check written against the
  C++ host mirror (darknet_zig_amd/host/dkz_gpu.hpp), linked with libdkz.so
  and the CPU oracle. It needs both built first.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[2]))
from darknet_zig_amd import build as pkg_build  # noqa: E402

HERE = Path(__file__).resolve().parent
SRC = HERE / "dkz_checks.hip"
LIB = HERE / "libdkz_checks.so"
GPUTEST_SRC = HERE / "gputest.cpp"
GPUTEST = HERE / "gputest"
ROOT = HERE.parents[1]


def build() -> Path:
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [pkg_build.hipcc(), *pkg_build.HIPCC_FLAGS, "-Xarch_host", "-march=x86-64-v3", "-shared",
           str(SRC), "-o", str(tmp), "-lpthread"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"building {LIB.name} failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB)
    build_gputest()
    return LIB


def build_gputest() -> Path:
    tmp = GPUTEST.with_suffix(".tmp")
    pkg, ora = ROOT / "darknet_zig_amd", ROOT / "oracle"
    cmd = ["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", f"-I{ROOT / 'include'}", f"-I{pkg / 'host'}", f"-I{ora}",
           str(GPUTEST_SRC), "-o", str(tmp), f"-L{pkg}", "-ldkz", f"-L{ora}", "-ldkz_oracle",
           "-Wl,-rpath,$ORIGIN/../../darknet_zig_amd", "-Wl,-rpath,$ORIGIN/../../oracle",
           "-Wl,-rpath-link,/opt/rocm/lib"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"building {GPUTEST.name} failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, GPUTEST)
    return GPUTEST


if __name__ == "__main__":
    print(build())
