"""Builds tests/native/libdkz_checks.so (test-only helpers, see dkz_checks.hip).

Uses the product's hipcc flags so the device header compiles exactly as it
does inside libdkz.so; the host half is built for x86-64-v3 (AVX2 + FMA).
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


def build() -> Path:
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [pkg_build.hipcc(), *pkg_build.HIPCC_FLAGS, "-Xarch_host", "-march=x86-64-v3", "-shared",
           str(SRC), "-o", str(tmp), "-lpthread"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"building {LIB.name} failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
