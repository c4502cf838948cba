"""Builds libdkz.so, the gfx950 tensor-op library, in-tree with hipcc.

Each .hip source under csrc/ is compiled to an object for gfx950 and the
objects are linked into darknet_zig_amd/libdkz.so. The flags are part of the
numerics: -ffp-contract=off and the correctly rounded fp32 divide/sqrt keep
every elementwise op bit-exact against the CPU twins, fp32 denormals stay
enabled as on the host, and packed-fp32 instructions are switched off.

Usage: python -m darknet_zig_amd.build [--jobs N]
"""

from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
OBJ_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libdkz.so"
VERSION_SCRIPT = PKG_DIR / "libdkz.map"  # exports dkz_* only

ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]

# libdkz.so's host code: only what include/dkz_ops.h declares (visibility
# pushed to default there) is exported; the device code objects keep their
# kernels' own (protected) visibility.
VISIBILITY_FLAGS = ["-Xarch_host", "-fvisibility=hidden", "-Xarch_host", "-fvisibility-inlines-hidden"]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: the HIP toolchain is required to build libdkz.so")
    return exe


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *VISIBILITY_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compiles every csrc/*.hip for gfx950 and links libdkz.so. Always rebuilds."""
    OBJ_DIR.mkdir(exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", f"-Wl,--version-script={VERSION_SCRIPT}",
           *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"linking libdkz.so failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources", file=sys.stderr)
    return LIB_PATH


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args()
    build(args.jobs, verbose=True)


if __name__ == "__main__":
    main()
