"""Both host-side mirrors of gpu.zig against the reference's own interface
(tests/golden/gpu_zig_api.json, transcribed from src/gpu.zig:483-830): every
public op exists under its gpu.zig name with the same number of parameters, in
the Python mirror (darknet_zig_amd/gpu.py) and in the C++ one
(darknet_zig_amd/host/dkz_gpu.hpp, checked by compiling static_asserts).
No GPU needed."""

from __future__ import annotations

import inspect
import json
import shutil
import subprocess
from pathlib import Path

import pytest

from darknet_zig_amd import gpu

ROOT = Path(__file__).resolve().parents[1]
API = json.loads((ROOT / "tests" / "golden" / "gpu_zig_api.json").read_text())["ops"]


def test_fixture_covers_the_op_surface():
    assert len(API) == 35
    assert {"axpy", "gemm", "im2col", "adamUpdate", "forwardMaxpool", "shortcut"} <= set(API)


@pytest.mark.parametrize("name", sorted(API))
def test_python_mirror_matches_gpu_zig(name):
    fn = getattr(gpu, name)
    params = list(inspect.signature(fn).parameters)
    assert len(params) == len(API[name]["params"]), (name, params, API[name]["params"])


def test_cpp_mirror_matches_gpu_zig(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("no g++")
    lines = ['#include "dkz_gpu.hpp"',
             "template <class R, class... A> constexpr int arity(R (*)(A...)) { return sizeof...(A); }"]
    for name, spec in sorted(API.items()):
        lines.append(f'static_assert(arity(&dkz::gpu::{name}) == {len(spec["params"])}, '
                     f'"{name}: gpu.zig:{spec["line"]} takes {len(spec["params"])}");')
    lines.append("int main() { return 0; }")
    src = tmp_path / "arity.cpp"
    src.write_text("\n".join(lines) + "\n")
    proc = subprocess.run([gxx, "-std=c++17", "-fsyntax-only", "-Wall", "-Wextra", f"-I{ROOT / 'include'}",
                           f"-I{ROOT / 'darknet_zig_amd' / 'host'}", str(src)], capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr


CALLERS = json.loads((Path(__file__).resolve().parent / "golden" / "gpu_zig_callers.json").read_text())["identifiers"]


@pytest.mark.parametrize("name", sorted(CALLERS))
def test_python_mirror_has_every_caller_identifier(name):
    """Every gpu.<name> the reference's callers use (gpu_zig_callers.json)
    exists in the Python mirror too, as a function where gpu.zig has one."""
    assert hasattr(gpu, name), name
    if CALLERS[name]["kind"] == "fn":
        assert callable(getattr(gpu, name)), name


def test_python_mirror_state_before_init():
    """gpu.zig:104-160: with no device selected the state reads "CPU"."""
    saved = gpu.device_index
    try:
        gpu.deinit()
        assert gpu.enabled is True and gpu.backend_label == "HIP"
        assert gpu.device_index == -1 and not gpu.active()
        assert gpu.deviceName() == "CPU" and gpu.deviceMemoryMib() == 0
        assert gpu.gemmPolicy() == "cpu" and gpu.gemmBlockMinTiles() == 0
    finally:
        gpu.device_index = saved
