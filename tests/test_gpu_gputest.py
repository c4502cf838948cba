"""gputest.zig's CPU-vs-GPU check, run as the reference runs it: one native
program (tests/native/gputest, built from gputest.cpp against the C++ host
mirror of gpu.zig) that calls every op through the C ABI and compares it with
the CPU twins, each check at gputest's 1e-3 and at this library's own bar."""

from __future__ import annotations

import json
import subprocess

import pytest

from tests.native import build as native_build

pytestmark = pytest.mark.gpu


def test_gputest_program_passes():
    proc = subprocess.run([str(native_build.GPUTEST), "0"], capture_output=True, text=True, timeout=120)
    print(proc.stdout)
    summary = json.loads(proc.stdout.strip().splitlines()[-1])
    assert proc.returncode == 0, (summary, proc.stdout[-3000:], proc.stderr[-2000:])
    assert summary["checks"] >= 39 and summary["passed"] == summary["checks"], summary
