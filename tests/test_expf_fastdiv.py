"""Host-side checks of two pieces of the device header (dkz_device.hpp),
compiled for the host from the same source (tests/native/dkz_checks.hip):

* expf_libm, the exp behind every exp-based activation and softmax, against
  the host C library's expf over all 2^32 float inputs (the GPU-side twin of
  this check is tests/test_gpu_expf.py);
* its 2^(i/32) table, against 2^(i/32) computed to 60 digits and rounded to
  double;
* expf_cw, softmax's exp, against exp in double over all 2^32 float inputs:
  within one ulp everywhere (its device build is checked bit for bit against
  this host build in tests/test_gpu_expf.py);
* the launch-constant division against Python's integer division;
* the workgroup renumbering that keeps runs of logical blocks on one XCD: a
  bijection, with every run on one XCD under round-robin dispatch.
"""

from __future__ import annotations

import ctypes as C
import os
import struct
from decimal import Decimal, getcontext

import numpy as np
import pytest

from tests.native import build as native_build


def lib():
    L = C.CDLL(str(native_build.LIB))
    L.chk_fastdiv.restype = C.c_uint32
    L.chk_fastdiv.argtypes = [C.c_uint32, C.c_uint32]
    L.chk_xcd_run_block.restype = C.c_uint32
    L.chk_xcd_run_block.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32]
    L.chk_exp2f_tab.restype = C.c_uint64
    L.chk_exp2f_tab.argtypes = [C.c_uint32]
    L.chk_expf_restated.restype = C.c_float
    L.chk_expf_restated.argtypes = [C.c_float]
    L.chk_expf_host_mismatches.restype = C.c_uint64
    L.chk_expf_host_mismatches.argtypes = [C.c_uint64, C.c_uint64, C.c_int]
    L.chk_expf_cw.restype = C.c_float
    L.chk_expf_cw.argtypes = [C.c_float]
    L.chk_expf_cw_max_err.restype = C.c_uint64
    L.chk_expf_cw_max_err.argtypes = [C.c_uint64, C.c_uint64, C.c_int]
    return L


def double_bits(x: float) -> int:
    return struct.unpack("<Q", struct.pack("<d", x))[0]


def test_exp2_table_is_2_pow_i_over_32():
    getcontext().prec = 60
    L = lib()
    for i in range(32):
        exact = Decimal(2) ** (Decimal(i) / Decimal(32))
        nearest = float(exact)  # Decimal -> float rounds correctly to nearest
        assert L.chk_exp2f_tab(i) == double_bits(nearest) - (i << 47), i


def test_expf_special_values():
    L = lib()
    assert L.chk_expf_restated(0.0) == 1.0
    assert L.chk_expf_restated(float("-inf")) == 0.0
    assert L.chk_expf_restated(float("inf")) == float("inf")
    assert np.isnan(L.chk_expf_restated(float("nan")))
    assert L.chk_expf_restated(89.0) == float("inf")
    assert L.chk_expf_restated(-104.0) == 0.0
    assert L.chk_expf_restated(1.0) == np.float32(np.e)


def test_expf_matches_libm_on_every_float():
    threads = min(os.cpu_count() or 4, 16)
    assert lib().chk_expf_host_mismatches(0, 1 << 32, threads) == 0


def test_expf_cw_special_values():
    L = lib()
    assert L.chk_expf_cw(0.0) == 1.0
    assert L.chk_expf_cw(-0.0) == 1.0
    assert L.chk_expf_cw(float("-inf")) == 0.0
    assert L.chk_expf_cw(float("inf")) == float("inf")
    assert np.isnan(L.chk_expf_cw(float("nan")))
    assert L.chk_expf_cw(89.0) == float("inf")
    assert L.chk_expf_cw(88.72) < float("inf")  # just below FLT_MAX's log
    assert L.chk_expf_cw(-104.0) == 0.0
    assert L.chk_expf_cw(-103.9) == np.float32(2.0 ** -149)  # the smallest subnormal
    assert L.chk_expf_cw(1.0) == np.float32(np.e)
    for k in range(-149, 128):  # near 2^k: every binade, subnormals included
        x = float(np.float32(k * np.log(2.0)))
        want = np.exp(x)
        ulp = 2.0 ** max(np.frexp(want)[1] - 24, -149)
        assert abs(L.chk_expf_cw(x) - want) < ulp, k


@pytest.mark.parametrize("part", range(4))
def test_expf_cw_within_one_ulp_everywhere(part):
    """max |expf_cw(x) - exp(x)| over a quarter of the float bit patterns, in
    ulps of the result (2^-149 for subnormals): measured 0.94 ulp."""
    threads = min(os.cpu_count() or 4, 16)
    lo, hi = part << 30, (part + 1) << 30
    assert lib().chk_expf_cw_max_err(lo, hi, threads) / 1024.0 < 1.0


DIVISORS = sorted({1, 2, 3, 5, 7, 13, 14, 28, 49, 53, 196, 784, 1024, 3136, 4096, 12544, 65535, 65536, 65537,
                   1000003, (1 << 20) - 1, (1 << 30) + 1, (1 << 31) - 1} | {(1 << k) + d for k in range(1, 31)
                                                                           for d in (-1, 0, 1)})


@pytest.mark.parametrize("d", DIVISORS)
def test_fastdiv(d):
    L = lib()
    g = np.random.default_rng(d)
    ns = {0, 1, d - 1, d, d + 1, 2 * d - 1, 2 * d, (1 << 31) - 1, (1 << 31) - 2, ((1 << 31) - 1) // d * d,
          ((1 << 31) - 1) // d * d - 1}
    ns |= set(int(v) for v in g.integers(0, 1 << 31, 2000))
    for n in ns:
        if 0 <= n < (1 << 31):
            assert L.chk_fastdiv(n, d) == n // d, (n, d)


@pytest.mark.parametrize("r", [1, 2, 4, 8, 16])
def test_xcd_run_block(r):
    """Logical blocks r*i .. r*i + r - 1 land on physical blocks b, b + 8, ...
    (one XCD when block b goes to XCD b % 8), and the renumbering is a
    permutation of [0, grid) for grids that are and are not multiples of 8r."""
    L = lib()
    for grid in list(range(1, 300)) + [676, 1352, 4096, 4099]:
        phys = {}
        for b in range(grid):
            t = L.chk_xcd_run_block(b, grid, r)
            assert 0 <= t < grid and t not in phys, (grid, r, b, t)
            phys[t] = b
        full = grid // (8 * r) * (8 * r)
        for t0 in range(0, full, r):
            assert len({phys[t0 + k] % 8 for k in range(r)}) == 1, (grid, r, t0)
