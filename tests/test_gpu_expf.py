"""The device expf against the host C library over every float32 input, and
softmax's expf_cw against its own host build.

expf_libm (darknet_zig_amd/csrc/dkz_device.hpp) is what makes the exp-based
activations and softmax bit-exact. Here it runs on the GPU over all 2^32 bit
patterns; an order-independent hash of its results is compared with the hash
of the host libm's results over the same inputs (NaNs canonicalised).
"""

from __future__ import annotations

import ctypes as C

import pytest

from tests.native import build as native_build

pytestmark = pytest.mark.gpu


def _lib():
    lib = C.CDLL(str(native_build.LIB))
    lib.chk_expf_hash_host.restype = C.c_uint64
    lib.chk_expf_hash_host.argtypes = [C.c_uint64, C.c_uint64, C.c_int]
    lib.chk_expf_hash_device.restype = C.c_int
    lib.chk_expf_hash_device.argtypes = [C.c_uint64, C.c_uint64, C.POINTER(C.c_uint64)]
    lib.chk_expf_cw_hash_host.restype = C.c_uint64
    lib.chk_expf_cw_hash_host.argtypes = [C.c_uint64, C.c_uint64, C.c_int]
    lib.chk_expf_cw_hash_device.restype = C.c_int
    lib.chk_expf_cw_hash_device.argtypes = [C.c_uint64, C.c_uint64, C.POINTER(C.c_uint64)]
    return lib


@pytest.mark.parametrize("part", range(4))
def test_device_expf_matches_libm_everywhere(dev, part):
    lib = _lib()
    lo, hi = part << 30, (part + 1) << 30
    h = C.c_uint64(0)
    rc = lib.chk_expf_hash_device(lo, hi, C.byref(h))
    assert rc == 0, rc
    assert h.value == lib.chk_expf_hash_host(lo, hi, 16)


@pytest.mark.parametrize("part", range(4))
def test_device_expf_cw_matches_its_host_build(dev, part):
    """expf_cw uses only IEEE-exact operations (multiply, fma, rint, ldexp),
    so the GPU must give the host build's bits on every input; the host build
    is the one checked against exp in double (tests/test_expf_fastdiv.py)."""
    lib = _lib()
    lo, hi = part << 30, (part + 1) << 30
    h = C.c_uint64(0)
    rc = lib.chk_expf_cw_hash_device(lo, hi, C.byref(h))
    assert rc == 0, rc
    assert h.value == lib.chk_expf_cw_hash_host(lo, hi, 16)
