"""dkz_batchnorm_backward_noalloc, the batch-norm backward step whose
scratch is a static device array (no allocation), against
dkz_batchnorm_backward through the C ABI: the same kernels and launch
geometry, so every output is bit-identical. Two calls in a row, the second
on a smaller tensor, then the first shape again (the static array keeps the
previous call's contents: partial sums are rewritten, counter slots cleared
by each call).

  * [8,128,4099]: spatial not a multiple of 4, so the per-op sequence runs,
    and its channel reductions (128 channels of 32792 elements, each split
    16 ways) count themselves in the slots;
  * [32,64,28,28]: the fused passes with each channel split over several
    workgroups, whose f64 partials go through the array.

A second test runs config 2's shape, whose one-launch pass holds part of
each chunk in registers and LDS and meets at per-channel barriers in the
array's slots, then the smaller shape again.
"""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from darknet_zig_amd import _lib, gpu
from darknet_zig_amd.activations import Activation
from tests.helpers import assert_bitexact, down, normal, rng, uniform, up

pytestmark = pytest.mark.gpu


def _inputs(shape, seed):
    B, F, S = shape
    n = B * F * S
    r = rng(seed)
    y = normal(r, n)
    y = np.where(y > 0, y, np.float32(0.1) * y).astype(np.float32)
    x = normal(r, n)
    xm = x.reshape(B, F, S).astype(np.float64)
    return dict(y=y, delta=normal(r, n), x=x, x_norm=normal(r, n),
                mean=xm.mean(axis=(0, 2)).astype(np.float32), var=xm.var(axis=(0, 2), ddof=1).astype(np.float32),
                scales=uniform(r, F, 0.5, 1.5), bu=normal(r, F), su=normal(r, F))


def _run(entry, shape, h):
    B, F, S = shape
    d = {k: up(v) for k, v in h.items()}
    md, vd = gpu.alloc(F), gpu.alloc(F)
    lib = _lib.load()
    rc = getattr(lib, entry)(B, F, S, int(Activation.leaky), d["y"].ptr, d["delta"].ptr, d["x"].ptr,
                             d["x_norm"].ptr, d["mean"].ptr, d["var"].ptr, d["scales"].ptr, d["bu"].ptr,
                             d["su"].ptr, md.ptr, vd.ptr)
    assert rc == 0, (entry, rc, lib.dkz_last_error_context())
    gpu.sync()
    out = {"delta": down(d["delta"], h["delta"]), "bias_updates": down(d["bu"], h["bu"]),
           "scale_updates": down(d["su"], h["su"]), "mean_delta": down(md, h["bu"]),
           "variance_delta": down(vd, h["bu"])}
    for b in list(d.values()) + [md, vd]:
        gpu.free(b)
    return out


def _check(shape, seed):
    h = _inputs(shape, seed)
    want = _run("dkz_batchnorm_backward", shape, h)
    got = _run("dkz_batchnorm_backward_noalloc", shape, h)
    for k in want:
        assert_bitexact(got[k], want[k], f"{shape} {k}")
        assert np.all(np.isfinite(got[k])), k


def test_two_calls_second_smaller(dev):
    _check((8, 128, 4099), 1)  # per-op sequence, split channel reductions counting in the slots
    _check((32, 64, 28 * 28), 2)  # smaller: fused passes, split partials
    _check((8, 128, 4099), 3)  # the first shape again, after the array was reused


def test_config2_register_holding_pass(dev):
    _check((64, 128, 3136), 4)  # one launch: partials and barrier words in the array
    _check((32, 64, 28 * 28), 5)  # smaller, after it


def test_zero_filters_is_a_no_op(dev):
    assert _lib.load().dkz_batchnorm_backward_noalloc(4, 0, 16, int(Activation.leaky), *([None] * 11)) == 0


def test_bad_sizes_are_rejected(dev):
    lib = _lib.load()
    assert lib.dkz_batchnorm_backward_noalloc(-1, 4, 16, int(Activation.leaky), *([None] * 11)) == 1
    big = lib.dkz_batchnorm_backward_noalloc(1 << 16, 1 << 10, 1 << 6, int(Activation.leaky), *([None] * 11))
    assert big == 1  # 2^32 elements: hipErrorInvalidValue, before any launch
    assert b"2^31-1" in lib.dkz_last_error_context()
