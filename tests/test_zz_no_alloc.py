"""dkz_batchnorm_backward_noalloc, the batch-norm backward step whose
scratch is a static device array (no allocation), against
dkz_batchnorm_backward through the C ABI: the same kernels and launch
geometry, so every output is bit-identical. Two calls in a row, the second
on a smaller tensor, then the first shape again (the static array keeps the
previous call's contents: partial sums are rewritten, counter slots cleared
by each call).

  * [8,128,4099]: spatial not a multiple of 4, so the per-op sequence runs;
    its 128 channels of 32792 elements take the two-workgroup pair
    reduction, whose halves meet in the slots by an atomic exchange;
  * [4,64,4099]: the per-op sequence again, but 64 channels of 16396
    elements split 8 ways: each channel's workgroups post f64 partials in
    the array and count themselves in its slots (the last one finalises);
  * [32,64,28,28]: the fused passes with each channel split over several
    workgroups, whose f64 partials go through the array.

A second test runs config 2's shape, whose one-launch pass holds part of
each chunk in registers and LDS and meets at per-channel barriers in the
array's slots, then the smaller shape again. A third captures the call in a
HIP graph (after dkz_init, which makes every first-use HIP query), replays
it three times with eager work in between, and checks each replay bit for
bit against the regular entry point and that neither the call nor a replay
changes the device's free memory.
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
    _check((8, 128, 4099), 1)  # per-op sequence, pair reductions meeting in the slots
    _check((4, 64, 4099), 6)  # smaller: per-op sequence, 8-way split reductions counting in the slots
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


class _Hip:
    def __init__(self):
        L = C.CDLL("libamdhip64.so")
        for name, args in {
            "hipStreamCreate": [C.POINTER(C.c_void_p)],
            "hipStreamDestroy": [C.c_void_p],
            "hipStreamSynchronize": [C.c_void_p],
            "hipStreamBeginCapture": [C.c_void_p, C.c_int],
            "hipStreamEndCapture": [C.c_void_p, C.POINTER(C.c_void_p)],
            "hipGraphInstantiate": [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t],
            "hipGraphLaunch": [C.c_void_p, C.c_void_p],
            "hipGraphExecDestroy": [C.c_void_p],
            "hipGraphDestroy": [C.c_void_p],
        }.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = C.c_int
        self.L = L

    def __getattr__(self, name):
        return getattr(self.L, name)


def _free_bytes() -> int:
    return gpu.mem_info()[0]


def test_captured_in_a_graph(dev):
    """The entry point for callers that cannot allocate, inside a HIP graph."""
    shape = (32, 64, 28 * 28)
    B, F, S = shape
    h = _inputs(shape, 7)
    want = _run("dkz_batchnorm_backward", shape, h)
    lib = _lib.load()
    sync_before = lib.dkz_get_sync_after_launch()
    lib.dkz_set_sync_after_launch(0)  # no synchronise inside a capture
    d = {k: up(v) for k, v in h.items()}
    md, vd = gpu.alloc(F), gpu.alloc(F)
    args = (B, F, S, int(Activation.leaky), d["y"].ptr, d["delta"].ptr, d["x"].ptr, d["x_norm"].ptr, d["mean"].ptr,
            d["var"].ptr, d["scales"].ptr, d["bu"].ptr, d["su"].ptr, md.ptr, vd.ptr)

    def restore():  # the call overwrites delta and accumulates into the updates
        gpu.push(d["delta"], h["delta"])
        gpu.push(d["bu"], h["bu"])
        gpu.push(d["su"], h["su"])

    def results():
        return {"delta": down(d["delta"], h["delta"]), "bias_updates": down(d["bu"], h["bu"]),
                "scale_updates": down(d["su"], h["su"]), "mean_delta": down(md, h["bu"]),
                "variance_delta": down(vd, h["bu"])}

    gpu.sync()
    free0 = _free_bytes()
    assert lib.dkz_batchnorm_backward_noalloc(*args) == 0, lib.dkz_last_error_context()
    gpu.sync()
    assert _free_bytes() == free0, "the eager call changed the device's free memory"
    for k, v in results().items():
        assert_bitexact(v, want[k], f"eager {k}")

    hip = _Hip()
    s, graph, exe = C.c_void_p(), C.c_void_p(), C.c_void_p()
    assert hip.hipStreamCreate(C.byref(s)) == 0
    try:
        lib.dkz_set_stream(s)
        assert hip.hipStreamBeginCapture(s, 0) == 0  # hipStreamCaptureModeGlobal
        rc = lib.dkz_batchnorm_backward_noalloc(*args)
        assert hip.hipStreamEndCapture(s, C.byref(graph)) == 0
        lib.dkz_set_stream(None)
        assert rc == 0, lib.dkz_last_error_context()
        assert hip.hipGraphInstantiate(C.byref(exe), graph, None, None, 0) == 0
        for replay in range(3):
            restore()  # eager work between the replays
            gpu.scal(4, 1.0, d["scales"])
            gpu.sync()
            free1 = _free_bytes()
            assert hip.hipGraphLaunch(exe, s) == 0
            assert hip.hipStreamSynchronize(s) == 0
            assert _free_bytes() == free1, f"replay {replay} changed the device's free memory"
            for k, v in results().items():
                assert_bitexact(v, want[k], f"replay {replay} {k}")
                assert np.all(np.isfinite(v)), k
    finally:
        lib.dkz_set_stream(None)
        lib.dkz_set_sync_after_launch(sync_before)
        gpu.sync()
        if exe.value:
            hip.hipGraphExecDestroy(exe)
        if graph.value:
            hip.hipGraphDestroy(graph)
        hip.hipStreamDestroy(s)
        for b in list(d.values()) + [md, vd]:
            gpu.free(b)
