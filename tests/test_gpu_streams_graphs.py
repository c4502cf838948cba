"""The library on a stream of the caller's choosing (dkz_set_stream) and
inside a captured HIP graph.

gpu.zig issues everything on the null stream (hip.zig:134); the C ABI lets a
caller pick another, and because no op allocates, copies or clears memory
(the reductions' scratch is allocated once, by dkz_init), a sequence of ops
can be captured into a HIP graph and replayed. Both are checked bit for bit
against the same ops issued eagerly on the null stream: the config-2 batch
norm backward chain (split and one-launch reductions, broadcasts) and the
fused backward pass, replayed several times with eager work in between.
"""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from darknet_zig_amd import _lib, gpu
from darknet_zig_amd.activations import Activation
from tests.helpers import assert_bitexact, down, normal, rng, uniform, up

pytestmark = pytest.mark.gpu

SHAPE = (16, 128, 784)  # splits channels for the two-stream reductions


class Hip:
    def __init__(self):
        L = C.CDLL("libamdhip64.so")
        sigs = {
            "hipStreamCreate": [C.POINTER(C.c_void_p)],
            "hipStreamDestroy": [C.c_void_p],
            "hipStreamSynchronize": [C.c_void_p],
            "hipStreamBeginCapture": [C.c_void_p, C.c_int],
            "hipStreamEndCapture": [C.c_void_p, C.POINTER(C.c_void_p)],
            "hipGraphInstantiate": [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t],
            "hipGraphLaunch": [C.c_void_p, C.c_void_p],
            "hipGraphExecDestroy": [C.c_void_p],
            "hipGraphDestroy": [C.c_void_p],
        }
        for name, args in sigs.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = C.c_int
        self.L = L

    def __getattr__(self, name):
        return getattr(self.L, name)


def _inputs(seed):
    B, F, S = SHAPE
    n = B * F * S
    r = rng(seed)
    y, delta, x, xn = normal(r, n), normal(r, n), normal(r, n), normal(r, n)
    y = np.where(y > 0, y, np.float32(0.1) * y).astype(np.float32)
    return dict(y=y, delta=delta, x=x, xn=xn, scales=uniform(r, F, 0.5, 1.5), mean=normal(r, F, 0, 0.1),
                var=uniform(r, F, 0.5, 1.5))


def _upload(h):
    F = SHAPE[1]
    d = {k: up(v) for k, v in h.items()}
    for k in ("bu", "su", "md", "vd"):
        d[k] = gpu.alloc(F)
    return d


def _chain(d):
    """convolutional.zig:280 + batchnorm.zig:155-174, per op."""
    B, F, S = SHAPE
    n = B * F * S
    gpu.gradientArray(d["y"], n, Activation.leaky, d["delta"])
    gpu.backwardBias(d["bu"], d["delta"], B, F, S)
    gpu.backwardScale(d["xn"], d["delta"], B, F, S, d["su"])
    gpu.scaleBias(d["delta"], d["scales"], B, F, S)
    gpu.meanDelta(d["delta"], d["var"], B, F, S, d["md"])
    gpu.varianceDelta(d["x"], d["delta"], d["mean"], d["var"], B, F, S, d["vd"])
    gpu.normalizeDelta(d["x"], d["mean"], d["var"], d["md"], d["vd"], B, F, S, d["delta"])


def _fused(d):
    B, F, S = SHAPE
    gpu.batchnormBackward(B, F, S, Activation.leaky, d["y"], d["delta"], d["x"], d["xn"], d["mean"], d["var"],
                          d["scales"], d["bu"], d["su"], d["md"], d["vd"])


def _results(d, h):
    F = SHAPE[1]
    return {k: down(d[k], h["delta"] if k == "delta" else np.empty(F, np.float32))
            for k in ("delta", "bu", "su", "md", "vd")}


def _reset(d, h):
    gpu.push(d["delta"], h["delta"])
    for k in ("bu", "su"):
        gpu.push(d[k], np.zeros(SHAPE[1], np.float32))


def _free(d):
    for b in d.values():
        gpu.free(b)


@pytest.fixture
def quiet(dev):
    """Sync-after-launch off (a synchronise is not allowed inside a capture);
    the null stream again afterwards."""
    lib = _lib.load()
    before = lib.dkz_get_sync_after_launch()
    lib.dkz_set_sync_after_launch(0)
    yield lib
    lib.dkz_set_stream(None)
    lib.dkz_set_sync_after_launch(before)
    gpu.sync()


@pytest.mark.parametrize("op", [_chain, _fused], ids=["per-op chain", "fused"])
def test_on_a_caller_stream(quiet, op):
    hip = Hip()
    h = _inputs(1)
    d = _upload(h)
    op(d)
    want = _results(d, h)
    _reset(d, h)
    s = C.c_void_p()
    assert hip.hipStreamCreate(C.byref(s)) == 0
    try:
        assert quiet.dkz_set_stream(s) == 0
        assert quiet.dkz_get_stream() == s.value
        op(d)
        got = _results(d, h)  # dkz_copy_to_host orders itself after the stream's work
        quiet.dkz_set_stream(None)
    finally:
        quiet.dkz_set_stream(None)
        gpu.sync()
        hip.hipStreamDestroy(s)
    for k in want:
        assert_bitexact(got[k], want[k], f"{op.__name__} {k} on a stream")
    _free(d)


@pytest.mark.parametrize("op", [_chain, _fused], ids=["per-op chain", "fused"])
def test_captured_graph_replays(quiet, op):
    hip = Hip()
    h = _inputs(2)
    d = _upload(h)
    op(d)
    want = _results(d, h)

    s, graph, exe = C.c_void_p(), C.c_void_p(), C.c_void_p()
    assert hip.hipStreamCreate(C.byref(s)) == 0
    try:
        quiet.dkz_set_stream(s)
        assert hip.hipStreamBeginCapture(s, 0) == 0  # hipStreamCaptureModeGlobal
        op(d)
        assert hip.hipStreamEndCapture(s, C.byref(graph)) == 0
        quiet.dkz_set_stream(None)
        assert hip.hipGraphInstantiate(C.byref(exe), graph, None, None, 0) == 0
        for replay in range(3):
            _reset(d, h)  # eager work between the replays
            gpu.scal(4, 1.0, d["scales"])
            gpu.sync()
            assert hip.hipGraphLaunch(exe, s) == 0
            assert hip.hipStreamSynchronize(s) == 0
            got = _results(d, h)
            for k in want:
                assert_bitexact(got[k], want[k], f"{op.__name__} {k} replay {replay}")
    finally:
        quiet.dkz_set_stream(None)
        gpu.sync()
        if exe.value:
            hip.hipGraphExecDestroy(exe)
        if graph.value:
            hip.hipGraphDestroy(graph)
        hip.hipStreamDestroy(s)
    _free(d)
